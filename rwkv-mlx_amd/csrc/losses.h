// Router loss partials -> (aux, z), shared by router_finalize_kernel and the
// key GEMM (which runs the reduction in whichever workgroup finishes first,
// so the forward needs no launch of its own for it).
#pragma once

#include "common.h"

namespace rwkvmoe {

constexpr int kLossMaxE = 64;

// Partials of router block b: part[v * nb + b] (fp64; v < E: Σ_t P[t,v],
// v = E: Σ_t lse_t²) and cnt[e * nb + b] (int32: assignments to e).
struct LossJob {
  const double* part;
  const int* cnt;
  int nb, N, E, k;
  float* losses;  // (aux, z); nullptr: no job
  int* claim;     // zeroed by the router pass; the first workgroup to take it runs the job
};

// Fixed-order reduction by all blockDim.x threads of one workgroup: each of
// the E+1 fp64 sums is split over tpv threads taking blocks j, j+tpv, ... in
// ascending order (consecutive threads read consecutive blocks), then the tpv
// partials are added by a fixed-shape tree.  aux = E · Σ_e f_e·p_e with
// f_e = count_e/(N·k), p_e = Σ_t P[t,e]/N (moe.py:76-84); z = Σ_t lse_t²/N
// (moe.py:62).  Scratch: sp, sc of blockDim.x entries, fe of E+1.
RWKV_DEV void reduce_losses(const LossJob& jb, double* sp, long long* sc, double* fe) {
  const int tid = threadIdx.x, E = jb.E, nb = jb.nb;
  const int nv = E + 1;
  int tpv = (int)blockDim.x / nv;  // threads per value, rounded down to a power of two
  while (tpv & (tpv - 1)) tpv &= tpv - 1;
  const int v = tid / tpv, j = tid % tpv;
  double s = 0.0;
  long long c = 0;
  if (v < nv) {
    const double* pp = jb.part + (size_t)v * nb;
    const int* pc = jb.cnt + (size_t)(v < E ? v : 0) * nb;
    constexpr int BATCH = 16;  // loads in flight per round
    for (int b0 = j; b0 < nb; b0 += BATCH * tpv) {
      double pv[BATCH];
      int cv[BATCH];
#pragma unroll
      for (int i = 0; i < BATCH; ++i) {
        const int b = min(b0 + i * tpv, nb - 1);
        pv[i] = pp[b];
        cv[i] = pc[b];
      }
#pragma unroll
      for (int i = 0; i < BATCH; ++i)
        if (b0 + i * tpv < nb) {
          s += pv[i];
          if (v < E) c += cv[i];
        }
    }
  }
  sp[tid] = s;
  sc[tid] = c;
  __syncthreads();
  for (int h = tpv / 2; h >= 1; h >>= 1) {
    if (v < nv && j < h) {
      sp[tid] += sp[tid + h];
      sc[tid] += sc[tid + h];
    }
    __syncthreads();
  }
  if (tid < nv) {
    const double ps = sp[tid * tpv];
    const long long cnt = sc[tid * tpv];
    fe[tid] = tid < E ? ((double)cnt / ((double)jb.N * jb.k)) * (ps / jb.N) : ps / jb.N;
  }
  __syncthreads();
  if (tid == 0) {
    double a = 0.0;
    for (int e = 0; e < E; ++e) a += fe[e];
    jb.losses[0] = (float)(E * a);
    jb.losses[1] = (float)fe[E];
  }
}

// LDS bytes reduce_losses needs for nt threads.
constexpr int loss_scratch_bytes(int nt) { return nt * 16 + (kLossMaxE + 1) * 8; }

}  // namespace rwkvmoe
