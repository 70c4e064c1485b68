// Router: logits, top-k, gates and the load-balance / z-loss partial sums
// (rwkv_mlx/moe.py:51-86).
//
// Logit definition (exact, implementation independent):
//   acc_q = Σ_{c in chunk q, ascending} x[t,c]·W_gate[e,c]     in fp64, q = c / 64
//   logit = fp32(Σ_{q ascending} acc_q) (+ logit_bias[e] in fp32)
// Every product of two fp32/fp16/bf16 numbers is exact in fp64, so each step is
// a single IEEE rounding and the oracle reproduces the bits.  The reference
// computes the same dot product in fp32 inside MLX (moe.py:56); this form sits
// within a few fp32 ulp of it and removes summation order from top-k.
//
// Workgroup = 256 threads over TT tokens.  Phase 1 spreads the TT·E·(C/64)
// chunk dot products over the threads (x and W_gate read with 16-byte loads,
// L1/L2 serving the E-fold reuse of each x chunk); phase 2 sums chunks;
// phase 3 runs one thread per token for top-k, gates, log-sum-exp and the
// softmax; phase 4 writes per-workgroup partial sums that a single-workgroup
// finalize kernel reduces in a fixed order.
#include "common.h"
#include "internal.h"

namespace rwkvmoe {
namespace {

constexpr int kRouterThreads = 256;
constexpr int kMaxE = 64;
constexpr int kMaxK = 8;

template <typename T>
__global__ __launch_bounds__(kRouterThreads) void router_kernel(const T* __restrict__ x, const T* __restrict__ wg,
                                                                const float* __restrict__ bias, int N, int C, int E,
                                                                int k, int TT, float* logits, int* inds, T* gates,
                                                                T* gate_dense, double* part_f64, int* part_cnt) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int VEC = 16 / sizeof(T);
  const int Q = C / 64;
  double* part = (double*)smem;                       // TT*E*Q
  float* lg = (float*)(part + (size_t)TT * E * Q);    // TT*E
  float* prob = lg + TT * E;                          // TT*E
  float* zt = prob + TT * E;                          // TT
  int* sel = (int*)(zt + TT);                         // TT*kMaxK

  const int tid = threadIdx.x;
  const int t0 = blockIdx.x * TT;

  // Phase 1: chunk dot products in fp64.
  const int ntask = TT * E * Q;
  for (int task = tid; task < ntask; task += kRouterThreads) {
    const int q = task % Q, e = (task / Q) % E, tl = task / (Q * E);
    const int t = t0 + tl;
    double acc = 0.0;
    if (t < N) {
      const T* xr = x + (size_t)t * C + q * 64;
      const T* wr = wg + (size_t)e * C + q * 64;
#pragma unroll 2
      for (int j = 0; j < 64; j += VEC) {
        Chunk<T> xc, wc;
        xc.raw = *(const u32x4*)(xr + j);
        wc.raw = *(const u32x4*)(wr + j);
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc = __builtin_fma((double)to_f(xc.e[i]), (double)to_f(wc.e[i]), acc);
      }
    }
    part[task] = acc;
  }
  __syncthreads();

  // Phase 2: sum the chunks in ascending order, round once to fp32.
  for (int pr = tid; pr < TT * E; pr += kRouterThreads) {
    const int e = pr % E, tl = pr / E;
    double s = 0.0;
    for (int q = 0; q < Q; ++q) s += part[(size_t)pr * Q + q];
    float l = (float)s;
    if (bias) l = l + bias[e];
    lg[pr] = l;
    if (logits && t0 + tl < N) logits[(size_t)(t0 + tl) * E + e] = l;
  }
  __syncthreads();

  // Phase 3: one thread per token.
  if (tid < TT) {
    const int t = t0 + tid;
    const float* l = lg + tid * E;
    if (t < N) {
      // top-k: k passes of argmax; strict '>' keeps the lower id on ties
      unsigned long long taken = 0ull;
      int s_e[kMaxK];
      for (int s = 0; s < k; ++s) {
        int be = -1;
        float bv = 0.f;
        for (int e = 0; e < E; ++e) {
          if ((taken >> e) & 1ull) continue;
          if (be < 0 || l[e] > bv) { be = e; bv = l[e]; }
        }
        taken |= 1ull << be;
        s_e[s] = be;
        sel[tid * kMaxK + s] = be;
      }
      // gates: softmax over the selected logits (moe.py:69-70), cast to T (moe.py:86)
      const float m = l[s_e[0]];
      float ex[kMaxK], den = 0.f;
      for (int s = 0; s < k; ++s) { ex[s] = expf(l[s_e[s]] - m); den += ex[s]; }
      float g[kMaxK];
      for (int s = 0; s < k; ++s) {
        g[s] = ex[s] / den;
        if (inds) inds[(size_t)t * k + s] = s_e[s];
        if (gates) gates[(size_t)t * k + s] = from_f<T>(g[s]);
      }
      if (gate_dense) {
        for (int e = 0; e < E; ++e) {
          float v = 0.f;
          for (int s = 0; s < k; ++s) if (s_e[s] == e) v = g[s];
          gate_dense[(size_t)t * E + e] = from_f<T>(v);
        }
      }
      // z-loss term: (log Σ_e exp ℓ_e)², no max shift (moe.py:61-62)
      float se = 0.f;
      for (int e = 0; e < E; ++e) se += expf(l[e]);
      const float lse = logf(se);
      zt[tid] = lse * lse;
      // full softmax for p_e (moe.py:76)
      float mx = l[0];
      for (int e = 1; e < E; ++e) mx = fmaxf(mx, l[e]);
      float sp = 0.f;
      for (int e = 0; e < E; ++e) sp += expf(l[e] - mx);
      for (int e = 0; e < E; ++e) prob[tid * E + e] = expf(l[e] - mx) / sp;
    } else {
      zt[tid] = 0.f;
      for (int e = 0; e < E; ++e) prob[tid * E + e] = 0.f;
      for (int s = 0; s < k; ++s) sel[tid * kMaxK + s] = -1;
    }
  }
  __syncthreads();

  // Phase 4: per-workgroup partials, tokens in ascending order.
  if (tid < E) {
    double ps = 0.0;
    int cnt = 0;
    for (int tl = 0; tl < TT; ++tl) {
      ps += (double)prob[tl * E + tid];
      for (int s = 0; s < k; ++s) cnt += sel[tl * kMaxK + s] == tid;
    }
    part_f64[(size_t)blockIdx.x * (E + 1) + tid] = ps;
    part_cnt[(size_t)blockIdx.x * E + tid] = cnt;
  } else if (tid == E) {
    double zs = 0.0;
    for (int tl = 0; tl < TT; ++tl) zs += (double)zt[tl];
    part_f64[(size_t)blockIdx.x * (E + 1) + E] = zs;
  }
}

// aux = E · Σ_e f_e·p_e with f_e = count_e/(N·k), p_e = Σ_t P[t,e]/N (moe.py:76-84);
// z = Σ_t lse_t² / N (moe.py:62).  Workgroup sums run in ascending block order.
__global__ __launch_bounds__(64) void router_finalize_kernel(const double* part_f64, const int* part_cnt, int nb,
                                                             int N, int E, int k, float* losses) {
  __shared__ double fp[kMaxE];
  const int tid = threadIdx.x;
  if (tid < E) {
    double ps = 0.0;
    long long cnt = 0;
    for (int b = 0; b < nb; ++b) {
      ps += part_f64[(size_t)b * (E + 1) + tid];
      cnt += part_cnt[(size_t)b * E + tid];
    }
    fp[tid] = ((double)cnt / ((double)N * k)) * (ps / N);
  }
  __syncthreads();
  if (tid == 0) {
    double zs = 0.0;
    for (int b = 0; b < nb; ++b) zs += part_f64[(size_t)b * (E + 1) + E];
    double a = 0.0;
    for (int e = 0; e < E; ++e) a += fp[e];
    losses[0] = (float)(E * a);
    losses[1] = (float)(zs / N);
  }
}

size_t router_smem(int TT, int C, int E) {
  return (size_t)TT * E * (C / 64) * sizeof(double) + (size_t)TT * E * 2 * sizeof(float) + TT * sizeof(float) +
         (size_t)TT * kMaxK * sizeof(int);
}

}  // namespace

int router_tile_tokens(int C, int E) {
  const int per_token = E * (C / 64);
  int tt = 4096 / (per_token > 0 ? per_token : 1);
  if (tt > 16) tt = 16;
  if (tt < 1) tt = 1;
  return tt;
}

hipError_t launch_router(int dtype, const void* x, const void* wg, const float* bias, int N, int C, int E, int k,
                         float* logits, int* inds, void* gates, void* gate_dense, double* part_f64, int* part_cnt,
                         hipStream_t s) {
  const int TT = router_tile_tokens(C, E);
  const int nb = (N + TT - 1) / TT;
  const size_t smem = router_smem(TT, C, E);
  RWKV_DISPATCH_DTYPE(dtype, T, {
    if (smem > 65536) {
      hipError_t err = hipFuncSetAttribute((const void*)router_kernel<T>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
      if (err != hipSuccess) return err;
    }
    hipLaunchKernelGGL(router_kernel<T>, dim3(nb), dim3(kRouterThreads), smem, s, (const T*)x, (const T*)wg, bias,
                       N, C, E, k, TT, logits, inds, (T*)gates, (T*)gate_dense, part_f64, part_cnt);
  });
  return hipGetLastError();
}

hipError_t launch_router_finalize(const double* part_f64, const int* part_cnt, int nb, int N, int E, int k,
                                  float* losses, hipStream_t s) {
  hipLaunchKernelGGL(router_finalize_kernel, dim3(1), dim3(64), 0, s, part_f64, part_cnt, nb, N, E, k, losses);
  return hipGetLastError();
}

}  // namespace rwkvmoe
