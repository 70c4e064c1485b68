// Router: logits, top-k, gates and the load-balance / z-loss partial sums
// (rwkv_mlx/moe.py:51-86), and — fused into the same pass over x — the
// token-shift mix xk of the base ChannelMix (model.py:67-75, 260-261).
//
// Logit definition (exact, implementation independent):
//   acc_q = Σ_{c in chunk q, ascending} x[t,c]·W_gate[e,c]     in fp64, q = c / 64
//   logit = fp32(Σ_{q ascending} acc_q) (+ logit_bias[e] in fp32)
// Every product of two fp32/fp16/bf16 numbers is exact in fp64, so each step is
// a single IEEE rounding and the oracle reproduces the bits.  The reference
// computes the same dot product in fp32 inside MLX (moe.py:56); this form sits
// within a few fp32 ulp of it and removes summation order from top-k.
//
// Workgroup = 256 threads over TT (<= 16) tokens:
//   1. the TT x C tile of x is staged in LDS once (16-byte loads);
//      1b. optional: xk = x + (shift(x) - x) * x_k for the tile's rows;
//   2. the TT·E·(C/64) chunk dot products are spread over the threads, fp64;
//   3. chunks are summed per (token, expert) and rounded to fp32;
//   4. one thread per token: top-k (descending logit, ties to the lower id),
//      gates (softmax over the selected logits, cast to T), lse² and softmax;
//   5. per-workgroup partial sums (tokens in ascending order) that a
//      single-workgroup finalize kernel reduces in a fixed order.
#include "common.h"
#include "internal.h"

namespace rwkvmoe {
namespace {

constexpr int kRouterThreads = 256;
constexpr int kMaxE = 64;
constexpr int kMaxK = 8;

struct RouterShape {
  int TT, Q, xs_stride;  // tokens per workgroup, 64-chunks per row, LDS row stride (elements)
};

template <typename T>
RWKV_DEV RouterShape router_shape(int C, int TT) {
  return RouterShape{TT, C / 64, C + 16 / (int)sizeof(T)};
}

template <typename T>
__global__ __launch_bounds__(kRouterThreads) void router_kernel(
    const T* __restrict__ x, const T* __restrict__ wg, const float* __restrict__ bias, const T* __restrict__ xprev,
    const T* __restrict__ mu, int N, int T_, int C, int E, int k, int TT, float* logits, int* inds, T* gates,
    T* gate_dense, T* xk, double* part_f64, int* part_cnt) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int VEC = 16 / sizeof(T);
  const RouterShape sh = router_shape<T>(C, TT);
  const int Q = sh.Q, XS = sh.xs_stride;
  double* part = (double*)smem;                               // TT*E*Q (region padded to 16 bytes)
  T* xs = (T*)(smem + ((size_t)TT * E * Q * sizeof(double) + 15) / 16 * 16);  // TT*XS; XS*sizeof(T) % 16 == 0
  float* lg = (float*)(xs + (size_t)TT * XS);                 // TT*E logits
  float* gd = lg + TT * E;                                    // TT*E dense gates (0 where not routed)
  float* prob = gd + TT * E;                                  // TT*E softmax
  float* zt = prob + TT * E;                                  // TT
  int* sel = (int*)(zt + TT);                                 // TT*kMaxK

  const int tid = threadIdx.x;
  const int t0 = blockIdx.x * TT;
  const int nt = min(TT, N - t0);

  // 1. x tile -> LDS
  const int cpr = C / VEC;
  for (int i = tid; i < TT * cpr; i += kRouterThreads) {
    const int tl = i / cpr, c = (i % cpr) * VEC;
    u32x4 v = tl < nt ? *(const u32x4*)(x + (size_t)(t0 + tl) * C + c) : zero4();
    *(u32x4*)(xs + (size_t)tl * XS + c) = v;
  }
  __syncthreads();

  // 1b. optional: the token-shift mix of the base ChannelMix for these rows,
  //     xk = x + (shift(x) - x) * x_k, each op rounded to T (model.py:260-261)
  if (xk) {
    for (int i = tid; i < nt * cpr; i += kRouterThreads) {
      const int tl = i / cpr, c = (i % cpr) * VEC;
      const int t = t0 + tl;
      Chunk<T> xc, pc, mc, o;
      xc.raw = *(const u32x4*)(xs + (size_t)tl * XS + c);
      if (t % T_ != 0)
        pc.raw = tl > 0 ? *(const u32x4*)(xs + (size_t)(tl - 1) * XS + c) : *(const u32x4*)(x + (size_t)(t - 1) * C + c);
      else
        pc.raw = xprev ? *(const u32x4*)(xprev + (size_t)(t / T_) * C + c) : zero4();
      mc.raw = *(const u32x4*)(mu + c);
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float xf = to_f(xc.e[j]);
        const float xx = rnd<T>(to_f(pc.e[j]) - xf);
        o.e[j] = from_f<T>(xf + rnd<T>(xx * to_f(mc.e[j])));
      }
      *(u32x4*)(xk + (size_t)t * C + c) = o.raw;
    }
  }

  // 2. chunk dot products in fp64 (x from LDS, W_gate from L1/L2)
  const int ntask = TT * E * Q;
  for (int task = tid; task < ntask; task += kRouterThreads) {
    const int q = task % Q, e = (task / Q) % E, tl = task / (Q * E);
    const T* xr = xs + (size_t)tl * XS + q * 64;
    const T* wr = wg + (size_t)e * C + q * 64;
    double acc = 0.0;
    for (int j = 0; j < 64; j += VEC) {
      Chunk<T> xc, wc;
      xc.raw = *(const u32x4*)(xr + j);
      wc.raw = *(const u32x4*)(wr + j);
#pragma unroll
      for (int i = 0; i < VEC; ++i) acc = __builtin_fma((double)to_f(xc.e[i]), (double)to_f(wc.e[i]), acc);
    }
    part[task] = acc;
  }
  __syncthreads();

  // 3. chunk sums in ascending order, one rounding to fp32
  for (int pr = tid; pr < TT * E; pr += kRouterThreads) {
    const int e = pr % E, tl = pr / E;
    double s = 0.0;
    for (int q = 0; q < Q; ++q) s += part[(size_t)pr * Q + q];
    float l = (float)s;
    if (bias) l = l + bias[e];
    lg[pr] = l;
    if (logits && tl < nt) logits[(size_t)(t0 + tl) * E + e] = l;
  }
  __syncthreads();

  // 4. one thread per token
  if (tid < TT) {
    const int t = t0 + tid;
    const float* l = lg + tid * E;
    float* gr = gd + tid * E;
    for (int e = 0; e < E; ++e) gr[e] = 0.f;
    if (tid < nt) {
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
      const float m = l[s_e[0]];
      float ex[kMaxK], den = 0.f;
      for (int s = 0; s < k; ++s) { ex[s] = expf(l[s_e[s]] - m); den += ex[s]; }
      for (int s = 0; s < k; ++s) {
        const T g = from_f<T>(ex[s] / den);
        gr[s_e[s]] = to_f(g);
        if (inds) inds[(size_t)t * k + s] = s_e[s];
        if (gates) gates[(size_t)t * k + s] = g;
      }
      if (gate_dense)
        for (int e = 0; e < E; ++e) gate_dense[(size_t)t * E + e] = from_f<T>(gr[e]);
      float se = 0.f;
      for (int e = 0; e < E; ++e) se += expf(l[e]);
      const float lse = logf(se);
      zt[tid] = lse * lse;
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

  // 5. per-workgroup partials, tokens in ascending order
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
// z = Σ_t lse_t² / N (moe.py:62).  One workgroup: each of the E+1 sums is
// split over `tpv` threads taking blocks j, j+tpv, ... in ascending order;
// the tpv partials are then added in ascending j.  The order is fixed, so the
// result is reproducible.
constexpr int kFinThreads = 1024;

__global__ __launch_bounds__(kFinThreads) void router_finalize_kernel(const double* __restrict__ part_f64,
                                                                      const int* __restrict__ part_cnt, int nb,
                                                                      int N, int E, int k, float* losses) {
  __shared__ double sp[kFinThreads];
  __shared__ long long sc[kFinThreads];
  __shared__ double fe[kMaxE + 1];
  const int tid = threadIdx.x;
  const int nv = E + 1;
  const int tpv = kFinThreads / nv;
  if (tid < tpv * nv) {
    const int v = tid / tpv, j = tid % tpv;
    double s = 0.0;
    long long c = 0;
    for (int b = j; b < nb; b += tpv) {
      s += part_f64[(size_t)b * nv + v];
      if (v < E) c += part_cnt[(size_t)b * E + v];
    }
    sp[tid] = s;
    sc[tid] = c;
  }
  __syncthreads();
  if (tid < nv) {
    double s = 0.0;
    long long c = 0;
    for (int j = 0; j < tpv; ++j) {
      s += sp[tid * tpv + j];
      c += sc[tid * tpv + j];
    }
    fe[tid] = tid < E ? ((double)c / ((double)N * k)) * (s / N) : s / N;
  }
  __syncthreads();
  if (tid == 0) {
    double a = 0.0;
    for (int e = 0; e < E; ++e) a += fe[e];
    losses[0] = (float)(E * a);
    losses[1] = (float)fe[E];
  }
}

template <typename T>
size_t router_smem(int TT, int C, int E) {
  const size_t xs = (size_t)TT * (C + 16 / sizeof(T)) * sizeof(T);
  return ((size_t)TT * E * (C / 64) * sizeof(double) + 15) / 16 * 16 + xs + (size_t)TT * E * 3 * sizeof(float) +
         TT * sizeof(float) + (size_t)TT * kMaxK * sizeof(int);
}

}  // namespace

int router_tile_tokens(int C, int E) {
  const int per_token = E * (C / 64);
  int tt = 4096 / (per_token > 0 ? per_token : 1);
  if (tt > 16) tt = 16;
  if (tt < 1) tt = 1;
  return tt;
}

hipError_t launch_router(int dtype, const void* x, const void* wg, const float* bias, const void* xprev,
                         const void* mu, int N, int T_, int C, int E, int k, float* logits, int* inds, void* gates,
                         void* gate_dense, void* xk, double* part_f64, int* part_cnt, hipStream_t s) {
  const int TT = router_tile_tokens(C, E);
  const int nb = (N + TT - 1) / TT;
  RWKV_DISPATCH_DTYPE(dtype, T, {
    const size_t smem = router_smem<T>(TT, C, E);
    if (smem > 65536) {
      hipError_t err = hipFuncSetAttribute((const void*)router_kernel<T>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
      if (err != hipSuccess) return err;
    }
    hipLaunchKernelGGL(router_kernel<T>, dim3(nb), dim3(kRouterThreads), smem, s, (const T*)x, (const T*)wg, bias,
                       (const T*)xprev, (const T*)mu, N, T_, C, E, k, TT, logits, inds, (T*)gates, (T*)gate_dense,
                       (T*)xk, part_f64, part_cnt);
  });
  return hipGetLastError();
}

hipError_t launch_router_finalize(const double* part_f64, const int* part_cnt, int nb, int N, int E, int k,
                                  float* losses, hipStream_t s) {
  hipLaunchKernelGGL(router_finalize_kernel, dim3(1), dim3(kFinThreads), 0, s, part_f64, part_cnt, nb, N, E, k,
                     losses);
  return hipGetLastError();
}

}  // namespace rwkvmoe
