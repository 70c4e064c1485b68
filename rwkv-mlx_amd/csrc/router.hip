// Router: logits, top-k, gates and the load-balance / z-loss partial sums
// (rwkv_mlx/moe.py:51-86), and — fused into the same pass over x — the
// token-shift mix xk of the base ChannelMix (model.py:67-75, 260-261) and,
// for adapter widths E*r <= 128, the gate-masked adapter down-projection
// U = w ⊙ (x · A_all) of the FUSED mode (moe.py:140-144).
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
//   1. the TT x C tile of x and all of W_gate (E x C) are staged in LDS
//      (16-byte loads);
//      1b. optional: xk = x + (shift(x) - x) * x_k for the tile's rows;
//   2. the TT·E·(C/64) chunk dot products are spread over the threads, fp64;
//   3. chunks are summed per (token, expert) and rounded to fp32;
//   4. one thread per token: top-k (descending logit, ties to the lower id),
//      gates (softmax over the selected logits, cast to T), lse² and softmax;
//   5. optional: U[t, e*r+j] = w_e[t] · round_T((x·A_e)[t, j]) with
//      v_mfma_f32_16x16x32 (16 token rows x 16 adapter columns per block,
//      two blocks per wave for the 128 columns); each wave issues the A_all
//      fragments of 12 K-steps for both blocks before its MFMAs, so one L2
//      round trip covers 384 K values;
//   6. per-workgroup partial sums (tokens in ascending order) that a
//      single-workgroup finalize kernel reduces in a fixed order.
#include "common.h"
#include "internal.h"

namespace rwkvmoe {
namespace {

constexpr int kRouterThreads = 256;
constexpr int kMaxE = 64;
constexpr int kMaxK = 8;

// Widths of A_all (rows) the router's fused down-projection handles.
constexpr int kRouterKx = 128;

struct RouterShape {
  int TT, Q, xs_stride;  // tokens per workgroup, 64-chunks per row, LDS row stride (elements)
};

template <typename T>
RWKV_DEV RouterShape router_shape(int C, int TT) {
  return RouterShape{TT, C / 64, C + 16 / (int)sizeof(T)};
}

template <typename T, int EB>
__global__ __launch_bounds__(kRouterThreads) void router_kernel(
    const T* __restrict__ x, const T* __restrict__ wg, const float* __restrict__ bias, const T* __restrict__ xprev,
    const T* __restrict__ mu, const T* __restrict__ at, int N, int T_, int C, int E, int k, int r, int TT,
    float* logits, int* inds, T* gates, T* gate_dense, T* xk, T* u, double* part_f64, int* part_cnt) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int VEC = 16 / sizeof(T);
  const RouterShape sh = router_shape<T>(C, TT);
  const int Q = sh.Q, XS = sh.xs_stride;
  double* part = (double*)smem;                               // TT*E*Q (region padded to 16 bytes)
  T* xs = (T*)(smem + ((size_t)TT * E * Q * sizeof(double) + 15) / 16 * 16);  // TT*XS; XS*sizeof(T) % 16 == 0
  T* ws_ = xs + (size_t)TT * XS;                              // E*XS W_gate
  float* lg = (float*)(ws_ + (size_t)E * XS);                 // TT*E logits
  float* gd = lg + TT * E;                                    // TT*E dense gates (0 where not routed)
  float* prob = gd + TT * E;                                  // TT*E softmax
  float* zt = prob + TT * E;                                  // TT
  int* sel = (int*)(zt + TT);                                 // TT*kMaxK

  const int tid = threadIdx.x;
  const int t0 = blockIdx.x * TT;
  const int nt = min(TT, N - t0);

  // 0. adapter down-projection: put the A_all fragments of the first K chunk
  //    in flight now, so their latency overlaps phases 1-4
  typedef typename Mma16<T>::frag ufrag;
  constexpr int UCH = 12;  // K-steps whose A_all fragments are in flight together
  ufrag ufb[2][UCH];
  f32x4 uacc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  int un[2] = {0, 0};
  const T* ubcol[2] = {at, at};
  auto u_load = [&](int k0) {
    const int kh = (tid & 63) >> 4;
#pragma unroll
    for (int j = 0; j < UCH; ++j) {
      const int kk = min(k0 + j * Mma16<T>::KS, C - Mma16<T>::KS);  // clamped; steps past C are skipped
#pragma unroll
      for (int b = 0; b < 2; ++b) ufb[b][j] = *(const ufrag*)(ubcol[b] + kk + kh * Mma16<T>::KV);
    }
  };
  if (u) {
    const int wave = tid >> 6, lr = tid & 15;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      un[b] = (wave * 2 + b) * 16 + lr;  // this lane's adapter column in block b
      ubcol[b] = at + (size_t)un[b] * C;
    }
    u_load(0);
  }

  // 1. x tile -> LDS
  const int cpr = C / VEC;
  for (int i = tid; i < TT * cpr; i += kRouterThreads) {
    const int tl = i / cpr, c = (i % cpr) * VEC;
    u32x4 v = tl < nt ? *(const u32x4*)(x + (size_t)(t0 + tl) * C + c) : zero4();
    *(u32x4*)(xs + (size_t)tl * XS + c) = v;
  }
  for (int i = tid; i < E * cpr; i += kRouterThreads) {
    const int e = i / cpr, c = (i % cpr) * VEC;
    *(u32x4*)(ws_ + (size_t)e * XS + c) = *(const u32x4*)(wg + (size_t)e * C + c);
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

  // 2. chunk dot products in fp64 (x and W_gate from LDS).  A task is a 2x2
  //    (token, expert) micro-tile of one chunk: each accumulator still runs
  //    over its chunk in ascending c, and every conversion feeds two FMAs.
  {
    const int TT2 = (TT + 1) / 2, E2 = (E + 1) / 2;
    const int ntask = TT2 * E2 * Q;
    for (int task = tid; task < ntask; task += kRouterThreads) {
      const int q = task % Q, ep = (task / Q) % E2, tp = task / (Q * E2);
      const int ta = 2 * tp, tb = min(2 * tp + 1, TT - 1);
      const int ea = 2 * ep, eb = min(2 * ep + 1, E - 1);
      const T* xa = xs + (size_t)ta * XS + q * 64;
      const T* xb = xs + (size_t)tb * XS + q * 64;
      const T* wa = ws_ + (size_t)ea * XS + q * 64;
      const T* wb = ws_ + (size_t)eb * XS + q * 64;
      double aa = 0.0, ab = 0.0, ba = 0.0, bb = 0.0;
#pragma unroll
      for (int j = 0; j < 64; j += VEC) {
        Chunk<T> cxa, cxb, cwa, cwb;
        cxa.raw = *(const u32x4*)(xa + j);
        cxb.raw = *(const u32x4*)(xb + j);
        cwa.raw = *(const u32x4*)(wa + j);
        cwb.raw = *(const u32x4*)(wb + j);
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          const double fxa = (double)to_f(cxa.e[i]), fxb = (double)to_f(cxb.e[i]);
          const double fwa = (double)to_f(cwa.e[i]), fwb = (double)to_f(cwb.e[i]);
          aa = __builtin_fma(fxa, fwa, aa);
          ab = __builtin_fma(fxa, fwb, ab);
          ba = __builtin_fma(fxb, fwa, ba);
          bb = __builtin_fma(fxb, fwb, bb);
        }
      }
      // duplicate lanes (odd TT or E) write the same value to the same slot
      part[((size_t)ta * E + ea) * Q + q] = aa;
      part[((size_t)ta * E + eb) * Q + q] = ab;
      part[((size_t)tb * E + ea) * Q + q] = ba;
      part[((size_t)tb * E + eb) * Q + q] = bb;
    }
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

  // 4. one thread per token; its E logits (E <= EB) sit in registers, every
  //    loop is unrolled over EB with e < E masks: top-k in k passes (largest
  //    untaken logit, strict '>' keeps the lower id on ties), gates in slot
  //    order, log-sum-exp and softmax.
  if (tid < TT) {
    const int t = t0 + tid;
    float l[EB];
#pragma unroll
    for (int e = 0; e < EB; ++e) l[e] = e < E ? lg[tid * E + e] : 0.f;
#pragma unroll
    for (int s = 0; s < kMaxK; ++s) sel[tid * kMaxK + s] = -1;
    if (tid < nt) {
      unsigned long long taken = 0ull;
      int s_e[kMaxK];
      float s_l[kMaxK];
#pragma unroll
      for (int s = 0; s < kMaxK; ++s) {
        if (s >= k) break;
        int be = -1;
        float bv = 0.f;
#pragma unroll
        for (int e = 0; e < EB; ++e) {
          const bool cand = e < E && !((taken >> e) & 1ull);
          if (cand && (be < 0 || l[e] > bv)) { be = e; bv = l[e]; }
        }
        taken |= 1ull << be;
        s_e[s] = be;
        s_l[s] = bv;
        sel[tid * kMaxK + s] = be;
      }
      const float m = s_l[0];
      float ex[kMaxK], den = 0.f;
#pragma unroll
      for (int s = 0; s < kMaxK; ++s) {
        if (s >= k) break;
        ex[s] = expf(s_l[s] - m);
        den += ex[s];
      }
      float gsel[EB];
#pragma unroll
      for (int e = 0; e < EB; ++e) gsel[e] = 0.f;
#pragma unroll
      for (int s = 0; s < kMaxK; ++s) {
        if (s >= k) break;
        const T g = from_f<T>(ex[s] / den);
        if (inds) inds[(size_t)t * k + s] = s_e[s];
        if (gates) gates[(size_t)t * k + s] = g;
#pragma unroll
        for (int e = 0; e < EB; ++e)
          if (e == s_e[s]) gsel[e] = to_f(g);
      }
      float se = 0.f, mx = l[0];
#pragma unroll
      for (int e = 0; e < EB; ++e)
        if (e < E) {
          se += expf(l[e]);
          mx = fmaxf(mx, l[e]);
        }
      const float lse = logf(se);
      zt[tid] = lse * lse;
      float pe[EB], sp = 0.f;
#pragma unroll
      for (int e = 0; e < EB; ++e) {
        pe[e] = e < E ? expf(l[e] - mx) : 0.f;
        sp += pe[e];
      }
#pragma unroll
      for (int e = 0; e < EB; ++e)
        if (e < E) {
          prob[tid * E + e] = pe[e] / sp;
          gd[tid * E + e] = gsel[e];
          if (gate_dense) gate_dense[(size_t)t * E + e] = from_f<T>(gsel[e]);
        }
    } else {
      zt[tid] = 0.f;
#pragma unroll
      for (int e = 0; e < EB; ++e)
        if (e < E) { prob[tid * E + e] = 0.f; gd[tid * E + e] = 0.f; }
    }
  }
  __syncthreads();

  // 5. fused adapter down-projection: finish the MFMAs on the prefetched
  //    chunk, then stream the remaining chunks
  if (u) {
    using M = Mma16<T>;
    const int lane = tid & 63;
    const int lr = lane & 15, kh = lane >> 4;
    const bool row_ok = lr < nt;
    const T* arow = xs + (size_t)(row_ok ? lr : 0) * XS;
    for (int k0 = 0; k0 < C; k0 += UCH * M::KS) {
      if (k0 > 0) u_load(k0);
#pragma unroll
      for (int j = 0; j < UCH; ++j) {
        const int kk = k0 + j * M::KS;
        if (kk < C) {
          const ufrag fa = row_ok ? *(const ufrag*)(arow + kk + kh * M::KV) : ufrag{};
#pragma unroll
          for (int b = 0; b < 2; ++b) uacc[b] = M::run(fa, ufb[b][j], uacc[b]);
        }
      }
    }
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int e = un[b] / r;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = kh * 4 + v;  // token within the tile
        if (row < nt) {
          const float g = (un[b] < E * r) ? gd[row * E + e] : 0.f;
          u[(size_t)(t0 + row) * kRouterKx + un[b]] = from_f<T>(g * rnd<T>(uacc[b][v]));
        }
      }
    }
  }

  // 6. per-workgroup partials, tokens in ascending order
  if (tid < E) {
    double ps = 0.0;
    int cnt = 0;
#pragma unroll
    for (int tl = 0; tl < 16; ++tl) {
      if (tl < TT) {
        ps += (double)prob[tl * E + tid];
#pragma unroll
        for (int s = 0; s < kMaxK; ++s) cnt += sel[tl * kMaxK + s] == tid;
      }
    }
    part_f64[(size_t)blockIdx.x * (E + 1) + tid] = ps;
    part_cnt[(size_t)blockIdx.x * E + tid] = cnt;
  } else if (tid == E) {
    double zs = 0.0;
#pragma unroll
    for (int tl = 0; tl < 16; ++tl)
      if (tl < TT) zs += (double)zt[tl];
    part_f64[(size_t)blockIdx.x * (E + 1) + E] = zs;
  }
}

// aux = E · Σ_e f_e·p_e with f_e = count_e/(N·k), p_e = Σ_t P[t,e]/N (moe.py:76-84);
// z = Σ_t lse_t² / N (moe.py:62).  One workgroup: each of the E+1 sums is
// split over `tpv` threads taking blocks j, j+tpv, ... in ascending order,
// then the tpv partials are added by a fixed-shape tree, so the result is
// reproducible run to run.
constexpr int kFinThreads = 1024;

__global__ __launch_bounds__(kFinThreads) void router_finalize_kernel(const double* __restrict__ part_f64,
                                                                      const int* __restrict__ part_cnt, int nb,
                                                                      int N, int E, int k, float* losses) {
  __shared__ double sp[kFinThreads];
  __shared__ long long sc[kFinThreads];
  __shared__ double fe[kMaxE + 1];
  const int tid = threadIdx.x;
  const int nv = E + 1;
  int tpv = kFinThreads / nv;              // threads per value, rounded down to a power of two
  while (tpv & (tpv - 1)) tpv &= tpv - 1;
  const int v = tid / tpv, j = tid % tpv;
  double s = 0.0;
  long long c = 0;
  if (v < nv) {
    for (int b = j; b < nb; b += tpv) {
      s += part_f64[(size_t)b * nv + v];
      if (v < E) c += part_cnt[(size_t)b * E + v];
    }
  }
  sp[tid] = s;
  sc[tid] = c;
  __syncthreads();
  // fixed-shape tree over the tpv partials of each value
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
    fe[tid] = tid < E ? ((double)cnt / ((double)N * k)) * (ps / N) : ps / N;
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
  const size_t xs = (size_t)(TT + E) * (C + 16 / sizeof(T)) * sizeof(T);
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
                         const void* mu, const void* at, int N, int T_, int C, int E, int k, int r, float* logits,
                         int* inds, void* gates, void* gate_dense, void* xk, void* u, double* part_f64, int* part_cnt,
                         hipStream_t s) {
  const int TT = router_tile_tokens(C, E);
  const int nb = (N + TT - 1) / TT;
  if (u && (TT > 16 || E * r > kRouterKx)) return hipErrorInvalidValue;
  RWKV_DISPATCH_DTYPE(dtype, T, {
    const size_t smem = router_smem<T>(TT, C, E);
    auto launch = [&](auto kern) -> hipError_t {
      if (smem > 65536) {
        hipError_t err = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (err != hipSuccess) return err;
      }
      hipLaunchKernelGGL(kern, dim3(nb), dim3(kRouterThreads), smem, s, (const T*)x, (const T*)wg, bias,
                         (const T*)xprev, (const T*)mu, (const T*)at, N, T_, C, E, k, r, TT, logits, inds, (T*)gates,
                         (T*)gate_dense, (T*)xk, (T*)u, part_f64, part_cnt);
      return mark(hipGetLastError(), "router", s);
    };
    if (E <= 8) return launch(router_kernel<T, 8>);
    if (E <= 16) return launch(router_kernel<T, 16>);
    if (E <= 32) return launch(router_kernel<T, 32>);
    return launch(router_kernel<T, 64>);
  });
  return hipGetLastError();
}

bool router_fuses_adapters(int C, int E, int r) { return E * r <= kRouterKx && router_tile_tokens(C, E) == 16; }

hipError_t launch_router_finalize(const double* part_f64, const int* part_cnt, int nb, int N, int E, int k,
                                  float* losses, hipStream_t s) {
  hipLaunchKernelGGL(router_finalize_kernel, dim3(1), dim3(kFinThreads), 0, s, part_f64, part_cnt, nb, N, E, k,
                     losses);
  return mark(hipGetLastError(), "router_finalize", s);
}

}  // namespace rwkvmoe
