// Backward (VJP) of the full-expert MoE ChannelMix (rwkv_mlx/moe.py:218-234,
// MoE_CMix; every parameter trainable: no stop_gradient in that layer).
// Routed rows are taken in the forward's expert-major order (dispatch.hip):
// row j = assignment perm[j] = t·k + slot, expert e = inds[perm[j]].
//
//   xk_j  = x[t] + (shift(x)[t] − x[t])·x_k[e]           (experts_mix_kernel)
//   p_j   = xk_j · W_key,eᵀ  rounded (grouped GEMM, no epilogue)
//   u_j   = dO[t] · W_val,e   (grouped GEMM over W_val,eᵀ)
//   dw_j  = <relu(p_j)², u_j>                             gate cotangent of the slot
//   dp_j  = g_j · u_j ⊙ 2·relu(p_j)                       (exb_hidden_kernel)
//   dk_j  = dp_j · W_key,e    (grouped GEMM over W_key,eᵀ)
//   dx[t] += dk_j ⊙ (1 − x_k[e]);  dx[t−1] (or d x_prev) += dk_j ⊙ x_k[e]
//   dx_k[e] = Σ_j dk_j ⊙ (shift(x)[t] − x[t])
//   dW_key,e = Σ_j dp_jᵀ xk_j ;  dW_val,e = Σ_j (g_j dO[t])ᵀ relu(p_j)²
//   router: dℓ from the slot cotangents and the loss cotangents, dW_gate = dℓᵀ x, dx += dℓ W_gate
//
// The weight gradients contract over each expert's routed rows.  Their
// products run on the NT GEMM with both operands transposed into token
// segments of a fixed, host-known length Np = round_up(N, 128) per expert
// (an expert serves each token at most once): segment e holds expert e's
// rows, zero past its count, so the host plans the GEMMs without reading the
// routing back.  Sums over tokens (dx_k, dW_gate) take fixed row chunks and
// add the chunks in ascending order: every result is independent of timing.
#include <algorithm>

#include "common.h"
#include "internal.h"

namespace rwkvmoe {
namespace {

// dO rows in perm order, and each row's gate: the softmax over its token's
// selected logits (moe.py:86), rounded to the element type as the forward's
// gates are.  Rows whose assignment id is out of range (never written by the
// dispatch of valid ids) get zeros.
template <typename T>
__global__ __launch_bounds__(256) void exb_gather_kernel(const T* __restrict__ dO, const int* __restrict__ perm,
                                                         const float* __restrict__ logits,
                                                         const int* __restrict__ inds, int nk, int C, int E, int k,
                                                         T* __restrict__ dog, float* __restrict__ gr) {
  constexpr int VEC = 16 / sizeof(T);
  const int cpr = C / VEC;
  const size_t id = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (id >= (size_t)nk * cpr) return;
  const int j = (int)(id / cpr), c = (int)(id % cpr) * VEC;
  const int a = perm[j];
  const bool ok = a >= 0 && a < nk;
  const int t = ok ? a / k : 0;
  *(u32x4*)(dog + (size_t)j * C + c) = ok ? *(const u32x4*)(dO + (size_t)t * C + c) : zero4();
  if (c == 0) {
    float g = 0.f;
    if (ok) {
      const float* lr = logits + (size_t)t * E;
      float m = -INFINITY;
      for (int q = 0; q < k; ++q) {
        const int e = inds[t * k + q];
        if (e >= 0 && e < E) m = fmaxf(m, lr[e]);
      }
      float den = 0.f, num = 0.f;
      for (int q = 0; q < k; ++q) {
        const int e = inds[t * k + q];
        if (e < 0 || e >= E) continue;
        const float ex = expf(lr[e] - m);
        den += ex;
        if (t * k + q == a) num = ex;
      }
      g = den > 0.f ? rnd<T>(num / den) : 0.f;
    }
    gr[j] = g;
  }
}

// One wave per routed row: dw_j = <relu(p)², u> (each lane adds its elements
// in ascending order, then a fixed butterfly), dp_j = round(g·u·2·relu(p)).
template <typename T>
__global__ __launch_bounds__(256) void exb_hidden_kernel(const T* __restrict__ P, const T* __restrict__ U,
                                                         const float* __restrict__ gr, int nk, int F,
                                                         T* __restrict__ dp, float* __restrict__ dw) {
  constexpr int VEC = 16 / sizeof(T);
  const int lane = threadIdx.x & 63;
  const int j = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (j >= nk) return;  // whole waves
  const float g = gr[j];
  const T* pr = P + (size_t)j * F;
  const T* ur = U + (size_t)j * F;
  T* dr = dp + (size_t)j * F;
  float s = 0.f;
  for (int f = lane * VEC; f < F; f += 64 * VEC) {
    Chunk<T> pc, uc, o;
    pc.raw = *(const u32x4*)(pr + f);
    uc.raw = *(const u32x4*)(ur + f);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const float rp = fmaxf(to_f(pc.e[i]), 0.f);
      const float h = rnd<T>(rp * rp);
      const float u = to_f(uc.e[i]);
      s = __builtin_fmaf(h, u, s);
      o.e[i] = from_f<T>(g * u * 2.f * rp);
    }
    *(u32x4*)(dr + f) = o.raw;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
  if (lane == 0) dw[j] = s;
}

// The packed token ranges of the weight-gradient products: range e holds
// expert e's rows (count c_e) in koff[e] .. koff[e+1], of length c_e rounded
// up to 128 (128 for an expert with no rows, so that no range is empty); the
// columns past c_e are zero.  One thread.
__global__ void exb_koff_kernel(const int* __restrict__ off, int E, int* __restrict__ koff) {
  if (threadIdx.x != 0) return;
  int acc = 0;
  koff[0] = 0;
  for (int e = 0; e < E; ++e) {
    const int c = off[e + 1] - off[e];
    acc += c > 0 ? (c + 127) / 128 * 128 : 128;
    koff[e + 1] = acc;
  }
}

// dst (W x ld) from src (nk x W) rows in perm order: column koff[e] + i of
// dst is row off[e] + i of src for i < off[e+1] − off[e], zero after, up to
// koff[e+1].  MODE 1 writes relu(v)² rounded (h from p), MODE 2 writes
// round(v · gr[row]).  64x64 tiles through LDS; W a multiple of 64; blocks
// past koff[E] exit.
template <typename T, int MODE>
__global__ __launch_bounds__(256) void exb_seg_transpose_kernel(const T* __restrict__ src, int W,
                                                                const int* __restrict__ off,
                                                                const int* __restrict__ koff, int E,
                                                                const float* __restrict__ gr, T* __restrict__ dst,
                                                                int ldd) {
  constexpr int VEC = 16 / sizeof(T), CPR = 64 / VEC;
  __shared__ float tile[64][65];
  const int w0 = blockIdx.x * 64, c0 = blockIdx.y * 64;
  if (c0 >= koff[E]) return;  // the whole workgroup
  int e = 0;
  while (e + 1 < E && koff[e + 1] <= c0) ++e;
  const int i0 = c0 - koff[e];
  const int r0 = off[e], nrow = off[e + 1] - r0;
  for (int q = threadIdx.x; q < 64 * CPR; q += 256) {
    const int il = q / CPR, cq = q - il * CPR, i = i0 + il;
    Chunk<T> c;
    c.raw = i < nrow ? *(const u32x4*)(src + (size_t)(r0 + i) * W + w0 + cq * VEC) : zero4();
    const float sc = MODE == 2 && i < nrow ? gr[r0 + i] : 1.f;
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      float f = to_f(c.e[v]);
      if constexpr (MODE == 1) {
        f = fmaxf(f, 0.f);
        f = rnd<T>(f * f);
      } else if constexpr (MODE == 2) {
        f = rnd<T>(f * sc);
      }
      tile[il][cq * VEC + v] = f;
    }
  }
  __syncthreads();
  for (int q = threadIdx.x; q < 64 * CPR; q += 256) {
    const int wl = q / CPR, cq = q - wl * CPR;
    Chunk<T> c;
#pragma unroll
    for (int v = 0; v < VEC; ++v) c.e[v] = from_f<T>(tile[cq * VEC + v][wl]);
    *(u32x4*)(dst + (size_t)(w0 + wl) * ldd + c0 + cq * VEC) = c.raw;
  }
}

constexpr int kRouteMaxE = 64;

// Router cotangents per token (moe.py:56-86): the slot cotangents dg_s =
// dw[inv[t·k+s]] through the softmax of the selected logits, plus
// d_aux·(E/N)·P ⊙ (f − <P, f>) and d_z·(2·lse/N)·P, with f_e = count_e/(N·k).
// DWT, BY_ASSIGN: the slot cotangents' type and order — fp32 in perm order
// (dw[inv[t·k + s]], the full-expert layer's), or the gates' dtype in
// assignment order (dw[t·k + s], the standalone router's); dw may be null
// (no gate cotangent).
template <typename DWT, bool BY_ASSIGN>
__global__ __launch_bounds__(256) void exb_route_kernel(const float* __restrict__ logits,
                                                        const int* __restrict__ inds, const int* __restrict__ inv,
                                                        const DWT* __restrict__ dw, const int* __restrict__ off,
                                                        const float* __restrict__ dloss, int N, int E, int k,
                                                        float* __restrict__ dl) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N) return;
  const float* lr = logits + (size_t)t * E;
  float* out = dl + (size_t)t * E;
  float mx = -INFINITY;
  for (int e = 0; e < E; ++e) mx = fmaxf(mx, lr[e]);
  double se = 0.0, sl = 0.0;
  for (int e = 0; e < E; ++e) {
    se += exp((double)lr[e] - mx);
    sl += exp((double)lr[e]);
  }
  const double lse = log(sl);
  const double da = dloss ? dloss[0] : 0.0, dz = dloss ? dloss[1] : 0.0;
  double pf = 0.0;
  for (int e = 0; e < E; ++e) pf += exp((double)lr[e] - mx) / se * ((double)(off[e + 1] - off[e]) / ((double)N * k));
  for (int e = 0; e < E; ++e) {
    const double P = exp((double)lr[e] - mx) / se;
    const double f = (double)(off[e + 1] - off[e]) / ((double)N * k);
    out[e] = (float)(da * ((double)E / N) * P * (f - pf) + dz * (2.0 * lse / N) * P);
  }
  // the selected logits' softmax (the gates before rounding)
  // (ids outside [0, E) or rows outside [0, N·k) take no part)
  double gs[8], dg[8], m = -INFINITY, den = 0.0, gdg = 0.0;
  int es[8];
  for (int s = 0; s < k; ++s) {
    const int e = inds[(size_t)t * k + s], j = inv[(size_t)t * k + s];
    es[s] = e >= 0 && e < E && j >= 0 && j < N * k ? e : -1;
    if (es[s] >= 0) m = fmax(m, (double)lr[e]);
  }
  for (int s = 0; s < k; ++s) {
    gs[s] = es[s] >= 0 ? exp((double)lr[es[s]] - m) : 0.0;
    den += gs[s];
  }
  for (int s = 0; s < k; ++s) {
    gs[s] = den > 0.0 ? gs[s] / den : 0.0;
    const size_t a = (size_t)t * k + s;
    dg[s] = es[s] >= 0 && dw ? (double)to_f(dw[BY_ASSIGN ? a : (size_t)inv[a]]) : 0.0;
    gdg += gs[s] * dg[s];
  }
  for (int s = 0; s < k; ++s)
    if (es[s] >= 0) out[es[s]] = (float)((double)out[es[s]] + gs[s] * (dg[s] - gdg));
}

// dx[t] = Σ_s dk[row of (t,s)] ⊙ (1 − x_k[e_s]) + Σ_s dk[row of (t+1,s)] ⊙ x_k[e'_s]
//         (t+1 in t's sequence) + Σ_e dℓ[t,e]·W_gate[e], in that order; the
// first token of a sequence also gives d x_prev = Σ_s dk ⊙ x_k[e_s].
template <typename T>
__global__ __launch_bounds__(256) void exb_dx_kernel(const T* __restrict__ dk, const int* __restrict__ inv,
                                                     const int* __restrict__ inds, const T* __restrict__ mu,
                                                     const float* __restrict__ dl, const T* __restrict__ wg, int N,
                                                     int T_, int C, int E, int k, T* __restrict__ dx,
                                                     T* __restrict__ dxprev) {
  constexpr int VEC = 16 / sizeof(T);
  const int cpr = C / VEC;
  const size_t id = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (id >= (size_t)N * cpr) return;
  const int t = (int)(id / cpr), c = (int)(id % cpr) * VEC;
  float acc[VEC], ap[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) acc[v] = ap[v] = 0.f;
  for (int s = 0; s < k && dk; ++s) {
    const int a = t * k + s, e = inds[a], j = inv[a];
    if (e < 0 || e >= E || j < 0 || j >= N * k) continue;  // ids the dispatch dropped add nothing
    Chunk<T> d, m;
    d.raw = *(const u32x4*)(dk + (size_t)j * C + c);
    m.raw = *(const u32x4*)(mu + (size_t)e * C + c);
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      acc[v] += to_f(d.e[v]) * (1.f - to_f(m.e[v]));
      ap[v] += to_f(d.e[v]) * to_f(m.e[v]);
    }
  }
  if ((t + 1) % T_ != 0 && dk) {
    for (int s = 0; s < k; ++s) {
      const int a = (t + 1) * k + s, e = inds[a], j = inv[a];
      if (e < 0 || e >= E || j < 0 || j >= N * k) continue;
      Chunk<T> d, m;
      d.raw = *(const u32x4*)(dk + (size_t)j * C + c);
      m.raw = *(const u32x4*)(mu + (size_t)e * C + c);
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] += to_f(d.e[v]) * to_f(m.e[v]);
    }
  }
  for (int e = 0; e < E; ++e) {
    const float g = dl[(size_t)t * E + e];
    Chunk<T> w;
    w.raw = *(const u32x4*)(wg + (size_t)e * C + c);
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] += g * to_f(w.e[v]);
  }
  Chunk<T> o;
#pragma unroll
  for (int v = 0; v < VEC; ++v) o.e[v] = from_f<T>(acc[v]);
  if (dx) *(u32x4*)(dx + (size_t)t * C + c) = o.raw;
  if (dxprev && t % T_ == 0) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) o.e[v] = from_f<T>(ap[v]);
    *(u32x4*)(dxprev + (size_t)(t / T_) * C + c) = o.raw;
  }
}

// Column sums in R fixed row chunks, written as part[e][r][c] (e < E):
//   MODE 0 (d x_k): the rows j of expert e (perm order) in chunk r, term
//                   dk[j][c] · round(shift(x)[t] − x[t])[c], t = perm[j] / k
//   MODE 1 (d W_gate): the tokens t of chunk r, term dℓ[t][e] · x[t][c], for
//                   the 8 experts of block column blockIdx.y at once
// A thread owns 16 bytes of columns (c .. c + VEC) and walks its rows in
// ascending order; the chunk sums are added in ascending r by the finish
// kernel, so every result is independent of timing.
constexpr int kGateTile = 8;

template <typename T, int MODE>
__global__ __launch_bounds__(256) void exb_colsum_kernel(const T* __restrict__ a, const T* __restrict__ x,
                                                         const T* __restrict__ xprev, const int* __restrict__ off,
                                                         const int* __restrict__ perm, const float* __restrict__ dl,
                                                         int N, int T_, int C, int E, int k, int R,
                                                         float* __restrict__ part) {
  constexpr int VEC = 16 / sizeof(T);
  const int r = blockIdx.x;
  const int cpr = C / VEC;
  if constexpr (MODE == 0) {
    const int e = blockIdx.y;
    const int r0 = off[e], nrow = off[e + 1] - r0;
    const int per = (nrow + R - 1) / R;
    const int lo = r0 + min(r * per, nrow), hi = r0 + min((r + 1) * per, nrow);
    for (int cc = threadIdx.x; cc < cpr; cc += 256) {
      const int c = cc * VEC;
      float acc[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] = 0.f;
      for (int j = lo; j < hi; ++j) {
        const int t = perm[j] / k, ts = t % T_;
        Chunk<T> d, xc, pc;
        d.raw = *(const u32x4*)(a + (size_t)j * C + c);
        xc.raw = *(const u32x4*)(x + (size_t)t * C + c);
        pc.raw = ts > 0 ? *(const u32x4*)(x + (size_t)(t - 1) * C + c)
                        : (xprev ? *(const u32x4*)(xprev + (size_t)(t / T_) * C + c) : zero4());
#pragma unroll
        for (int v = 0; v < VEC; ++v)
          acc[v] = __builtin_fmaf(to_f(d.e[v]), rnd<T>(to_f(pc.e[v]) - to_f(xc.e[v])), acc[v]);
      }
      float* dst = part + ((size_t)e * R + r) * C + c;
#pragma unroll
      for (int v = 0; v < VEC; ++v) dst[v] = acc[v];
    }
  } else {
    const int e0 = blockIdx.y * kGateTile, ne = min(kGateTile, E - e0);
    const int per = (N + R - 1) / R;
    const int lo = min(r * per, N), hi = min((r + 1) * per, N);
    for (int cc = threadIdx.x; cc < cpr; cc += 256) {
      const int c = cc * VEC;
      float acc[kGateTile][VEC];
#pragma unroll
      for (int q = 0; q < kGateTile; ++q)
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[q][v] = 0.f;
      for (int t = lo; t < hi; ++t) {
        Chunk<T> xc;
        xc.raw = *(const u32x4*)(x + (size_t)t * C + c);
        const float* dr = dl + (size_t)t * E + e0;
#pragma unroll
        for (int q = 0; q < kGateTile; ++q) {
          const float g = q < ne ? dr[q] : 0.f;
#pragma unroll
          for (int v = 0; v < VEC; ++v) acc[q][v] = __builtin_fmaf(g, to_f(xc.e[v]), acc[q][v]);
        }
      }
#pragma unroll
      for (int q = 0; q < kGateTile; ++q) {
        if (q >= ne) break;
        float* dst = part + ((size_t)(e0 + q) * R + r) * C + c;
#pragma unroll
        for (int v = 0; v < VEC; ++v) dst[v] = acc[q][v];
      }
    }
  }
}

// out[e][c] = Σ_r part[e][r][c]: a workgroup of 16 waves takes 64 columns of
// one e; wave q adds r = q·R/16 .. (q+1)·R/16 − 1 in ascending order, then
// the 16 wave sums are added in ascending q (R is a multiple of 8; a fixed
// association either way).
constexpr int kFinWaves = 16;

template <typename T>
__global__ __launch_bounds__(64 * kFinWaves) void exb_colsum_finish_kernel(const float* __restrict__ part, int E,
                                                                          int R, int C, T* __restrict__ out) {
  __shared__ float red[kFinWaves][64];
  const int lane = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int cb = C / 64;
  const int e = blockIdx.x / cb, c = (blockIdx.x % cb) * 64 + lane;
  const int per = (R + kFinWaves - 1) / kFinWaves;
  const int lo = min(q * per, R), hi = min((q + 1) * per, R);
  float s = 0.f;
  for (int r = lo; r < hi; ++r) s += part[((size_t)e * R + r) * C + c];
  red[q][lane] = s;
  __syncthreads();
  if (q == 0) {
    float t = red[0][lane];
#pragma unroll
    for (int w = 1; w < kFinWaves; ++w) t += red[w][lane];
    out[(size_t)e * C + c] = from_f<T>(t);
  }
}

}  // namespace

int exb_col_chunks(int N, int C, int E) {
  int R = std::min(256, std::max(8, (N + 15) / 16));
  while (R > 8 && (long long)E * R * C > (1ll << 24)) R /= 2;
  return R;
}


hipError_t launch_exb_gather(int dtype, const void* dO, const int* perm, const float* logits, const int* inds,
                             int nk, int C, int E, int k, void* dog, float* gr, hipStream_t s) {
  const size_t total = (size_t)nk * (C / (dtype == 0 ? 4 : 8));
  const dim3 grid((unsigned)((total + 255) / 256));
  RWKV_DISPATCH_DTYPE(dtype, T, {
    launch_kernel(exb_gather_kernel<T>, grid, dim3(256), 0, s, (const T*)dO, perm, logits, inds, nk, C, E, k,
                       (T*)dog, gr);
  });
  return mark(hipGetLastError(), "experts_bwd_gather", s);
}

hipError_t launch_exb_hidden(int dtype, const void* P, const void* U, const float* gr, int nk, int F, void* dp,
                             float* dw, hipStream_t s) {
  if (F % 64) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((nk + 3) / 4));
  RWKV_DISPATCH_DTYPE(dtype, T, {
    launch_kernel(exb_hidden_kernel<T>, grid, dim3(256), 0, s, (const T*)P, (const T*)U, gr, nk, F, (T*)dp, dw);
  });
  return mark(hipGetLastError(), "experts_bwd_hidden", s);
}

hipError_t launch_exb_koff(const int* off, int E, int* koff, hipStream_t s) {
  launch_kernel(exb_koff_kernel, dim3(1), dim3(64), 0, s, off, E, koff);
  return mark(hipGetLastError(), "experts_bwd_koff", s);
}

int exb_seg_cols(int nk, int E) { return (nk + 128 * E + 127) / 128 * 128; }

hipError_t launch_exb_seg_transpose(int dtype, int mode, const void* src, int W, const int* off, const int* koff,
                                    int E, int ld, const float* gr, void* dst, hipStream_t s) {
  if (W % 64 || ld % 128) return hipErrorInvalidValue;
  const dim3 grid(W / 64, ld / 64);
  RWKV_DISPATCH_DTYPE(dtype, T, {
    if (mode == 1)
      launch_kernel((exb_seg_transpose_kernel<T, 1>), grid, dim3(256), 0, s, (const T*)src, W, off, koff, E, gr,
                         (T*)dst, ld);
    else if (mode == 2)
      launch_kernel((exb_seg_transpose_kernel<T, 2>), grid, dim3(256), 0, s, (const T*)src, W, off, koff, E, gr,
                         (T*)dst, ld);
    else
      launch_kernel((exb_seg_transpose_kernel<T, 0>), grid, dim3(256), 0, s, (const T*)src, W, off, koff, E, gr,
                         (T*)dst, ld);
  });
  return mark(hipGetLastError(), "experts_bwd_transpose", s);
}

hipError_t launch_exb_route(const float* logits, const int* inds, const int* inv, const float* dw, const int* off,
                            const float* dloss, int N, int E, int k, float* dl, hipStream_t s) {
  if (E > kRouteMaxE || k > 8) return hipErrorInvalidValue;
  launch_kernel((exb_route_kernel<float, false>), dim3((N + 255) / 256), dim3(256), 0, s, logits, inds, inv, dw, off,
                dloss, N, E, k, dl);
  return mark(hipGetLastError(), "experts_bwd_route", s);
}

hipError_t launch_router_route(int dtype, const float* logits, const int* inds, const int* inv, const void* d_gates,
                               const int* off, const float* dloss, int N, int E, int k, float* dl, hipStream_t s) {
  if (E > kRouteMaxE || k > 8) return hipErrorInvalidValue;
  RWKV_DISPATCH_DTYPE(dtype, T, {
    launch_kernel((exb_route_kernel<T, true>), dim3((N + 255) / 256), dim3(256), 0, s, logits, inds, inv,
                  (const T*)d_gates, off, dloss, N, E, k, dl);
  });
  return mark(hipGetLastError(), "router_bwd_route", s);
}

hipError_t launch_exb_dx(int dtype, const void* dk, const int* inv, const int* inds, const void* mu, const float* dl,
                         const void* wg, int N, int T_, int C, int E, int k, void* dx, void* dxprev, hipStream_t s) {
  const size_t total = (size_t)N * (C / (dtype == 0 ? 4 : 8));
  const dim3 grid((unsigned)((total + 255) / 256));
  RWKV_DISPATCH_DTYPE(dtype, T, {
    launch_kernel(exb_dx_kernel<T>, grid, dim3(256), 0, s, (const T*)dk, inv, inds, (const T*)mu, dl,
                       (const T*)wg, N, T_, C, E, k, (T*)dx, (T*)dxprev);
  });
  return mark(hipGetLastError(), "experts_bwd_dx", s);
}

hipError_t launch_exb_colsum(int dtype, int mode, const void* a, const void* x, const void* xprev, const int* off,
                             const int* perm, const float* dl, int N, int T_, int C, int E, int k, float* part,
                             void* out, hipStream_t s) {
  const int R = exb_col_chunks(N, C, E);
  const dim3 grid(R, mode == 0 ? E : (E + kGateTile - 1) / kGateTile);
  RWKV_DISPATCH_DTYPE(dtype, T, {
    if (mode == 0)
      launch_kernel((exb_colsum_kernel<T, 0>), grid, dim3(256), 0, s, (const T*)a, (const T*)x,
                         (const T*)xprev, off, perm, dl, N, T_, C, E, k, R, part);
    else
      launch_kernel((exb_colsum_kernel<T, 1>), grid, dim3(256), 0, s, (const T*)a, (const T*)x,
                         (const T*)xprev, off, perm, dl, N, T_, C, E, k, R, part);
    if (const hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    launch_kernel(exb_colsum_finish_kernel<T>, dim3(E * (C / 64)), dim3(64 * kFinWaves), 0, s, part, E, R, C,
                       (T*)out);
  });
  return mark(hipGetLastError(), mode == 0 ? "experts_bwd_dxk" : "experts_bwd_dwg", s);
}

}  // namespace rwkvmoe
