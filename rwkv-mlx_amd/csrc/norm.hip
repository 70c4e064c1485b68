// ln2 of the Block in front of the ChannelMix (model.py:321 with
// nn.LayerNorm(C), model.py:283; the RNN form _layer_norm_1d, model.py:434-438):
//   y = (x - mean) / sqrt(var + 1e-5) · w + b,   per token row of C values,
// mean and var = mean((x - mean)²) over the row, with the order-fixed fp64
// arithmetic of ln.h (the router's fused form uses the same, so the two give
// the same bits).  For fp16 rows the sum of x is exact in fp64 (every value
// is a multiple of 2^-24 below 2^16, so the row sum stays within 53 bits),
// so the mean does not depend on the order at all.
//
// Sixteen lanes per row, 16 rows per workgroup of 256 threads.  Rows of up
// to 16·kLnHeld chunks stay in registers, and ln2's weight and bias are
// requested with them, so a row costs one memory round trip; wider rows are
// re-read for each pass (L1 / L2 hits after the first).
#include <algorithm>

#include "common.h"
#include "internal.h"
#include "ln.h"

namespace rwkvmoe {
namespace {

constexpr int kLnRows = 256 / kLnGroup;
constexpr int kLnHeld = 8;  // chunks per lane held in registers

template <typename T>
__global__ __launch_bounds__(256) void layer_norm_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                         const T* __restrict__ b, T* __restrict__ y, int N, int C) {
  constexpr int VEC = 16 / sizeof(T);
  const int j = threadIdx.x % kLnGroup;
  const int row = min(blockIdx.x * kLnRows + (int)threadIdx.x / kLnGroup, N - 1);
  const bool live = blockIdx.x * kLnRows + (int)threadIdx.x / kLnGroup < N;  // (dead groups mirror the last row)
  const int cpr = C / VEC;
  const T* xr = x + (size_t)row * C;
  T* yr = y + (size_t)row * C;
  if (cpr <= kLnGroup * kLnHeld) {
    Chunk<T> v[kLnHeld], wc[kLnHeld], bc[kLnHeld];
#pragma unroll
    for (int i = 0; i < kLnHeld; ++i) {
      const int ch = min(j + kLnGroup * i, cpr - 1);  // (clamped: loads without branches)
      v[i].raw = *(const u32x4*)(xr + ch * VEC);
      wc[i].raw = *(const u32x4*)(w + ch * VEC);
      bc[i].raw = *(const u32x4*)(b + ch * VEC);
    }
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < kLnHeld; ++i)
      if (j + kLnGroup * i < cpr) s = ln_add(s, v[i]);
    const double mean = ln_group_sum(s) / (double)C;
    double q = 0.0;
#pragma unroll
    for (int i = 0; i < kLnHeld; ++i)
      if (j + kLnGroup * i < cpr) q = ln_add_sq(q, v[i], mean);
    const double rstd = ln_rstd(ln_group_sum(q), C);
#pragma unroll
    for (int i = 0; i < kLnHeld; ++i) {
      const int ch = j + kLnGroup * i;
      if (live && ch < cpr) *(u32x4*)(yr + ch * VEC) = ln_apply(v[i], wc[i], bc[i], (float)mean, (float)rstd).raw;
    }
    return;
  }
  double s = 0.0;
  for (int ch = j; ch < cpr; ch += kLnGroup) {
    Chunk<T> c;
    c.raw = *(const u32x4*)(xr + ch * VEC);
    s = ln_add(s, c);
  }
  const double mean = ln_group_sum(s) / (double)C;
  double q = 0.0;
  for (int ch = j; ch < cpr; ch += kLnGroup) {
    Chunk<T> c;
    c.raw = *(const u32x4*)(xr + ch * VEC);
    q = ln_add_sq(q, c, mean);
  }
  const double rstd = ln_rstd(ln_group_sum(q), C);
  for (int ch = j; ch < cpr; ch += kLnGroup) {
    Chunk<T> c, wc, bc;
    c.raw = *(const u32x4*)(xr + ch * VEC);
    wc.raw = *(const u32x4*)(w + ch * VEC);
    bc.raw = *(const u32x4*)(b + ch * VEC);
    const Chunk<T> o = ln_apply(c, wc, bc, (float)mean, (float)rstd);
    if (live) *(u32x4*)(yr + ch * VEC) = o.raw;
  }
}

// ---- the VJP of ln2 ----------------------------------------------------------------
// With g = dy·w and x̂ = (x - mean)·rstd (the forward's fp32 d, from the
// same ln.h statistics):
//   dx = rstd·(g - mean(g) - x̂·mean(g·x̂)) [+ d_res],
//   dw = Σ_rows dy·x̂,   db = Σ_rows dy.
// Row sums in fp64 (a chunk's pairwise tree, then the lanes' butterfly, as
// ln.h); dx in fp32, rounded to T.  The column sums take a fixed order, so
// results do not depend on timing: a workgroup's 16 rows in ascending row
// order through an LDS slab, its passes (rows r0, r0 + 16·grid, ...) in
// ascending order into its own fp32 partial row, then the workgroups in
// ascending order (layer_norm_bwd_cols_kernel).

constexpr int kLnbMaxBlocks = 1024;  // partial rows: at most this many workgroups

int lnb_blocks(int N) { return std::min((N + kLnRows - 1) / kLnRows, kLnbMaxBlocks); }

// fp64 row sums of g and g·x̂ over one chunk
template <typename T>
RWKV_DEV void lnb_sums(const Chunk<T>& x, const Chunk<T>& dy, const Chunk<T>& w, float m, float rs, double& sa,
                       double& sb) {
  constexpr int VEC = 16 / sizeof(T);
  double ta[VEC], tb[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    const float xh = (to_f(x.e[e]) - m) * rs;
    const float g = to_f(dy.e[e]) * to_f(w.e[e]);
    ta[e] = (double)g;
    tb[e] = (double)g * (double)xh;
  }
  sa += ln_tree<VEC>(ta);
  sb += ln_tree<VEC>(tb);
}

// dx of one chunk (written when `store`), and its column products into the
// slab (zeros for a dead row or a chunk past the row's end)
template <typename T>
RWKV_DEV void lnb_apply(const Chunk<T>& x, const Chunk<T>& dy, const Chunk<T>& w, const T* dres, T* dx, bool store,
                        bool live, float m, float rs, float ma, float mb, float* pw, float* pb) {
  constexpr int VEC = 16 / sizeof(T);
  Chunk<T> r, o;
  if (dres && store) r.raw = *(const u32x4*)dres;
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    const float xh = (to_f(x.e[e]) - m) * rs;
    const float yv = to_f(dy.e[e]);
    float v = rs * ((yv * to_f(w.e[e]) - ma) - xh * mb);
    if (dres && store) v += to_f(r.e[e]);
    o.e[e] = from_f<T>(v);
    pw[e] = live ? yv * xh : 0.f;
    pb[e] = live ? yv : 0.f;
  }
  if (store) *(u32x4*)dx = o.raw;
}

template <typename T, bool HELD>
__global__ __launch_bounds__(256) void layer_norm_bwd_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                             const T* dy, const T* dres, T* dx,
                                                             float* __restrict__ part, int N, int C) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int SLAB = kLnGroup * VEC;  // the columns of one chunk index across a row's 16 lanes
  __shared__ float slab[2][kLnRows][SLAB];
  const int j = threadIdx.x % kLnGroup, rg = threadIdx.x / kLnGroup;
  const int cpr = C / VEC, nch = (cpr + kLnGroup - 1) / kLnGroup;
  auto ld = [](const T* p, int ch) {
    Chunk<T> c;
    c.raw = *(const u32x4*)(p + ch * VEC);
    return c;
  };
  // the slab of chunk index i: 16 rows' products, summed per column in row
  // order into this workgroup's partial row (pass 0 writes, later passes add)
  auto reduce = [&](int i, int pass, const float* pw, const float* pb) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      slab[0][rg][j * VEC + e] = pw[e];
      slab[1][rg][j * VEC + e] = pb[e];
    }
    __syncthreads();
    if ((int)threadIdx.x < 2 * SLAB) {
      const int q = threadIdx.x / SLAB, cc = threadIdx.x % SLAB, col = i * SLAB + cc;
      float t = 0.f;
#pragma unroll
      for (int r = 0; r < kLnRows; ++r) t += slab[q][r][cc];
      if (col < C) {
        float* pp = part + ((size_t)blockIdx.x * 2 + q) * C + col;
        *pp = pass ? *pp + t : t;
      }
    }
    __syncthreads();
  };
  for (int pass = 0, r0 = blockIdx.x * kLnRows; r0 < N; ++pass, r0 += gridDim.x * kLnRows) {
    const bool live = r0 + rg < N;  // (dead rows mirror the last row and add zeros)
    const int row = min(r0 + rg, N - 1);
    const T* xr = x + (size_t)row * C;
    const T* dyr = dy + (size_t)row * C;
    const T* rr = dres ? dres + (size_t)row * C : nullptr;
    T* dxr = dx ? dx + (size_t)row * C : nullptr;
    float pw[VEC], pb[VEC];
    if constexpr (HELD) {
      Chunk<T> xv[kLnHeld], dv[kLnHeld], wv[kLnHeld];
#pragma unroll
      for (int i = 0; i < kLnHeld; ++i) {
        const int ch = min(j + kLnGroup * i, cpr - 1);
        xv[i] = ld(xr, ch);
        dv[i] = ld(dyr, ch);
        wv[i] = ld(w, ch);
      }
      double s = 0.0;
#pragma unroll
      for (int i = 0; i < kLnHeld; ++i)
        if (j + kLnGroup * i < cpr) s = ln_add(s, xv[i]);
      const double mean = ln_group_sum(s) / (double)C;
      double q = 0.0;
#pragma unroll
      for (int i = 0; i < kLnHeld; ++i)
        if (j + kLnGroup * i < cpr) q = ln_add_sq(q, xv[i], mean);
      const float m = (float)mean, rs = (float)ln_rstd(ln_group_sum(q), C);
      double sa = 0.0, sb = 0.0;
#pragma unroll
      for (int i = 0; i < kLnHeld; ++i)
        if (j + kLnGroup * i < cpr) lnb_sums(xv[i], dv[i], wv[i], m, rs, sa, sb);
      const float ma = (float)(ln_group_sum(sa) / (double)C), mb = (float)(ln_group_sum(sb) / (double)C);
#pragma unroll
      for (int i = 0; i < kLnHeld; ++i) {
        if (i >= nch) break;
        const int ch = j + kLnGroup * i;
        const bool in = ch < cpr;
        lnb_apply(xv[i], dv[i], wv[i], rr ? rr + ch * VEC : nullptr, dxr ? dxr + ch * VEC : nullptr,
                  dxr && live && in, live && in, m, rs, ma, mb, pw, pb);
        if (part) reduce(i, pass, pw, pb);
      }
    } else {  // wide rows: each pass over the row re-reads it (L1 / L2 hits after the first)
      double s = 0.0;
      for (int ch = j; ch < cpr; ch += kLnGroup) s = ln_add(s, ld(xr, ch));
      const double mean = ln_group_sum(s) / (double)C;
      double q = 0.0;
      for (int ch = j; ch < cpr; ch += kLnGroup) q = ln_add_sq(q, ld(xr, ch), mean);
      const float m = (float)mean, rs = (float)ln_rstd(ln_group_sum(q), C);
      double sa = 0.0, sb = 0.0;
      for (int ch = j; ch < cpr; ch += kLnGroup) lnb_sums(ld(xr, ch), ld(dyr, ch), ld(w, ch), m, rs, sa, sb);
      const float ma = (float)(ln_group_sum(sa) / (double)C), mb = (float)(ln_group_sum(sb) / (double)C);
      for (int i = 0; i < nch; ++i) {
        const int ch = min(j + kLnGroup * i, cpr - 1);
        const bool in = j + kLnGroup * i < cpr;
        lnb_apply(ld(xr, ch), ld(dyr, ch), ld(w, ch), rr ? rr + ch * VEC : nullptr, dxr ? dxr + ch * VEC : nullptr,
                  dxr && live && in, live && in, m, rs, ma, mb, pw, pb);
        if (part) reduce(i, pass, pw, pb);
      }
    }
  }
}

// dw and db: the partial rows of `nblk` workgroups summed in ascending order
// (each wave a quarter of them, the quarters then in order).  Entry e of
// [dw | db] is column e of dw for e < C, else column e - C of db.
template <typename T>
__global__ __launch_bounds__(256) void layer_norm_bwd_cols_kernel(const float* __restrict__ part, int nblk, int C,
                                                                  T* dw, T* db) {
  __shared__ float red[4][64];
  const int lane = threadIdx.x % 64, wv = threadIdx.x / 64;
  const int e = blockIdx.x * 64 + lane;
  float t = 0.f;
  if (e < 2 * C) {
    const int b0 = wv * nblk / 4, b1 = (wv + 1) * nblk / 4;
#pragma unroll 8
    for (int b = b0; b < b1; ++b) t += part[(size_t)b * 2 * C + e];
  }
  red[wv][lane] = t;
  __syncthreads();
  if (wv == 0 && e < 2 * C) {
    const float v = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
    T* o = e < C ? dw : db;
    if (o) o[e < C ? e : e - C] = from_f<T>(v);
  }
}

}  // namespace

size_t layer_norm_bwd_part_bytes(int N, int C) { return (size_t)lnb_blocks(N) * 2 * C * sizeof(float); }

hipError_t launch_layer_norm_bwd(int dtype, const void* x, const void* w, const void* dy, const void* dres, void* dx,
                                 void* dw, void* db, float* part, int N, int C, hipStream_t s) {
  if (N < 1 || C < 64 || C > 8192 || C % 64) return hipErrorInvalidValue;
  const bool cols = dw || db;
  if (cols && !part) return hipErrorInvalidValue;
  const int nb = lnb_blocks(N);
  RWKV_DISPATCH_DTYPE(dtype, T, {
    const bool held = C / (int)(16 / sizeof(T)) <= kLnGroup * kLnHeld;
    if (held)
      launch_kernel(layer_norm_bwd_kernel<T, true>, dim3(nb), dim3(256), 0, s, (const T*)x, (const T*)w,
                    (const T*)dy, (const T*)dres, (T*)dx, cols ? part : nullptr, N, C);
    else
      launch_kernel(layer_norm_bwd_kernel<T, false>, dim3(nb), dim3(256), 0, s, (const T*)x, (const T*)w,
                    (const T*)dy, (const T*)dres, (T*)dx, cols ? part : nullptr, N, C);
  });
  const hipError_t e = mark(hipGetLastError(), "layer_norm_bwd", s);
  if (e != hipSuccess || !cols) return e;
  RWKV_DISPATCH_DTYPE(dtype, T, {
    launch_kernel(layer_norm_bwd_cols_kernel<T>, dim3((2 * C + 63) / 64), dim3(256), 0, s, (const float*)part, nb,
                  C, (T*)dw, (T*)db);
  });
  return mark(hipGetLastError(), "layer_norm_bwd_cols", s);
}

hipError_t launch_layer_norm(int dtype, const void* x, const void* w, const void* b, void* y, int N, int C,
                             hipStream_t s) {
  if (N < 1 || C < 64 || C > 8192 || C % 64) return hipErrorInvalidValue;
  const dim3 grid((N + kLnRows - 1) / kLnRows);
  RWKV_DISPATCH_DTYPE(dtype, T, {
    launch_kernel(layer_norm_kernel<T>, grid, dim3(256), 0, s, (const T*)x, (const T*)w, (const T*)b,
                       (T*)y, N, C);
  });
  return mark(hipGetLastError(), "layer_norm", s);
}

}  // namespace rwkvmoe
