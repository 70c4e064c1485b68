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

}  // namespace

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
