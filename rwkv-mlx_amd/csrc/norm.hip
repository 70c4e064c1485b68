// ln2 of the Block in front of the ChannelMix (model.py:321 with
// nn.LayerNorm(C), model.py:283; the RNN form _layer_norm_1d, model.py:434-438):
//   y = (x - mean) / sqrt(var + 1e-5) · w + b,   per token row of C values,
// mean and var = mean((x - mean)²) over the row, with the order-fixed fp64
// arithmetic of ln.h (the router's fused form uses the same, so the two give
// the same bits).  For fp16 rows the sum of x is exact in fp64 (every value
// is a multiple of 2^-24 below 2^16, so the row sum stays within 53 bits),
// so the mean does not depend on the order at all.
//
// Sixteen lanes per row, 16 rows per workgroup of 256 threads; the passes
// re-read the row (L1 / L2 hits after the first).
#include "common.h"
#include "internal.h"
#include "ln.h"

namespace rwkvmoe {
namespace {

constexpr int kLnRows = 256 / kLnGroup;

template <typename T>
__global__ __launch_bounds__(256) void layer_norm_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                         const T* __restrict__ b, T* __restrict__ y, int N, int C) {
  constexpr int VEC = 16 / sizeof(T);
  const int j = threadIdx.x % kLnGroup;
  const int row = min(blockIdx.x * kLnRows + (int)threadIdx.x / kLnGroup, N - 1);
  const bool live = blockIdx.x * kLnRows + (int)threadIdx.x / kLnGroup < N;  // (dead groups mirror the last row)
  const int cpr = C / VEC;
  const T* xr = x + (size_t)row * C;
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
  T* yr = y + (size_t)row * C;
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
    hipLaunchKernelGGL(layer_norm_kernel<T>, grid, dim3(256), 0, s, (const T*)x, (const T*)w, (const T*)b,
                       (T*)y, N, C);
  });
  return mark(hipGetLastError(), "layer_norm", s);
}

}  // namespace rwkvmoe
