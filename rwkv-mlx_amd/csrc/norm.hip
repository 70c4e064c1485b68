// ln2 of the Block in front of the ChannelMix (model.py:321 with
// nn.LayerNorm(C), model.py:283; the RNN form _layer_norm_1d, model.py:434-438):
//   y = (x - mean) / sqrt(var + 1e-5) · w + b,   per token row of C values,
// mean and var = mean((x - mean)²) over the row.  Definition (order fixed):
// every operation in fp64 — the row sums as per-lane partial sums over the
// lane's 16-byte chunks in ascending order, then an xor butterfly over the
// wave (each step adds the same two values on both lanes, so every lane holds
// the same total); y = ((x - mean) · rstd) · w + b with rstd = 1 / sqrt(var +
// 1e-5), each step one fp64 rounding — then y goes to fp32 and from there to
// the row's dtype (round to nearest even both times).  For fp16 rows the sum
// of x is exact in fp64 (every value is a multiple of 2^-24 below 2^16, so
// the row sum stays within 53 bits), so the mean does not depend on the
// order at all.
//
// One wave per row, four rows per workgroup; the row stays in registers
// between the two reductions and the output pass (C ≤ 8192: at most 16
// 16-byte chunks per lane for 16-bit rows, 32 for fp32).
#include "common.h"
#include "internal.h"

namespace rwkvmoe {
namespace {

constexpr double kLnEps = 1e-5;
constexpr int kLnRows = 4;

RWKV_DEV double wave_sum(double v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}

template <typename T>
__global__ __launch_bounds__(64 * kLnRows) void layer_norm_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                                 const T* __restrict__ b, T* __restrict__ y, int N,
                                                                 int C) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int MCH = 8192 / VEC / 64;  // chunks per lane at C = 8192
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kLnRows + (threadIdx.x >> 6);
  if (row >= N) return;  // the whole wave
  const int cpr = C / VEC;
  const T* xr = x + (size_t)row * C;
  Chunk<T> v[MCH];
#pragma unroll
  for (int i = 0; i < MCH; ++i) {
    const int ch = lane + 64 * i;
    if (ch < cpr) v[i].raw = *(const u32x4*)(xr + ch * VEC);
  }
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < MCH; ++i)
    if (lane + 64 * i < cpr) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) s += (double)to_f(v[i].e[j]);
    }
  const double mean = wave_sum(s) / (double)C;
  double q = 0.0;
#pragma unroll
  for (int i = 0; i < MCH; ++i)
    if (lane + 64 * i < cpr) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const double d = (double)to_f(v[i].e[j]) - mean;
        q += d * d;
      }
    }
  const double rstd = 1.0 / sqrt(wave_sum(q) / (double)C + kLnEps);
  T* yr = y + (size_t)row * C;
#pragma unroll
  for (int i = 0; i < MCH; ++i) {
    const int ch = lane + 64 * i;
    if (ch < cpr) {
      Chunk<T> wc, bc, o;
      wc.raw = *(const u32x4*)(w + ch * VEC);
      bc.raw = *(const u32x4*)(b + ch * VEC);
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const double d = ((double)to_f(v[i].e[j]) - mean) * rstd;
        o.e[j] = from_f<T>((float)(d * (double)to_f(wc.e[j]) + (double)to_f(bc.e[j])));
      }
      *(u32x4*)(yr + ch * VEC) = o.raw;
    }
  }
}

}  // namespace

hipError_t launch_layer_norm(int dtype, const void* x, const void* w, const void* b, void* y, int N, int C,
                             hipStream_t s) {
  if (N < 1 || C < 64 || C > 8192 || C % 64) return hipErrorInvalidValue;
  const dim3 grid((N + kLnRows - 1) / kLnRows);
  RWKV_DISPATCH_DTYPE(dtype, T, {
    hipLaunchKernelGGL(layer_norm_kernel<T>, grid, dim3(64 * kLnRows), 0, s, (const T*)x, (const T*)w, (const T*)b,
                       (T*)y, N, C);
  });
  return mark(hipGetLastError(), "layer_norm", s);
}

}  // namespace rwkvmoe
