// The arithmetic of ln2 (model.py:321 with nn.LayerNorm(C), model.py:283;
// _layer_norm_1d, model.py:434-438), shared by layer_norm_kernel (norm.hip)
// and the router's fused form (router.hip), so both give the same bits:
//   mean = (Σ x) / C, var = (Σ (x - mean)²) / C, rstd = 1 / sqrt(var + 1e-5)
// in fp64, then mean and rstd rounded to fp32 and
//   y = ((x - mean)·rstd)·w + b
// in fp32 (four roundings, no fused multiply-add; MLX's nn.LayerNorm computes
// in fp32 too), rounded to T.  A row belongs to an aligned group of 16 lanes:
// lane j of the group takes the row's 16-byte chunks j, j + 16, ...; a
// chunk's terms are summed as a pairwise tree (elements 0+1, 2+3, ..., then
// the pairs, then the quads), and the chunk sums join the lane's running sum
// in ascending chunk order; the 16 lane sums meet in a butterfly of DPP moves
// within the row of lanes (each step adds the same two values on both lanes,
// so every lane ends with the same total).
#pragma once

#include "common.h"

namespace rwkvmoe {

constexpr double kLnEps = 1e-5;

constexpr int kLnGroup = 16;  // lanes per row

template <int CTRL>
RWKV_DEV double ln_dpp(double v) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)u, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(u >> 32), CTRL, 0xF, 0xF, false);
  return __builtin_bit_cast(double, ((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}

// the total of v over this lane's group of 16 (a DPP row), on every lane
RWKV_DEV double ln_group_sum(double v) {
  v += ln_dpp<0xB1>(v);   // quad_perm [1,0,3,2]: pairs
  v += ln_dpp<0x4E>(v);   // quad_perm [2,3,0,1]: quads
  v += ln_dpp<0x141>(v);  // row_half_mirror: halves of the row
  v += ln_dpp<0x140>(v);  // row_mirror: the row
  return v;
}

// pairwise tree over the VEC terms t[0..VEC)
template <int VEC>
RWKV_DEV double ln_tree(double (&t)[VEC]) {
#pragma unroll
  for (int w = 1; w < VEC; w <<= 1)
#pragma unroll
    for (int i = 0; i + w < VEC; i += 2 * w) t[i] += t[i + w];
  return t[0];
}

// s + the chunk's elements (their tree sum)
template <typename T>
RWKV_DEV double ln_add(double s, const Chunk<T>& c) {
  constexpr int VEC = 16 / sizeof(T);
  double t[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) t[j] = (double)to_f(c.e[j]);
  return s + ln_tree<VEC>(t);
}

// q + the chunk's (x - mean)² (their tree sum)
template <typename T>
RWKV_DEV double ln_add_sq(double q, const Chunk<T>& c, double mean) {
  constexpr int VEC = 16 / sizeof(T);
  double t[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    const double d = (double)to_f(c.e[j]) - mean;
    t[j] = d * d;
  }
  return q + ln_tree<VEC>(t);
}

RWKV_DEV double ln_rstd(double q_total, int C) { return 1.0 / sqrt(q_total / (double)C + kLnEps); }

// y for one chunk, with m = fp32(mean) and rs = fp32(rstd)
template <typename T>
RWKV_DEV Chunk<T> ln_apply(const Chunk<T>& x, const Chunk<T>& w, const Chunk<T>& b, float m, float rs) {
  Chunk<T> o;
#pragma unroll
  for (int j = 0; j < (int)(16 / sizeof(T)); ++j) {
    const float d = (to_f(x.e[j]) - m) * rs;
    o.e[j] = from_f<T>(d * to_f(w.e[j]) + to_f(b.e[j]));
  }
  return o;
}

}  // namespace rwkvmoe
