// Dispatch: (token, slot) assignments → expert-major order.
//
// The reference has no dispatch: it evaluates every expert on every token and
// masks (rwkv_mlx/moe.py:139-145).  This replaces the mask with a stable
// counting sort on the expert id of each assignment a = t*k + slot:
//   offsets[e] = Σ_{e' < e} count(e')                      (exclusive scan)
//   perm[offsets[e] + rank] = a, rank = #{a' < a : expert(a') = e}
//   inv_perm[a] = position of a in perm
// Two kernels: per-block histograms (LDS counters), then a scatter in which
// every block derives its starting position per expert from the histograms
// of the blocks before it and ranks its own assignments with wavefront
// ballots, 256 assignments per round in ascending order, so the result is
// the unique stable order (bit-exact, no atomics on the output).
#include "common.h"
#include "internal.h"

namespace rwkvmoe {
namespace {

constexpr int kDispThreads = 256;
constexpr int kDispRounds = 4;
constexpr int kDispBlock = kDispThreads * kDispRounds;  // assignments per workgroup
constexpr int kMaxE = 64;

__global__ __launch_bounds__(kDispThreads) void dispatch_count_kernel(const int* __restrict__ inds, int nk, int E,
                                                                      int* block_counts) {
  __shared__ int cnt[kMaxE];
  const int tid = threadIdx.x;
  if (tid < E) cnt[tid] = 0;
  __syncthreads();
  for (int r = 0; r < kDispRounds; ++r) {
    const int a = blockIdx.x * kDispBlock + r * kDispThreads + tid;
    if (a < nk) {
      const int e = inds[a];
      if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);  // ids outside [0,E) are dropped, never indexed
    }
  }
  __syncthreads();
  if (tid < E) block_counts[(size_t)blockIdx.x * E + tid] = cnt[tid];
}

__global__ __launch_bounds__(kDispThreads) void dispatch_scatter_kernel(const int* __restrict__ inds, int nk, int E,
                                                                        int nb, const int* __restrict__ block_counts,
                                                                        int* perm, int* inv, int* offsets) {
  __shared__ int tot[kMaxE], pre[kMaxE], base[kMaxE];
  __shared__ int wcnt[kDispThreads / 64][kMaxE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid < E) {
    int t = 0, p = 0;
    for (int b = 0; b < nb; ++b) {
      const int c = block_counts[(size_t)b * E + tid];
      t += c;
      if (b < (int)blockIdx.x) p += c;
    }
    tot[tid] = t;
    pre[tid] = p;
  }
  __syncthreads();
  if (tid < E) {
    int off = 0;
    for (int e = 0; e < tid; ++e) off += tot[e];
    base[tid] = off + pre[tid];
    if (blockIdx.x == 0) {
      offsets[tid] = off;
      if (tid == E - 1) offsets[E] = off + tot[tid];
    }
  }
  const unsigned long long lt_mask = (1ull << lane) - 1ull;
  for (int r = 0; r < kDispRounds; ++r) {
    for (int i = tid; i < (kDispThreads / 64) * kMaxE; i += kDispThreads) (&wcnt[0][0])[i] = 0;
    __syncthreads();
    const int a = blockIdx.x * kDispBlock + r * kDispThreads + tid;
    int e = a < nk ? inds[a] : -1;
    if (e >= E) e = -1;
    const bool valid = e >= 0;
    unsigned long long same = 0ull;
    for (int ee = 0; ee < E; ++ee) {
      const unsigned long long m = __ballot(e == ee);
      if (e == ee) same = m;
    }
    const int rank = __popcll(same & lt_mask);
    if (valid && rank == 0) wcnt[wave][e] = __popcll(same);
    __syncthreads();
    if (valid) {
      int pos = base[e] + rank;
      for (int w = 0; w < wave; ++w) pos += wcnt[w][e];
      perm[pos] = a;
      inv[a] = pos;
    }
    __syncthreads();
    if (tid < E) {
      int s = 0;
      for (int w = 0; w < kDispThreads / 64; ++w) s += wcnt[w][tid];
      base[tid] += s;
    }
    __syncthreads();
  }
}

}  // namespace

int dispatch_blocks(int nk) { return (nk + kDispBlock - 1) / kDispBlock; }

hipError_t launch_dispatch(const int* inds, int nk, int E, int* block_counts, int* perm, int* inv, int* offsets,
                           hipStream_t s) {
  const int nb = dispatch_blocks(nk);
  if (nb == 0) return hipSuccess;
  hipLaunchKernelGGL(dispatch_count_kernel, dim3(nb), dim3(kDispThreads), 0, s, inds, nk, E, block_counts);
  const hipError_t e = mark(hipGetLastError(), "dispatch_count", s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(dispatch_scatter_kernel, dim3(nb), dim3(kDispThreads), 0, s, inds, nk, E, nb, block_counts, perm,
                     inv, offsets);
  return mark(hipGetLastError(), "dispatch_scatter", s);
}

}  // namespace rwkvmoe
