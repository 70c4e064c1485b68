// Dispatch: (token, slot) assignments → expert-major order.
//
// The reference has no dispatch: it evaluates every expert on every token and
// masks (rwkv_mlx/moe.py:139-145).  This replaces the mask with a stable
// counting sort on the expert id of each assignment a = t*k + slot:
//   offsets[e] = Σ_{e' < e} count(e')                      (exclusive scan)
//   perm[offsets[e] + rank] = a, rank = #{a' < a : expert(a') = e}
//   inv_perm[a] = position of a in perm
// Up to kDispOneMax assignments (decode batches), one workgroup does it all
// in LDS, in one launch:
//   1. each wave takes 64-assignment segments; per segment, the lanes of one
//      expert are found with one ballot per distinct expert present, giving
//      each lane its rank and the segment's count per expert;
//   2. one exclusive scan over the counts laid out expert-major
//      (count[e][segment]) gives, for every (e, segment), the number of
//      assignments that precede it in the stable order;
//   3. position = scan[e][segment] + rank.
// Larger inputs take a scatter over blocks of assignments in which every
// block sums the histograms of the blocks before it (one wave per expert,
// lanes over blocks) and ranks its own assignments with the same ballots, in
// ascending order.  The histograms are the router's per-workgroup expert
// counts when the caller has them (the router pass that wrote the ids also
// counted them: one launch), else per-block histograms of 256 assignments
// (1024 past 65536) from a launch of their own.  Either way the result is the
// unique stable order (bit-exact; the output positions never depend on
// timing).
#include "common.h"
#include "dispatch.h"
#include "internal.h"

namespace rwkvmoe {
namespace {

constexpr int kMaxE = kDispMaxE;
constexpr int kDispOneThreads = 1024;
constexpr int kDispOneMax = 2048;  // assignments of the single-workgroup path
constexpr int kDispOneSeg = kDispOneMax / 64 / (kDispOneThreads / 64);  // segments per wave, at most
// Router count entries (blocks x experts) the scatter sums per workgroup,
// at most, when it takes the router's histograms.
constexpr int kDispRouterMaxEntries = 8192;

// Rounds of 256 assignments per block of the two-launch path.
inline int disp_rounds(int nk) { return nk > 65536 ? 4 : 1; }

// Block-wide exclusive scan of one value per thread (1024 threads); *total
// receives the sum.  Uses wsum[16] in LDS.
RWKV_DEV int block_excl_scan(int v, int* wsum, int* total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int u = __shfl_up(incl, d);
    if (lane >= d) incl += u;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kDispOneThreads / 64; ++w) {
    const int s = wsum[w];
    before += w < wave ? s : 0;
    all += s;
  }
  *total = all;
  return before + incl - v;
}

__global__ __launch_bounds__(kDispOneThreads) void dispatch_one_kernel(const int* __restrict__ inds, int nk, int E,
                                                                       int* perm, int* inv, int* offsets) {
  extern __shared__ int cnt[];  // [E][S]: count of expert e in segment s, then its exclusive scan
  __shared__ int wsum[kDispOneThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int S = (nk + 63) >> 6;  // segments of 64 assignments
  for (int i = tid; i < E * S; i += kDispOneThreads) cnt[i] = 0;
  // assignment a = (wave + 16 j) * 64 + lane
  int ev[kDispOneSeg];
#pragma unroll
  for (int j = 0; j < kDispOneSeg; ++j) {
    const int a = (wave + 16 * j) * 64 + lane;
    const int e = a < nk ? inds[a] : -1;
    ev[j] = (e >= 0 && e < E) ? e : -1;  // ids outside [0,E) are dropped, never indexed
  }
  __syncthreads();  // counters zeroed
  int rk[kDispOneSeg];
#pragma unroll
  for (int j = 0; j < kDispOneSeg; ++j) {
    const int sg = wave + 16 * j;
    rk[j] = 0;
    if (sg < S) {  // wave-uniform
      int c;
      rk[j] = wave_rank(ev[j], &c);
      if (ev[j] >= 0 && rk[j] == 0) cnt[ev[j] * S + sg] = c;
    }
  }
  __syncthreads();
  // exclusive scan of cnt (expert-major); thread tid owns entries [tid*per, tid*per + per)
  const int T = E * S, per = (T + kDispOneThreads - 1) / kDispOneThreads;
  int own = 0;
  for (int i = 0; i < per; ++i) {
    const int q = tid * per + i;
    own += q < T ? cnt[q] : 0;
  }
  int total;
  int run = block_excl_scan(own, wsum, &total);
  __syncthreads();  // all counts read
  for (int i = 0; i < per; ++i) {
    const int q = tid * per + i;
    if (q < T) {
      const int c = cnt[q];
      cnt[q] = run;
      run += c;
    }
  }
  __syncthreads();
  if (tid < E) offsets[tid] = cnt[tid * S];
  if (tid == E) offsets[E] = total;
#pragma unroll
  for (int j = 0; j < kDispOneSeg; ++j) {
    const int sg = wave + 16 * j;
    const int a = sg * 64 + lane;
    if (ev[j] >= 0) {
      const int pos = cnt[ev[j] * S + sg] + rk[j];
      perm[pos] = a;
      inv[a] = pos;
    } else if (a < nk) {
      inv[a] = -1;  // dropped: not in perm
    }
  }
}

__global__ __launch_bounds__(kDispThreads) void dispatch_count_kernel(const int* __restrict__ inds, int nk, int E,
                                                                      int rounds, int* block_counts) {
  __shared__ int cnt[kMaxE];
  const int tid = threadIdx.x;
  if (tid < E) cnt[tid] = 0;
  __syncthreads();
  for (int r = 0; r < rounds; ++r) {
    const int a = (blockIdx.x * rounds + r) * kDispThreads + tid;
    if (a < nk) {
      const int e = inds[a];
      if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);  // ids outside [0,E) are dropped, never indexed
    }
  }
  __syncthreads();
  if (tid < E) block_counts[(size_t)blockIdx.x * E + tid] = cnt[tid];
}

// Workgroup w is block w of the scatter (dispatch_block, dispatch.h).
__global__ __launch_bounds__(kDispThreads) void dispatch_scatter_kernel(DispatchJob j) {
  __shared__ int scratch[kDispScratchInts];
  dispatch_block(j, blockIdx.x, scratch);
}

}  // namespace

int dispatch_blocks(int nk) {
  const int per = kDispThreads * disp_rounds(nk);
  return (nk + per - 1) / per;
}

bool dispatch_job_plan(const int* inds, int nk, int E, int* perm, int* inv, int* offsets, const int* router_cnt,
                       int router_tt, int k, int* ticket, DispatchJob* job) {
  if (nk < 1 || E > kMaxE || !router_cnt || router_tt < 1 || k < 1 || router_tt * k > kDispThreads || !ticket)
    return false;
  const int nbr = (nk / k + router_tt - 1) / router_tt;
  // (each block sums the counts of every router workgroup; at the wide
  // layer's 16384 entries the job did not beat the standalone launches)
  if ((long long)nbr * E > kDispRouterMaxEntries) return false;
  const int gpb = kDispThreads / (router_tt * k), per = gpb * router_tt * k;
  const int nw = (nbr + gpb - 1) / gpb;
  *job = DispatchJob{inds, nk, E, per, 1, nbr, gpb, router_cnt, 1, nbr, perm, inv, offsets, nw, ticket};
  return true;
}

hipError_t launch_dispatch(const int* inds, int nk, int E, int* block_counts, int* perm, int* inv, int* offsets,
                           hipStream_t s, const int* router_cnt, int router_tt, int k) {
  const int nb = dispatch_blocks(nk);
  if (nb == 0) return hipSuccess;
  if (nk <= kDispOneMax && E <= kMaxE) {
    const size_t lds = (size_t)E * ((nk + 63) / 64) * sizeof(int);  // <= 8 KB
    launch_kernel(dispatch_one_kernel, dim3(1), dim3(kDispOneThreads), lds, s, inds, nk, E, perm, inv, offsets);
    return mark(hipGetLastError(), "dispatch", s);
  }
  if (router_cnt && router_tt > 0 && k > 0 && router_tt * k <= kDispThreads) {
    // the router's per-workgroup counts ([e][block], router_tt tokens a
    // block) are the histograms: one launch, gpb router blocks a workgroup
    const int nbr = (nk / k + router_tt - 1) / router_tt;
    if ((long long)nbr * E <= kDispRouterMaxEntries) {
      const int gpb = kDispThreads / (router_tt * k), per = gpb * router_tt * k;
      const int nw = (nbr + gpb - 1) / gpb;
      const DispatchJob j{inds, nk, E, per, 1, nbr, gpb, router_cnt, 1, nbr, perm, inv, offsets, nw, nullptr};
      launch_kernel(dispatch_scatter_kernel, dim3(nw), dim3(kDispThreads), 0, s, j);
      return mark(hipGetLastError(), "dispatch_scatter", s);
    }
  }
  const int rounds = disp_rounds(nk);
  launch_kernel(dispatch_count_kernel, dim3(nb), dim3(kDispThreads), 0, s, inds, nk, E, rounds, block_counts);
  const hipError_t e = mark(hipGetLastError(), "dispatch_count", s);
  if (e != hipSuccess) return e;
  const DispatchJob j{inds, nk, E, rounds * kDispThreads, rounds, nb, 1, block_counts, E, 1, perm, inv, offsets, nb,
                      nullptr};
  launch_kernel(dispatch_scatter_kernel, dim3(nb), dim3(kDispThreads), 0, s, j);
  return mark(hipGetLastError(), "dispatch_scatter", s);
}

}  // namespace rwkvmoe
