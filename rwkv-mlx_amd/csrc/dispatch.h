// One block of the dispatch scatter as a device function, so that a kernel
// other than dispatch_scatter_kernel can run it: the SPARSE forward hands the
// scatter to the key GEMM's launch, whose workgroups take blocks by ticket
// once their tile is done (the key product does not read the dispatch, and
// the grouped LoRA after it does: the kernel boundary orders the two).
// See dispatch.hip for the algorithm (a stable counting sort on the expert
// id of each assignment a = t·k + slot).
#pragma once

#include "common.h"

namespace rwkvmoe {

constexpr int kDispThreads = 256;
constexpr int kDispMaxE = 64;

// Rank of this lane among the lanes of its wave holding the same expert e
// (e < 0: not ranked); *count (written by the lowest such lane) is their
// number.  One ballot per distinct expert present in the wave.
RWKV_DEV int wave_rank(int e, int* count) {
  const int lane = threadIdx.x & 63;
  const unsigned long long lt_mask = (1ull << lane) - 1ull;
  int rank = 0;
  *count = 0;
  unsigned long long todo = __ballot(e >= 0);
  while (todo) {
    const int e0 = __shfl(e, __builtin_ctzll(todo));
    const unsigned long long m = __ballot(e == e0);
    if (e == e0) {
      rank = __popcll(m & lt_mask);
      *count = __popcll(m);
    }
    todo &= ~m;
  }
  return rank;
}

// The scatter over histograms: block w ranks assignments
// [w·per, min(nk, (w+1)·per)) in `rounds` rounds of 256; count block b (of
// nbc) holds the assignments of the blocks' ranges in order, gpb count blocks
// per block; entry (b, e) is at counts[b·bs + e·es].  `nblk` blocks;
// `ticket` (zeroed before the launch) hands them out when the job runs
// inside another kernel.
struct DispatchJob {
  const int* inds;
  int nk, E, per, rounds, nbc, gpb;
  const int* counts;
  int bs, es;
  int* perm;
  int* inv;
  int* offsets;
  int nblk;
  int* ticket;
};

// LDS of one block (ints): tot, pre, base (kDispMaxE each), wcnt (4 x kDispMaxE)
constexpr int kDispScratchInts = 3 * kDispMaxE + (kDispThreads / 64) * kDispMaxE;

// Block `blk` of the job.  Every thread of the workgroup calls it (it holds
// barriers); threads 0..255 do the work.
RWKV_DEV void dispatch_block(const DispatchJob& j, int blk, int* scratch) {
  int* tot = scratch;
  int* pre = tot + kDispMaxE;
  int* base = pre + kDispMaxE;
  int* wcnt = base + kDispMaxE;  // [kDispThreads / 64][kDispMaxE]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const bool act = tid < kDispThreads;
  const int E = j.E;
  for (int i = tid; i < (kDispThreads / 64) * kDispMaxE; i += blockDim.x) wcnt[i] = 0;
  const int a0 = blk * j.per, lim = min(j.nk, a0 + j.per);
  // this round's expert ids, loaded before the histogram sums are awaited
  int a = a0 + tid;
  int e = act && a < lim ? j.inds[a] : -1;
  // totals and the prefix over earlier count blocks: wave w sums experts
  // w, w+4, ... (lanes over blocks, then a butterfly)
  const int first = blk * j.gpb;
  if (act) {
    for (int ee = wave; ee < E; ee += kDispThreads / 64) {
      int t = 0, q = 0;
#pragma unroll 4
      for (int b = lane; b < j.nbc; b += 64) {
        const int c = j.counts[(size_t)b * j.bs + (size_t)ee * j.es];
        t += c;
        q += b < first ? c : 0;
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        t += __shfl_xor(t, o);
        q += __shfl_xor(q, o);
      }
      if (lane == 0) {
        tot[ee] = t;
        pre[ee] = q;
      }
    }
  }
  __syncthreads();
  if (tid < E) {
    int off = 0;
    for (int q = 0; q < tid; ++q) off += tot[q];
    base[tid] = off + pre[tid];
    if (blk == 0) {
      j.offsets[tid] = off;
      if (tid == E - 1) j.offsets[E] = off + tot[tid];
    }
  }
  for (int r = 0; r < j.rounds; ++r) {
    const int o = r * kDispThreads + tid;  // offset in this block's range
    if (r > 0) {
      a = a0 + o;
      e = act && a < lim ? j.inds[a] : -1;
    }
    if (e >= E) e = -1;
    int c = 0, rank = 0;
    if (act) rank = wave_rank(e, &c);  // (whole waves: act is uniform per wave)
    if (e >= 0 && rank == 0) wcnt[wave * kDispMaxE + e] = c;
    __syncthreads();  // wcnt of this round and base are complete
    if (e >= 0) {
      int pos = base[e] + rank;
      for (int w = 0; w < wave; ++w) pos += wcnt[w * kDispMaxE + e];
      j.perm[pos] = a;
      j.inv[a] = pos;
    } else if (act && a < lim) {
      j.inv[a] = -1;  // dropped: not in perm
    }
    __syncthreads();  // every lane has read base and wcnt
    if (tid < E) {
      int s = 0;
      for (int w = 0; w < kDispThreads / 64; ++w) {
        s += wcnt[w * kDispMaxE + tid];
        wcnt[w * kDispMaxE + tid] = 0;
      }
      base[tid] += s;
    }
    __syncthreads();
  }
}

// Blocks of the job by ticket until none is left (every thread of the
// workgroup calls it; flag: one int of LDS).
RWKV_DEV void dispatch_job_run(const DispatchJob& j, int* flag, int* scratch) {
  if (j.nblk <= 0) return;
  for (;;) {
    __syncthreads();
    if (threadIdx.x == 0) flag[0] = atomicAdd(j.ticket, 1);
    __syncthreads();
    const int blk = flag[0];
    if (blk >= j.nblk) return;  // (uniform over the workgroup)
    dispatch_block(j, blk, scratch);
  }
}

}  // namespace rwkvmoe
