// Router: logits, top-k, gates and the load-balance / z losses
// (rwkv_mlx/moe.py:51-86), and — fused into the same pass over x — the
// token-shift mix xk of the base ChannelMix (model.py:67-75, 260-261) and,
// for adapter widths E*r <= 128, the gate-masked adapter down-projection
// U = w ⊙ (x · A_all) of the FUSED mode (moe.py:140-144).
//
// Logit definition (order fixed, implementation independent):
//   acc_q = Σ_{c in chunk q, ascending} x[t,c]·W_gate[e,c],  q = c / 64, one
//           fused multiply-add per term (fp32 for fp16/bf16 inputs, fp64 for
//           fp32 inputs: the product is exact in that format, so each step is
//           one IEEE rounding)
//   logit = fp32(Σ_{q ascending} acc_q in fp64) (+ logit_bias[e] in fp32)
// The oracle reproduces the bits.  The reference computes the same dot product
// in fp32 inside MLX (moe.py:56), in an order MLX does not specify.
//
// Workgroup = 512 threads (8 waves) over TT (<= 16) tokens:
//   1. the TT x C tile of x, the row before it and x_k (for xk) — and W_gate
//      (E x C) when it fits — go to LDS, all loads in flight together;
//      then (U) each wave puts the A_all fragments of its 16 adapter columns
//      for the first UCH K-steps in flight, so their latency overlaps
//      phases 1b-4 (issued after the tile's loads: a wave's loads complete in
//      order, so the tile does not wait behind them);
//      1b. optional: xk = x + (shift(x) - x) * x_k for the tile's rows;
//   2. the TT·E·(C/64) chunk dot products, as 2x2 (token, expert) micro-tiles
//      (2x4 for bf16); consecutive lanes take consecutive expert groups, then
//      token pairs, so a wave's LDS reads hit distinct banks;
//   3. chunks are summed per (token, expert) and rounded to fp32 (for E <= 32
//      by the lane that routes that pair in phase 4);
//   4. one thread per token: top-k (descending logit, ties to the lower id),
//      gates (softmax over the selected logits, cast to T), lse² and softmax;
//   5. optional: U[t, e*r+j] = w_e[t] · round_T((x·A_e)[t, j]) with
//      v_mfma_f32_16x16x32 (16 token rows x 16 adapter columns per wave),
//      or (opts bit 1, for the SPARSE value product) u = round_T(x·A_e)
//      for every expert, without the gates;
//      with fp32 adapters (FPK = 2: A_all as fp16 pairs, two fragments per
//      K-step) u = x·A_hi + (2^-11·x)·A_lo' in one fp32 accumulator, and
//      U = w_e·u goes out as the three fp16 blocks [U_hi | 2^-11·U_hi | U_lo]
//      the value GEMM's K-extension reads (moe.py:140-145 in fp32);
//   6. per-workgroup partial sums of p_e, counts and lse² (tokens in ascending
//      order); router_finalize_kernel reduces them in a fixed order, so the
//      losses do not depend on the order in which workgroups run.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "internal.h"
#include "ln.h"
#include "losses.h"

namespace rwkvmoe {
namespace {

constexpr int kRouterThreads = 512;
constexpr int kMaxK = 8;
constexpr int kXsBytes = 64 * 1024;  // LDS budget of the x tile
constexpr int kLdsBytes = 160 * 1024;  // W_gate is staged in LDS when the whole plan still fits this

// Widths of A_all (rows) the router's fused down-projection handles: one
// 16-column MFMA block per wave.
constexpr int kRouterKx = 16 * (kRouterThreads / 64);

template <typename T>
RWKV_DEV int xs_stride(int C) { return C + 16 / (int)sizeof(T); }  // LDS row stride (elements), 16 B padding

RWKV_DEV float fma_acc(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
RWKV_DEV double fma_acc(double a, double b, double c) { return __builtin_fma(a, b, c); }

// Workgroup barrier for data exchanged through LDS only: waits for this
// wave's LDS accesses, not for its global loads or stores (which
// __syncthreads would also drain, including the adapter prefetch).
RWKV_DEV void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Partner value of a butterfly step `off` within aligned groups of L lanes:
// off 1 and 2 swap lanes inside quads and off 4 / 8 mirror each half-row /
// row (lane i <-> 7 - i / 15 - i), all as DPP moves (no LDS round trip);
// off >= 16 uses an LDS permute.  Each step pairs every lane with a lane of
// the other half of its current sub-group, so after the steps 1, 2, 4, ...
// every lane holds the group's reduction for any commutative, associative
// combine, and a sum is bit-identical on every lane (each step adds the same
// two values, in either order).
template <int L>
RWKV_DEV int bfly(int v, int off) {
  if (off == 1) return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  if (off == 2) return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  if (off == 4) return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);  // row_half_mirror
  if (off == 8) return __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);  // row_mirror
  return __shfl_xor(v, off, L);
}
template <int L>
RWKV_DEV float bfly(float v, int off) {
  return __builtin_bit_cast(float, bfly<L>(__builtin_bit_cast(int, v), off));
}

// LDS plan shared by host and device.
struct RouterSmem {
  size_t part, xs, ws, lg, ln, total;
  bool w_in_lds;
};
// Accumulator of the chunk dot products: fp32 when x and W_gate are both
// 16-bit (their products are exact in fp32), fp64 when either is fp32.
template <typename T, typename WT>
using logit_acc_t = typename std::conditional<sizeof(T) == 2 && sizeof(WT) == 2, float, double>::type;

// `ln`: ln2's weight and bias (C elements each) after the rest, for the
// kernels that normalize their tile.
template <typename T, typename WT>
__host__ __device__ RouterSmem router_smem(int TT, int C, int E, bool w_ok, bool ln = false) {
  RouterSmem m;
  const int XS = C + 16 / (int)sizeof(T);
  const int WS = C + 16 / (int)sizeof(WT);  // W_gate rows in LDS, 16 B padding
  const size_t part = (size_t)TT * E * (C / 64) * sizeof(logit_acc_t<T, WT>);
  m.part = 0;
  m.xs = (part + 15) / 16 * 16;
  m.ws = m.xs + (size_t)(TT + 2) * XS * sizeof(T);  // tile rows, the row before the tile, x_k
  // lg, gd, prob (TT*E floats each), zt (16 floats), selected-expert masks (16
  // uint64; zt and the masks are read for 16 rows, zeros past the tile)
  const size_t tail = (size_t)TT * E * 3 * sizeof(float) + 16 * sizeof(float) + 8 + 16 * 8;
  const size_t wbytes = (size_t)E * WS * sizeof(WT);
  const size_t lnbytes = ln ? 2 * (size_t)C * sizeof(T) : 0;
  m.w_in_lds = w_ok && m.ws + wbytes + tail + 16 + lnbytes <= (size_t)kLdsBytes;
  m.lg = m.ws + (m.w_in_lds ? wbytes : 0);
  m.ln = (m.lg + tail + 15) / 16 * 16;
  m.total = ln ? m.ln + lnbytes : m.lg + tail;
  return m;
}

// Loss partials -> losses (the standalone router entry point; the forward
// runs the same reduction inside the key GEMM).
constexpr int kFinThreads = 1024;

__global__ __launch_bounds__(kFinThreads) void router_finalize_kernel(LossJob jb) {
  __shared__ double sp[kFinThreads];
  __shared__ long long sc[kFinThreads];
  __shared__ double fe[kLossMaxE + 1];
  reduce_losses(jb, sp, sc, fe);
}

// ---- decode front: key and adapter tiles in the router's launch -----------
// For a few tokens (N <= 64: a decode step of a batch of sequences), the
// products that do not need the routing run as extra workgroups of the
// router's launch, so a forward is two launches:
//   key tiles      h = relu(xk · W_keyᵀ)²        (model.py:260-262)
//   adapter tiles  u = x · A_allᵀ, rounded once  (moe.py:140, for all E·r
//                  adapter columns; the value launch applies the gates)
// Each takes one block of 16 tokens and 64 output columns (two K-steps of the
// value product): it stages the 16 input rows (xk = x + (shift(x) - x)·x_k
// rounded as model.py:260-261 does, the shift per sequence or from the
// carried state; or x itself) in LDS while each wave's weight fragments are
// in flight; wave w runs the 16x16 MFMA block of columns 16·(w % 4) over
// half of K = C (w / 4), and the two halves are added through LDS in a fixed
// order.  Weights are read in fragment order (frag_pos: a wave's load is one
// contiguous KB) where they are stored so (A_all always, W_key when laid out
// by rwkvmoe_prepare_base), else as fragments of the row-major matrix; h and
// u are written in fragment order, the layout the value launch reads.  The
// token blocks of one key column tile get workgroup ids of one residue mod
// 8 (one XCD under round-robin dispatch: its L2 serves their shared W_key
// rows; placement affects speed only).
constexpr int kDecTok = 64, kDecCols = 64, kDecCh = 12;

template <typename T>
struct DecodeKey {
  const T* wk;   // (F, C) row-major, or fragment order with wk_packed
  T* h;          // (16·nb, F) fragment order
  int F;
  const T* at;   // (kx, C) A_all, fragment order
  T* u;          // (16·nb, kx) fragment order
  int kx;
  int wk_packed;
  T* g;          // (16·nb, kx) per-column gates, fragment order (rows < N), from the router blocks
};

// Workgroups of the decode front past the router's: key tiles (XCD-grouped,
// padded to whole groups of 8 column tiles), then adapter tiles.
__host__ __device__ inline int decode_key_groups(int F) { return (F / kDecCols + 7) / 8; }
__host__ __device__ inline int decode_front_tiles(int N, int F, int kx) {
  const int nb = (N + 15) / 16;
  return decode_key_groups(F) * 8 * nb + kx / kDecCols * nb;
}

template <typename T>
RWKV_DEV void decode_key_tile(const DecodeKey<T>& dk, const T* __restrict__ x, const T* __restrict__ xprev,
                              const T* __restrict__ mu, int N, int T_, int C, unsigned char* smem, int blk) {
  using M = Mma16<T>;
  typedef typename M::frag frag;
  constexpr int VEC = 16 / sizeof(T);
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int XS = C + VEC;  // LDS row stride (elements)
  T* xs = (T*)smem;
  f32x4* red = (f32x4*)(smem + (size_t)16 * XS * sizeof(T));  // 4 x 64 partial blocks of the upper K half
  const int nb = (N + 15) / 16;
  const int nkey = decode_key_groups(dk.F) * 8 * nb;
  const bool key = blk < nkey;
  int tb, ct;
  if (key) {
    const int g = blk / (8 * nb), rem = blk % (8 * nb);
    tb = rem / 8;
    ct = g * 8 + rem % 8;
    if (ct >= dk.F / kDecCols) return;  // padding of the grouping: the whole workgroup
  } else {
    tb = (blk - nkey) % nb;
    ct = (blk - nkey) / nb;
  }
  const int f0 = ct * kDecCols;
  const int ld = key ? dk.F : dk.kx;
  T* const dst = key ? dk.h : dk.u;
  const int cb = wave & 3, kh = wave >> 2;
  const int frow = f0 + cb * 16 + (lane & 15);
  const int nkc = C / M::KS, nkh = nkc / 2, ks0 = kh * nkh;  // C % 64 == 0: whole K-steps per half
  // fragment order: block (frow / 16, k-step) at ((frow/16)·nkc + step)·512 + 8·lane
  const bool packed = !key || dk.wk_packed;
  const T* wsrc = packed ? (key ? dk.wk : dk.at) + ((size_t)(frow >> 4) * nkc * 64 + lane) * 8
                         : dk.wk + (size_t)frow * C + (lane >> 4) * M::KV;
  frag wf[kDecCh];
  auto w_load = [&](int j0) {  // steps ks0 + j0 .. of this wave's half
#pragma unroll
    for (int j = 0; j < kDecCh; ++j) {
      const int ks = ks0 + min(j0 + j, nkh - 1);
      wf[j] = *(const frag*)(wsrc + (packed ? (size_t)ks * 512 : (size_t)ks * M::KS));
    }
  };
  // the 16 input rows (zero past N), SB 16-byte chunks per thread in flight.
  // The first batch is issued before the weight fragments: a wave's loads
  // complete in order, so its math then waits for its own loads only while
  // the fragments stay in flight (later batches wait for the fragments too,
  // which the MFMAs need in any case).
  constexpr int SB = 2;
  const int cpr = C / VEC, total = 16 * cpr, nbatch = (total + SB * 512 - 1) / (SB * 512);
  // every thread runs every batch (loads at clamped indices, stores guarded),
  // so that every wave issues its fragments in the first one
  for (int bt = 0; bt < nbatch; ++bt) {
    const int i0 = tid + bt * SB * 512;
    Chunk<T> xc[SB], pc[SB], mc[SB];
    bool zp[SB];  // a sequence start without carried state: shift(x) is 0 (applied after the loads)
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      const int i = min(i0 + j * 512, total - 1);
      const int n = min(tb * 16 + i / cpr, N - 1), c = (i % cpr) * VEC, t = n % T_;
      xc[j].raw = *(const u32x4*)(x + (size_t)n * C + c);
      zp[j] = t == 0 && !xprev;
      if (key) {
        const T* prow = t > 0 ? x + (size_t)(n - 1) * C : (xprev ? xprev + (size_t)(n / T_) * C : x);
        pc[j].raw = *(const u32x4*)(prow + c);
        mc[j].raw = *(const u32x4*)(mu + c);
      }
    }
    if (bt == 0) w_load(0);
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      const int i = i0 + j * 512;
      if (i < total) {
        const int rl = i / cpr, c = (i % cpr) * VEC;
        Chunk<T> o = xc[j];
        if (key) o.raw = shift_mix_chunk<T>(xc[j].raw, zp[j] ? zero4() : pc[j].raw, mc[j].raw);
        if (tb * 16 + rl >= N) o.raw = zero4();
        *(u32x4*)(xs + (size_t)rl * XS + c) = o.raw;
      }
    }
  }
  __syncthreads();
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const T* xrow = xs + (size_t)(lane & 15) * XS + (lane >> 4) * M::KV;
  for (int j0 = 0; j0 < nkh; j0 += kDecCh) {
    if (j0 > 0) w_load(j0);
#pragma unroll
    for (int j = 0; j < kDecCh; ++j)
      if (j0 + j < nkh) acc = M::run(wf[j], *(const frag*)(xrow + (ks0 + j0 + j) * M::KS), acc);
  }
  if (kh == 1) red[cb * 64 + lane] = acc;
  __syncthreads();
  if (kh == 1) return;
  const f32x4 hi = red[cb * 64 + lane];
  acc = f32x4{acc[0] + hi[0], acc[1] + hi[1], acc[2] + hi[2], acc[3] + hi[3]};
  // lane: token tb*16 + lane%16, columns f0 + cb*16 + 4*(lane/16) + 0..3 —
  // in fragment order (K-step f0/32 + cb/2 of the value product) the 4
  // values go to lane (2·(cb & 1) + (lane/16)/2)·16 + lane%16, elements
  // 4·((lane/16) & 1) + 0..3; rows past N hold zeros
  union { T e[4]; unsigned long long u; } pk;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    float r = rnd<T>(acc[v]);
    if (key) {
      r = r > 0.f ? r : 0.f;
      r = rnd<T>(r * r);  // relu(key(k)) ** 2 (model.py:262)
    }
    pk.e[v] = from_f<T>(r);
  }
  const int g = lane >> 4, dl = (2 * (cb & 1) + (g >> 1)) * 16 + (lane & 15);
  const size_t blkp = (size_t)tb * (ld / 32) + f0 / 32 + (cb >> 1);
  *(unsigned long long*)(dst + (blkp * 64 + dl) * 8 + 4 * (g & 1)) = pk.u;
}

size_t decode_key_smem(int C, int s) { return (size_t)16 * (C + 16 / s) * s + 4 * 64 * sizeof(f32x4); }

// The decode front's router: one wave per token, 8 tokens per workgroup, no
// LDS and no barrier (a workgroup per token spent most of its time on the
// staging and barriers of the many-token plan).  Workgroups come in whole
// groups of 8, so the key tiles after them keep their XCD placement.
constexpr int kDecRouterWaves = kRouterThreads / 64;
__host__ __device__ inline int decode_router_groups(int N) {
  return ((N + kDecRouterWaves - 1) / kDecRouterWaves + 7) / 8 * 8;
}

// Token t = 8·blockIdx + wave.  The same values as the many-token kernel at
// one token per block (partials: block = token, stride nbr = N): W_gate is
// staged in LDS once per workgroup while every wave's x loads are in flight;
// the chunk dot products of (expert e, chunk q) run in lane q·EB + e of round
// (q·EB + e) / 64, each over its 64 products in ascending order from 0 in
// the accumulator format; every lane then adds the chunk sums of expert
// lane % EB in ascending q in float64, rounds once to fp32 and adds the bias.
// Routing, gates, softmax and log-sum-exp are the many-token kernel's
// butterfly code over groups of EB lanes (every group holds all EB logits,
// group 0 writes).  The gate of every adapter column goes to dk.g in u's
// fragment order.  One barrier (the W_gate staging); waves past the last
// token take part in it and then leave.
template <typename T, typename WT, int EB>
RWKV_DEV void decode_router_wave(const T* __restrict__ x, const WT* __restrict__ wg, const float* __restrict__ bias,
                                 int N, int C, int E, int k, int r, float* logits, int* inds, T* gates, T* gate_dense,
                                 double* part_f64, int* part_cnt, int nbr, const DecodeKey<T>& dk,
                                 unsigned char* smem) {
  typedef logit_acc_t<T, WT> acc_t;
  constexpr int VEC = 16 / sizeof(T), WVEC = 16 / sizeof(WT), XN = 64 / VEC, WN = 64 / WVEC;
  constexpr int L = EB, XR = 2;  // rounds whose x loads are issued before the staging wait
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = blockIdx.x * kDecRouterWaves + wave;
  const bool live = t < N;
  const int tc = min(t, N - 1);
  const int Q = C / 64;
  const int rounds = (Q * EB + 63) / 64;
  const int i = lane % EB;  // this lane's expert in the routing phase
  const int WS = C + 16 / (int)sizeof(WT);
  WT* wl = (WT*)(smem + router_smem<T, WT>(1, C, E, true).ws);
  // W_gate rows -> LDS: every thread's loads first, then this wave's x
  // chunks of the first XR rounds, then wait for the W_gate loads alone
  constexpr int WB = 4;  // W_gate 16-byte loads per thread per batch
  const int wcpr = C / WVEC, wtot = E * wcpr;
  u32x4 xv[XR][XN];
  auto x_load = [&](int rd, u32x4 (&dst)[XN]) {
    const int tau = rd * 64 + lane, q = min(tau / EB, Q - 1);
    const T* xr = x + (size_t)tc * C + q * 64;
#pragma unroll
    for (int j = 0; j < XN; ++j) dst[j] = *(const u32x4*)(xr + j * VEC);
  };
  for (int i0 = tid; i0 < wtot; i0 += WB * kRouterThreads) {
    u32x4 v[WB];
#pragma unroll
    for (int j = 0; j < WB; ++j) {
      const int ii = min(i0 + j * kRouterThreads, wtot - 1);
      v[j] = *(const u32x4*)(wg + (size_t)(ii / wcpr) * C + (ii % wcpr) * WVEC);
    }
    if (i0 == tid) {
#pragma unroll
      for (int rd = 0; rd < XR; ++rd) x_load(rd, xv[rd]);  // behind the first batch of W_gate loads
    }
#pragma unroll
    for (int j = 0; j < WB; ++j) {
      const int ii = i0 + j * kRouterThreads;
      if (ii < wtot) *(u32x4*)(wl + (size_t)(ii / wcpr) * WS + (ii % wcpr) * WVEC) = v[j];
    }
  }
  if (tid >= wtot) {  // (threads with no W_gate batch still issue their x loads)
#pragma unroll
    for (int rd = 0; rd < XR; ++rd) x_load(rd, xv[rd]);
  }
  lds_barrier();
  if (!live) return;  // the whole wave
  double s = 0.0;     // Σ_q chunk sums of expert i, ascending q
  for (int rd = 0; rd < rounds; ++rd) {
    const int tau = rd * 64 + lane, q = tau / EB, e = tau % EB;
    const bool ok = q < Q && e < E;
    const int qc = min(q, Q - 1), ec = min(e, E - 1);
    u32x4 xc[XN];
    if (rd < XR) {
#pragma unroll
      for (int j = 0; j < XN; ++j) xc[j] = rd == 0 ? xv[0][j] : xv[XR - 1][j];
    } else {
      x_load(rd, xc);
    }
    const WT* wr = wl + (size_t)ec * WS + qc * 64;
    acc_t a = 0;
#pragma unroll
    for (int j0 = 0; j0 < WN; ++j0) {
      Chunk<WT> cw;
      cw.raw = *(const u32x4*)(wr + j0 * WVEC);
#pragma unroll
      for (int jj = 0; jj < WVEC; ++jj) {
        const int j = j0 * WVEC + jj;
        Chunk<T> cx;
        cx.raw = xc[j / VEC];
        a = fma_acc((acc_t)to_f(cx.e[j % VEC]), (acc_t)to_f(cw.e[jj]), a);
      }
    }
    if (!ok) a = 0;
    // expert i's chunks of this round, ascending q
    const int q0 = rd * 64 / EB;
#pragma unroll
    for (int qq = 0; qq < 64 / EB; ++qq) {
      const double v = (double)__shfl(a, qq * EB + i, 64);
      if (q0 + qq < Q) s += v;
    }
  }
  float li = 0.f;
  if (i < E) {
    li = (float)s;
    if (bias) li = li + bias[i];
  }
  if (logits && lane < E) logits[(size_t)t * E + lane] = li;

  bool avail = i < E;
  unsigned long long taken = 0ull;
  int s_e[kMaxK];
  float s_l[kMaxK];
#pragma unroll
  for (int sl = 0; sl < kMaxK; ++sl) {
    if (sl >= k) break;
    float bv = li;
    int be = avail ? i : -1;
#pragma unroll
    for (int off = 1; off < L; off <<= 1) {
      const float ov = bfly<L>(bv, off);
      const int oe = bfly<L>(be, off);
      if (oe >= 0 && (be < 0 || ov > bv || (ov == bv && oe < be))) {
        bv = ov;
        be = oe;
      }
    }
    s_e[sl] = be;
    s_l[sl] = bv;
    taken |= 1ull << be;
    if (i == be) avail = false;
  }
  const float m = s_l[0];
  float ex[kMaxK], den = 0.f;
#pragma unroll
  for (int sl = 0; sl < kMaxK; ++sl) {
    if (sl >= k) break;
    ex[sl] = expf(s_l[sl] - m);
    den += ex[sl];
  }
  float gs = 0.f;  // this lane's dense gate
#pragma unroll
  for (int sl = 0; sl < kMaxK; ++sl) {
    if (sl >= k) break;
    const T g = from_f<T>(ex[sl] / den);
    if (i == s_e[sl]) gs = to_f(g);
    if (lane == 0) {
      if (inds) inds[(size_t)t * k + sl] = s_e[sl];
      if (gates) gates[(size_t)t * k + sl] = g;
    }
  }
  float se = i < E ? expf(li) : 0.f;
  float mx = i < E ? li : -INFINITY;
#pragma unroll
  for (int off = 1; off < L; off <<= 1) {
    se += bfly<L>(se, off);
    mx = fmaxf(mx, bfly<L>(mx, off));
  }
  float pe = i < E ? expf(li - mx) : 0.f;
  float sp = pe;
#pragma unroll
  for (int off = 1; off < L; off <<= 1) sp += bfly<L>(sp, off);
  if (lane < E) {
    if (gate_dense) gate_dense[(size_t)t * E + lane] = from_f<T>(gs);
    // loss partials of this token (block t): softmax, selection, z
    part_f64[(size_t)lane * nbr + t] = (double)(pe / sp);
    part_cnt[(size_t)lane * nbr + t] = (int)((taken >> lane) & 1ull);
  }
  if (lane == 0) {
    const float lse = logf(se);
    part_f64[(size_t)E * nbr + t] = (double)(lse * lse);
  }
  // the gate of every adapter column e·r + j (0 for padding columns), in u's
  // fragment order
  const int kx = dk.kx, nku = kx / 32;
  for (int col = lane; col < kx; col += 64) {
    const int e = col / r;
    const float g = __shfl(gs, min(e, EB - 1), 64);
    dk.g[(((size_t)(t >> 4) * nku + (col >> 5)) * 64 + ((col & 31) >> 3) * 16 + (t & 15)) * 8 + (col & 7)] =
        from_f<T>(col < E * r ? g : 0.f);
  }
}

// ln2 fused into the router's tile pass: the rows are normalized in LDS
// (ln.h's arithmetic, the same bits as layer_norm_kernel) and, with xn, also
// written out for the kernels that read x after the router.
template <typename T>
struct RouterLn {
  const T* w;  // (C) ln2.weight
  const T* b;  // (C) ln2.bias
  T* xn;       // (N, C) LN(x), or null
};

// T: x and the outputs; WT: W_gate as stored (T, or fp32); FPK: adapter
// fragments per K-step (2: fp32 adapters as fp16 pairs, T = f16 only); KT:
// the decode front (decode_router_groups(N) workgroups of the wave-per-token
// router, then the decode key and adapter tiles); LN: x is the residual
// stream and the tile's rows are LN(x) (not with KT).
template <typename T, typename WT, int EB, bool WU, int FPK, bool KT, bool LN = false>
__global__ __launch_bounds__(kRouterThreads) __attribute__((amdgpu_waves_per_eu(KT ? 4 : (std::is_same<T, f16>::value && std::is_same<WT, f16>::value && !WU && EB <= 32 ? 8 : 1)))) void router_kernel(
    const T* __restrict__ x, const WT* __restrict__ wg, const float* __restrict__ bias, const T* __restrict__ xprev,
    const T* __restrict__ mu, const T* __restrict__ at, int N, int T_, int C, int E, int k, int r, int TT,
    float* logits, int* inds, T* gates, T* gate_dense, T* xk, T* u_arg, double* part_f64, int* part_cnt,
    int* loss_claim, int opts, int nbr, DecodeKey<T> dk, RouterLn<T> ln) {
  static_assert(!(KT && LN), "the decode front reads LN(x) written by layer_norm_kernel");
  static_assert(FPK == 1 || (FPK == 2 && std::is_same<T, f16>::value), "fp16 pairs need an fp16 layer");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  // the argument lines at offsets 0x00 (x), 0x40 (k), 0x80 (part_f64), 0xc0 (dk.kx)
  RWKV_KERNARG_LINES("s"(x), "s"(k), "s"(part_f64), "s"(dk.kx));
  if constexpr (KT) {
    const int nrw = decode_router_groups(N);
    if ((int)blockIdx.x >= nrw) {
      decode_key_tile(dk, x, xprev, mu, N, T_, C, smem, (int)blockIdx.x - nrw);
      return;
    }
    // the loss reduction of this forward is claimed by the value launch
    if (loss_claim && blockIdx.x == 0 && threadIdx.x == 0) *loss_claim = 0;
    decode_router_wave<T, WT, EB>(x, wg, bias, N, C, E, k, r, logits, inds, gates, gate_dense, part_f64, part_cnt,
                                  nbr, dk, smem);
    return;
  }
  constexpr int VEC = 16 / sizeof(T);
  constexpr bool WSAME = std::is_same<T, WT>::value;
  // opts bit 0: W_gate staged in LDS; bit 1: U without the gates (u)
  const RouterSmem sm = router_smem<T, WT>(TT, C, E, (opts & 1) != 0, LN);
  T* const u = WU ? u_arg : nullptr;  // the instance without U drops its registers
  const int Q = C / 64, XS = xs_stride<T>(C), WS = C + 16 / (int)sizeof(WT);
  typedef logit_acc_t<T, WT> acc_t;
  acc_t* part = (acc_t*)smem;                      // TT*E*Q chunk dot products
  T* xs = (T*)(smem + sm.xs);                      // TT*XS
  float* lg = (float*)(smem + sm.lg);              // TT*E logits
  float* gd = lg + TT * E;                         // TT*E dense gates (0 where not routed)
  float* prob = gd + TT * E;                       // TT*E softmax (0 past the last token)
  float* zt = prob + TT * E;                       // 16 (0 past the last token)
  unsigned long long* selm = (unsigned long long*)(((size_t)(zt + 16) + 7) & ~(size_t)7);  // 16 masks

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t0 = blockIdx.x * TT;
  // the loss reduction of this forward is claimed later by the first key GEMM
  // workgroup to finish (kernels on one stream run in order)
  // (and the dispatch ticket beside it, claim[1], for a dispatch job in the
  // key GEMM's launch)
  if (loss_claim && blockIdx.x == 0 && tid == 0) {
    loss_claim[0] = 0;
    loss_claim[1] = 0;
  }
  const int nt = min(TT, N - t0);

  // adapter down-projection operands: this wave's 16 columns of A_all
  using UM = Mma16<T>;
  typedef typename UM::frag ufrag;
  constexpr int UCH = EB <= 32 ? 24 : 12;  // A_all fragments in flight together
  constexpr int UKS = UCH / FPK;           // the K-steps they cover
  ufrag ufb[UCH];
  f32x4 uacc = {0.f, 0.f, 0.f, 0.f};
  const int un = wave * 16 + (lane & 15);  // this lane's adapter column
  // A_all is in fragment order: this wave's fragment for K-step kk / 32 (pass
  // p) is the 1 KB at (((wave·C/32 + kk/32)·FPK + p)·64 + lane)·8
  const T* ufr = WU ? at + ((size_t)wave * (C / UM::KS) * FPK * 64 + lane) * UM::KV : nullptr;
  // fragments [j0, j1) of the chunk starting at k0: fragment j is pass j % FPK
  // of K-step k0/32 + j/FPK (clamped; steps past C are skipped)
  auto u_load = [&](int k0, int j0, int j1) {
#pragma unroll
    for (int j = 0; j < UCH; ++j)
      if (j >= j0 && j < j1) {
        const int kk = min(k0 + (j / FPK) * UM::KS, C - UM::KS);
        ufb[j] = *(const ufrag*)(ufr + ((size_t)(kk / UM::KS) * FPK + j % FPK) * 64 * UM::KV);
      }
  };
  // the first chunk goes out in four batches, one ahead of each of phases
  // 1b-4: a wave stalls issuing loads once its CU's misses in flight are at
  // their limit, and a whole chunk at once would hold every wave at the next
  // barrier
  constexpr int UB = UCH / 4;

  // 1. x tile, the row before it and x_k (both for xk), and W_gate -> LDS,
  //    up to LB 16-byte loads per thread in flight before any is stored.
  //    The LDS rows are consecutive (tile rows, prev, x_k, then W_gate), so
  //    a thread walks (row, chunk) coordinates with one division up front.
  const int cpr = C / VEC;
  T* prow = xs + (size_t)TT * XS;  // shift(x) of the tile's first token
  T* mrow = prow + XS;             // x_k
  const int dq = kRouterThreads / cpr, dr = kRouterThreads % cpr;  // the walker's stride in rows, chunks
  // ln2's weight and bias (2·cpr chunks): a thread's first chunk goes out
  // ahead of the tile's loads (they complete in order, so it is in by the
  // time the tile is) and lands in LDS after the plan's other regions
  T* const lnl = (T*)(smem + sm.ln);
  u32x4 lnv = zero4();
  if constexpr (LN) {
    const int i0 = min(tid, 2 * cpr - 1);  // (an unconditional load: no branch around it)
    lnv = *(const u32x4*)(i0 < cpr ? ln.w + i0 * VEC : ln.b + (i0 - cpr) * VEC);
  }
  {
    const int nrows = TT + 2 + (WSAME && sm.w_in_lds ? E : 0);
    // the row before the tile: x[t0-1] inside a sequence, else the carried
    // state or 0; x itself stands in for rows that read as zero
    const bool ok_prev = xk && (t0 % T_ != 0 || xprev), ok_mu = xk != nullptr;
    const T* prev_src = t0 % T_ != 0 ? x + (size_t)(t0 - 1) * C : (xprev ? xprev + (size_t)(t0 / T_) * C : x);
    const T* mu_src = mu ? mu : x;
    constexpr int LB = 8;
    int R = tid / cpr, cc = tid % cpr;
    for (int b0 = 0; b0 < nrows * cpr; b0 += LB * kRouterThreads) {
      u32x4 v[LB];
      int rr[LB], cs[LB];
#pragma unroll
      for (int j = 0; j < LB; ++j) {
        // source row chosen by selects, then one unconditional load: loads in
        // divergent branches would each wait for the one before
        const int c = cc * VEC;
        const T* xrow = x + (size_t)(t0 + min(R, nt - 1)) * C;
        const T* wrow = (const T*)wg + (size_t)min(max(R - TT - 2, 0), E - 1) * C;  // (WSAME only)
        const T* src = R < TT ? xrow : (R == TT ? prev_src : (R == TT + 1 ? mu_src : wrow));
        const bool ok = R < TT ? R < nt : (R == TT ? ok_prev : (R == TT + 1 ? ok_mu : R < nrows));
        const u32x4 w = *(const u32x4*)(src + c);
        v[j] = ok ? w : zero4();
        rr[j] = R;
        cs[j] = c;
        cc += dr;
        R += dq;
        if (cc >= cpr) {
          cc -= cpr;
          ++R;
        }
      }
#pragma unroll
      for (int j = 0; j < LB; ++j)
        if (rr[j] < nrows) *(u32x4*)(xs + (size_t)rr[j] * XS + cs[j]) = v[j];
    }
  }
  // an fp32 W_gate beside a 16-bit x: its rows go to LDS in a loop of their
  // own (row stride WS), four 16-byte loads per thread in flight
  if constexpr (!WSAME) {
    if (sm.w_in_lds) {
      constexpr int WV = 16 / sizeof(WT), LB = 4;
      const int wcpr = C / WV, total = E * wcpr;
      WT* wl = (WT*)(smem + sm.ws);
      for (int i0 = tid; i0 < total; i0 += LB * kRouterThreads) {
        u32x4 v[LB];
#pragma unroll
        for (int j = 0; j < LB; ++j) {
          const int i = min(i0 + j * kRouterThreads, total - 1);
          v[j] = *(const u32x4*)(wg + (size_t)(i / wcpr) * C + (i % wcpr) * WV);
        }
#pragma unroll
        for (int j = 0; j < LB; ++j) {
          const int i = i0 + j * kRouterThreads;
          if (i < total) *(u32x4*)(wl + (size_t)(i / wcpr) * WS + (i % wcpr) * WV) = v[j];
        }
      }
    }
  }
  if constexpr (LN) {
    if (tid < 2 * cpr) *(u32x4*)(lnl + (size_t)tid * VEC) = lnv;
    for (int i = tid + kRouterThreads; i < 2 * cpr; i += kRouterThreads)  // rows of more than 256 chunks
      *(u32x4*)(lnl + (size_t)i * VEC) = *(const u32x4*)(i < cpr ? ln.w + i * VEC : ln.b + (i - cpr) * VEC);
  }
  asm volatile("" ::: "memory");  // the tile's loads and LDS stores stay ahead of the prefetch
  if (u) u_load(0, 0, UB);
  lds_barrier();
  if constexpr (LN) {
    // the tile's rows, and the row before the tile when it is x[t0 - 1]
    // (a carried state is already ln2's output): a group of 16 lanes per row
    const int nln = nt + (xk && t0 % T_ != 0 ? 1 : 0);
    const int j = lane % kLnGroup;
    for (int i = tid / kLnGroup; i < nln; i += kRouterThreads / kLnGroup) {  // whole groups
      T* rp = xs + (size_t)(i < nt ? i : TT) * XS;
      double sm = 0.0;
#pragma unroll 4
      for (int ch = j; ch < cpr; ch += kLnGroup) {
        Chunk<T> c;
        c.raw = *(const u32x4*)(rp + ch * VEC);
        sm = ln_add(sm, c);
      }
      const double mean = ln_group_sum(sm) / (double)C;
      double q = 0.0;
#pragma unroll 4
      for (int ch = j; ch < cpr; ch += kLnGroup) {
        Chunk<T> c;
        c.raw = *(const u32x4*)(rp + ch * VEC);
        q = ln_add_sq(q, c, mean);
      }
      const double rstd = ln_rstd(ln_group_sum(q), C);
      T* xo = ln.xn && i < nt ? ln.xn + (size_t)(t0 + i) * C : nullptr;
#pragma unroll 2
      for (int ch = j; ch < cpr; ch += kLnGroup) {
        Chunk<T> c, wc, bc;
        c.raw = *(const u32x4*)(rp + ch * VEC);
        wc.raw = *(const u32x4*)(lnl + (size_t)ch * VEC);
        bc.raw = *(const u32x4*)(lnl + (size_t)(cpr + ch) * VEC);
        const Chunk<T> o = ln_apply(c, wc, bc, (float)mean, (float)rstd);
        *(u32x4*)(rp + ch * VEC) = o.raw;
        if (xo) *(u32x4*)(xo + ch * VEC) = o.raw;
      }
    }
    lds_barrier();
  }

  if (u) u_load(0, UB, 2 * UB);
  // 1b. optional: the token-shift mix of the base ChannelMix for these rows,
  //     xk = x + (shift(x) - x) * x_k, each op rounded to T (model.py:260-261).
  //     When no sequence starts inside the tile (tl > 0) every operand is in
  //     LDS; otherwise those rows read the carried state from global memory,
  //     in a separate loop, so the common case never waits for a load (a wait
  //     for one would also wait for the adapter prefetch issued before it).
  if (xk) {
    auto mix = [&](int tl, int c, const Chunk<T>& pc) {
      const u32x4 xv = *(const u32x4*)(xs + (size_t)tl * XS + c);
      const u32x4 mv = *(const u32x4*)(mrow + c);
      *(u32x4*)(xk + (size_t)(t0 + tl) * C + c) = shift_mix_chunk<T>(xv, pc.raw, mv);
    };
    const bool inner_start = (t0 % T_) + nt > T_;  // some t0 < t < t0 + nt has t % T_ == 0
    if (!inner_start) {
      for (int tl = tid / cpr, cc = tid % cpr; tl < nt;) {
        const int c = cc * VEC;
        Chunk<T> pc;
        pc.raw = *(const u32x4*)((tl == 0 ? prow : xs + (size_t)(tl - 1) * XS) + c);
        mix(tl, c, pc);
        cc += dr;
        tl += dq;
        if (cc >= cpr) {
          cc -= cpr;
          ++tl;
        }
      }
    } else {
      for (int i = tid; i < nt * cpr; i += kRouterThreads) {
        const int tl = i / cpr, c = (i % cpr) * VEC;
        const int t = t0 + tl;
        Chunk<T> pc;
        if (tl == 0)
          pc.raw = *(const u32x4*)(prow + c);
        else if (t % T_ != 0)
          pc.raw = *(const u32x4*)(xs + (size_t)(tl - 1) * XS + c);
        else  // a sequence starts inside the tile
          pc.raw = xprev ? *(const u32x4*)(xprev + (size_t)(t / T_) * C + c) : zero4();
        mix(tl, c, pc);
      }
    }
  }

  if (u) u_load(0, 2 * UB, 3 * UB);
  // 2. chunk dot products.  A task is a 2x2 (2x4 for bf16) (token, expert)
  //    micro-tile of one chunk: each accumulator still runs over its chunk in
  //    ascending c, and every conversion feeds two (four) FMAs.  W_gate rows come from LDS or, when
  //    they did not fit, from global memory: two instances, so that the LDS
  //    one is compiled with LDS reads only (generic-pointer reads would also
  //    wait for the adapter prefetch).
  // VEC elements of W_gate (T or fp32) as accumulator values
  auto w_vec = [&](const WT* p, acc_t (&o)[VEC]) {
    union {
      u32x4 raw[VEC * sizeof(WT) / 16];
      WT e[VEC];
    } w;
#pragma unroll
    for (int i = 0; i < (int)(VEC * sizeof(WT) / 16); ++i) w.raw[i] = *(const u32x4*)(p + i * (16 / sizeof(WT)));
#pragma unroll
    for (int i = 0; i < VEC; ++i) o[i] = (acc_t)to_f(w.e[i]);
  };
  auto chunk_dots = [&](const WT* wsrc, int wstr) {
    // RT x RE (token, expert) micro-tiles: 2x4 for bf16, whose operands take
    // a conversion each (3 conversions per 8 FMAs instead of 4 per 4), else
    // 2x2 (4x4 left half the threads without a task at 8 tokens x 16
    // experts and measured slower)
    constexpr int RT = 2, RE = std::is_same<T, bf16>::value ? 4 : 2;
    const int TTn = (TT + RT - 1) / RT, En = (E + RE - 1) / RE;
    const int ntask = TTn * En * Q;
    for (int task = tid; task < ntask; task += kRouterThreads) {
      const int ep = task % En, tp = (task / En) % TTn, q = task / (En * TTn);
      int tr[RT], er[RE];
#pragma unroll
      for (int r = 0; r < RT; ++r) tr[r] = min(RT * tp + r, TT - 1);
#pragma unroll
      for (int c = 0; c < RE; ++c) er[c] = min(RE * ep + c, E - 1);
      const T* xr[RT];
      const WT* wr[RE];
#pragma unroll
      for (int r = 0; r < RT; ++r) xr[r] = xs + (size_t)tr[r] * XS + q * 64;
#pragma unroll
      for (int c = 0; c < RE; ++c) wr[c] = wsrc + (size_t)er[c] * wstr + q * 64;
      acc_t a[RT][RE];
#pragma unroll
      for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int c = 0; c < RE; ++c) a[r][c] = 0;
      // The chains advance together, one term each per step (a scheduling
      // barrier after every step keeps them interleaved: left to itself the
      // scheduler ran some of them as lone dependent chains), and the next
      // VEC-wide block's operands are read from LDS one block ahead.
      Chunk<T> cx[RT];
      acc_t cw[RE][VEC];
#pragma unroll
      for (int r = 0; r < RT; ++r) cx[r].raw = *(const u32x4*)xr[r];
#pragma unroll
      for (int c = 0; c < RE; ++c) w_vec(wr[c], cw[c]);
#pragma unroll
      for (int j = 0; j < 64; j += VEC) {
        Chunk<T> nx[RT];
        acc_t nw[RE][VEC];
        if (j + VEC < 64) {
#pragma unroll
          for (int r = 0; r < RT; ++r) nx[r].raw = *(const u32x4*)(xr[r] + j + VEC);
#pragma unroll
          for (int c = 0; c < RE; ++c) w_vec(wr[c] + j + VEC, nw[c]);
        }
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          acc_t fx[RT];
#pragma unroll
          for (int r = 0; r < RT; ++r) fx[r] = (acc_t)to_f(cx[r].e[i]);
#pragma unroll
          for (int r = 0; r < RT; ++r)
#pragma unroll
            for (int c = 0; c < RE; ++c) a[r][c] = fma_acc(fx[r], cw[c][i], a[r][c]);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (j + VEC < 64) {
#pragma unroll
          for (int r = 0; r < RT; ++r) cx[r] = nx[r];
#pragma unroll
          for (int c = 0; c < RE; ++c)
#pragma unroll
            for (int i = 0; i < VEC; ++i) cw[c][i] = nw[c][i];
        }
      }
      // duplicate lanes (TT or E not a multiple of RT) write the same value
      // to the same slot
#pragma unroll
      for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int c = 0; c < RE; ++c) part[((size_t)tr[r] * E + er[c]) * Q + q] = a[r][c];
    }
  };
  // W_gate in global memory, fp16: a task is one expert's chunk for 8 tokens,
  // so every W_gate element is read once per tile (through a two-deep
  // register pipeline), and the lanes of a wave that share a chunk read the
  // same x addresses from LDS.  (fp16 operands convert inside the mixed FMA;
  // bf16 and fp32 ones take a conversion each, which the micro-tiles share
  // between two or four FMAs.)
  auto chunk_cols = [&]() {
    constexpr int MT = 8, NJ = 64 / VEC;
    const int ntask = (TT + MT - 1) / MT * E * Q;
    for (int task = tid; task < ntask; task += kRouterThreads) {
      const int e = task % E, q = (task / E) % Q, tb = task / (E * Q);
      const T* wr = (const T*)wg + (size_t)e * C + q * 64;  // (WSAME only)
      const T* xr = xs + q * 64;
      acc_t a[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) a[m] = 0;
      Chunk<T> cw, nw;
      cw.raw = *(const u32x4*)wr;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        if (j + 1 < NJ) nw.raw = *(const u32x4*)(wr + (j + 1) * VEC);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          Chunk<T> cx;
          cx.raw = *(const u32x4*)(xr + (size_t)min(tb * MT + m, TT - 1) * XS + j * VEC);
#pragma unroll
          for (int i = 0; i < VEC; ++i) a[m] = fma_acc((acc_t)to_f(cx.e[i]), (acc_t)to_f(cw.e[i]), a[m]);
        }
        cw = nw;
      }
      // rows past the tile repeat its last row: same value, same slot
#pragma unroll
      for (int m = 0; m < MT; ++m) part[((size_t)min(tb * MT + m, TT - 1) * E + e) * Q + q] = a[m];
    }
  };
  if (sm.w_in_lds) chunk_dots((const WT*)(smem + sm.ws), WS);
  else if constexpr (std::is_same<T, f16>::value && WSAME && !WU && !KT) chunk_cols();  // (the decode front stages W_gate)
  else chunk_dots(wg, C);
  lds_barrier();

  // 3. chunk sums in ascending order, one rounding to fp32 (+ bias).  With
  //    E <= 32 the lane that routes (token, expert) in phase 4 computes it
  //    there; otherwise here, into lg.
  auto logit_of = [&](int tl, int e) -> float {
    const acc_t* pp = part + (size_t)(tl * E + e) * Q;
    double s = 0.0;
    for (int q0 = 0; q0 < Q; q0 += 4) {  // loads of 4 chunks in flight, added in ascending q
      double v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = (double)pp[min(q0 + i, Q - 1)];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (q0 + i < Q) s += v[i];
    }
    float l = (float)s;
    if (bias) l = l + bias[e];
    if (logits && tl < nt) logits[(size_t)(t0 + tl) * E + e] = l;
    return l;
  };
  if constexpr (EB > 32) {
    for (int pr = tid; pr < TT * E; pr += kRouterThreads) lg[pr] = logit_of(pr / E, pr % E);
    lds_barrier();
  }

  if (u) u_load(0, 3 * UB, UCH);
  // 4. routing per token.  E <= 32: a group of EB lanes per token, lane i
  //    holding expert i: top-k in k butterfly arg-max passes over (logit
  //    descending, id ascending), so ties go to the lower id; gates in slot
  //    order; log-sum-exp and softmax from butterfly max / sums (every lane of
  //    a group ends with the same bits: each step adds a pair in either order).
  //    E > 32: one thread per token with its E logits in registers.
  if (tid >= TT && tid < 16) {  // rows past the tile: nothing routed
    zt[tid] = 0.f;
    selm[tid] = 0ull;
  }
  if constexpr (EB <= 32) {
    constexpr int L = EB;
    const int tl = tid / L, i = tid % L;
    if (tl < TT) {
      const int t = t0 + tl;
      const bool live = tl < nt;
      const float li = i < E ? logit_of(tl, i) : 0.f;
      bool avail = i < E;
      unsigned long long taken = 0ull;
      int s_e[kMaxK];
      float s_l[kMaxK];
#pragma unroll
      for (int s = 0; s < kMaxK; ++s) {
        if (s >= k) break;
        float bv = li;
        int be = avail ? i : -1;
#pragma unroll
        for (int off = 1; off < L; off <<= 1) {
          const float ov = bfly<L>(bv, off);
          const int oe = bfly<L>(be, off);
          if (oe >= 0 && (be < 0 || ov > bv || (ov == bv && oe < be))) {
            bv = ov;
            be = oe;
          }
        }
        s_e[s] = be;
        s_l[s] = bv;
        taken |= 1ull << be;
        if (i == be) avail = false;
      }
      const float m = s_l[0];
      float ex[kMaxK], den = 0.f;
#pragma unroll
      for (int s = 0; s < kMaxK; ++s) {
        if (s >= k) break;
        ex[s] = expf(s_l[s] - m);
        den += ex[s];
      }
      float gs = 0.f;  // this lane's dense gate
#pragma unroll
      for (int s = 0; s < kMaxK; ++s) {
        if (s >= k) break;
        const T g = from_f<T>(ex[s] / den);
        if (i == s_e[s]) gs = to_f(g);
        if (i == 0 && live) {
          if (inds) inds[(size_t)t * k + s] = s_e[s];
          if (gates) gates[(size_t)t * k + s] = g;
        }
      }
      float se = i < E ? expf(li) : 0.f;
      float mx = i < E ? li : -INFINITY;
#pragma unroll
      for (int off = 1; off < L; off <<= 1) {
        se += bfly<L>(se, off);
        mx = fmaxf(mx, bfly<L>(mx, off));
      }
      float pe = i < E ? expf(li - mx) : 0.f;
      float sp = pe;
#pragma unroll
      for (int off = 1; off < L; off <<= 1) sp += bfly<L>(sp, off);
      if (i < E) {
        prob[tl * E + i] = live ? pe / sp : 0.f;
        gd[tl * E + i] = live ? gs : 0.f;
        if (gate_dense && live) gate_dense[(size_t)t * E + i] = from_f<T>(gs);
      }
      if (i == 0) {
        const float lse = logf(se);
        zt[tl] = live ? lse * lse : 0.f;
        selm[tl] = live ? taken : 0ull;
      }
    }
  } else {
    if (tid < TT) {
      const int t = t0 + tid;
      float l[EB];
  #pragma unroll
      for (int e = 0; e < EB; ++e) l[e] = e < E ? lg[tid * E + e] : 0.f;
      selm[tid] = 0ull;
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
        }
        selm[tid] = taken;
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
  }
  lds_barrier();

  // 4b. decode front: the gate of every adapter column (e·r + j -> the gate
  //     of expert e, 0 for padding columns) in u's fragment order, which the
  //     decode value launch multiplies into u as it reads both
  if constexpr (KT) {
    const int kx = dk.kx, nku = kx / 32;
    for (int i = tid; i < nt * kx; i += kRouterThreads) {
      const int tl = i / kx, col = i % kx, t = t0 + tl;
      const float g = col < E * r ? gd[tl * E + col / r] : 0.f;
      dk.g[(((size_t)(t >> 4) * nku + (col >> 5)) * 64 + ((col & 31) >> 3) * 16 + (t & 15)) * 8 + (col & 7)] =
          from_f<T>(g);
    }
  }

  // 5. fused adapter down-projection: finish the MFMAs on the prefetched
  //    chunk, then stream the remaining chunks
  if (u) {
    const int lr = lane & 15, kh = lane >> 4;
    const T* arow = xs + (size_t)lr * XS + kh * UM::KV;  // rows past the last token are zero in LDS
    // one K-step: x·A_all, and with fp16 pairs also (2^-11·x)·A_lo' (the
    // scaled x is exact wherever it stays a normal fp16)
    auto ustep = [&](const ufrag& xf, int j) {
      uacc = UM::run(xf, ufb[j * FPK], uacc);
      if constexpr (FPK == 2) uacc = UM::run(xf * (T)kLoUnscale, ufb[j * FPK + 1], uacc);
    };
    for (int k0 = 0; k0 < C; k0 += UKS * UM::KS) {
      if (k0 > 0) u_load(k0, 0, UCH);
      if (k0 + UKS * UM::KS <= C) {
        // whole chunk: the x fragments of 8 K-steps are read ahead of their MFMAs
#pragma unroll
        for (int j0 = 0; j0 < UKS; j0 += 8) {
          ufrag fa[8];
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (j0 + j < UKS) fa[j] = *(const ufrag*)(arow + k0 + (j0 + j) * UM::KS);
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (j0 + j < UKS) ustep(fa[j], j0 + j);
        }
      } else {
#pragma unroll
        for (int j = 0; j < UKS; ++j) {
          const int kk = k0 + j * UM::KS;
          if (kk < C) ustep(*(const ufrag*)(arow + kk), j);
        }
      }
    }
    const int e = un / r;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = kh * 4 + v;  // token within the tile
      if (row < nt) {
        const float g = (un < E * r) ? ((opts & 2) ? 1.f : gd[row * E + e]) : 0.f;
        if constexpr (FPK == 2) {
          // U = w_e·u in fp32, then [U_hi | 2^-11·U_hi | U_lo] (row stride 3·128)
          const float uf = g * uacc[v];
          const T hi = (T)uf;
          T* ur = u + (size_t)(t0 + row) * 3 * kRouterKx;
          ur[un] = hi;
          ur[kRouterKx + un] = (T)((float)hi * kLoUnscale);
          ur[2 * kRouterKx + un] = (T)(uf - (float)hi);
        } else {
          u[(size_t)(t0 + row) * kRouterKx + un] = from_f<T>(g * rnd<T>(uacc[v]));
        }
      }
    }
  }

  // 6. per-workgroup partials, tokens in ascending order (rows past the last
  //    token hold zeros)
  if (tid < E) {
    float pv[16];
    unsigned long long mv[16];
#pragma unroll
    for (int tl = 0; tl < 16; ++tl) {
      pv[tl] = prob[min(tl, TT - 1) * E + tid];
      mv[tl] = selm[tl];
    }
    double ps = 0.0;
    int cnt = 0;
#pragma unroll
    for (int tl = 0; tl < 16; ++tl) {
      if (tl < TT) ps += (double)pv[tl];
      cnt += (int)((mv[tl] >> tid) & 1ull);
    }
    part_f64[(size_t)tid * nbr + blockIdx.x] = ps;  // value-major: the finalize reads blocks in a row
    part_cnt[(size_t)tid * nbr + blockIdx.x] = cnt;
  } else if (tid == E) {
    float zv[16];
#pragma unroll
    for (int tl = 0; tl < 16; ++tl) zv[tl] = zt[tl];
    double zs = 0.0;
#pragma unroll
    for (int tl = 0; tl < 16; ++tl) zs += (double)zv[tl];
    part_f64[(size_t)E * nbr + blockIdx.x] = zs;
  }
}


}  // namespace

// W_gate goes to LDS unless that costs resident workgroups per CU that the
// grid would use: the instance without the adapter MFMAs needs few enough
// registers that LDS alone bounds its occupancy, and at the shapes with many
// 8-token tiles the overlapping load / FMA / routing phases of several
// workgroups are worth more than reading W_gate from LDS instead of L2.
template <typename T, typename WT>
int router_w_in_lds_ok(int nb, int TT, int C, int E, bool with_u, bool ln) {
  if (with_u) return 1;  // the adapter instance's registers allow one workgroup per CU
  const int cus = num_cus(), want = (nb + cus - 1) / cus;
  auto occ = [&](bool w) {
    const int o = kLdsBytes / (int)router_smem<T, WT>(TT, C, E, w, ln).total;
    return o < want ? o : want;
  };
  return occ(true) >= occ(false);
}

int router_tile_tokens(int N, int C, int E, int dtype) {
  const int s = dtype == 0 ? 4 : 2;
  const int per_token = E * (C / 64);
  int tt = 4096 / (per_token > 0 ? per_token : 1);
  if (tt > 16) tt = 16;
  const int by_lds = kXsBytes / ((C + 16 / s) * s) - 2;  // two more rows: shift(x) of the first token, x_k
  if (tt > by_lds) tt = by_lds;
  // small batches (decode steps): fewer tokens per workgroup, so that up to
  // 64 workgroups share them; each one's chain is mostly memory latency
  const int spread = (N + 63) / 64;
  if (N > 0 && tt > spread) tt = spread;
  if (tt < 1) tt = 1;
  return tt;
}

hipError_t launch_router(int dtype, bool gate32, int fpk, const void* x, const void* wg, const float* bias,
                         const void* xprev, const void* mu, const void* at, int N, int T_, int C, int E, int k, int r,
                         float* logits, int* inds, void* gates, void* gate_dense, void* xk, void* u, double* part_f64,
                         int* part_cnt, int* loss_claim, int TT, hipStream_t s, const DecodeFront* front,
                         const void* ln_w, const void* ln_b, void* xn, bool u_raw) {
  if (TT < 1 || TT > 16) return hipErrorInvalidValue;
  if (u_raw && (!u || fpk != 1)) return hipErrorInvalidValue;
  const int nb = (N + TT - 1) / TT;
  if (u && (TT != 16 || E * r > kRouterKx)) return hipErrorInvalidValue;
  if (fpk != 1 && (fpk != 2 || dtype != 1 || !u)) return hipErrorInvalidValue;
  if (front && (dtype == 0 || u || TT != 1 || N > kDecTok || front->F % kDecCols || front->kx % kDecCols || C % 64 ||
                E > 16))
    return hipErrorInvalidValue;
  if ((ln_w != nullptr) != (ln_b != nullptr) || (front && ln_w) || (xn && !ln_w)) return hipErrorInvalidValue;
  auto go = [&](auto tag_t, auto tag_w) -> hipError_t {
    typedef decltype(tag_t) T;
    typedef decltype(tag_w) WT;
    const int w_ok = front ? 1 : router_w_in_lds_ok<T, WT>(nb, TT, C, E, u != nullptr, ln_w != nullptr);
    const int opts = w_ok | (u_raw ? 2 : 0);
    size_t smem = router_smem<T, WT>(TT, C, E, w_ok != 0, ln_w != nullptr).total;
    DecodeKey<T> dk{nullptr, nullptr, 0, nullptr, nullptr, 0, 0, nullptr};
    const RouterLn<T> lnp{(const T*)ln_w, (const T*)ln_b, (T*)xn};
    int grid = nb;
    if (front) {
      grid = decode_router_groups(N);
      dk = DecodeKey<T>{(const T*)front->wk, (T*)front->h, front->F, (const T*)front->at, (T*)front->u, front->kx,
                        front->wk_packed ? 1 : 0, (T*)front->g};
      grid += decode_front_tiles(N, front->F, front->kx);
      smem = std::max(smem, decode_key_smem(C, (int)sizeof(T)));
    }
    auto launch = [&](auto kern) -> hipError_t {
      if (smem > 65536) {
        hipError_t err = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (err != hipSuccess) return err;
      }
      launch_kernel(kern, dim3(grid), dim3(kRouterThreads), smem, s, (const T*)x, (const WT*)wg, bias,
                         (const T*)xprev, (const T*)mu, (const T*)at, N, T_, C, E, k, r, TT, logits, inds, (T*)gates,
                         (T*)gate_dense, (T*)xk, (T*)u, part_f64, part_cnt, loss_claim, opts, nb, dk, lnp);
      return mark(hipGetLastError(), front ? "decode_front" : "router", s);
    };
// the many-token kernel with or without ln2 in its tile pass
#define RWKV_ROUTER(EB, WU, FPK)                                                    \
  (ln_w ? launch(router_kernel<T, WT, EB, WU, FPK, false, true>)                   \
        : launch(router_kernel<T, WT, EB, WU, FPK, false, false>))
    if (front) {
      if constexpr (sizeof(T) == 2 && !(std::is_same<T, bf16>::value && std::is_same<WT, float>::value)) {
        if (E <= 8) return launch(router_kernel<T, WT, 8, false, 1, true>);
        return launch(router_kernel<T, WT, 16, false, 1, true>);
      }
      return hipErrorInvalidValue;
    }
    if (u) {
      if constexpr (std::is_same<T, f16>::value) {
        if (fpk == 2) {
          if (E <= 8) return RWKV_ROUTER(8, true, 2);
          if (E <= 16) return RWKV_ROUTER(16, true, 2);
          return hipErrorInvalidValue;
        }
      }
      if (E <= 8) return RWKV_ROUTER(8, true, 1);
      if (E <= 16) return RWKV_ROUTER(16, true, 1);
      return hipErrorInvalidValue;  // E * r <= 128 with r >= 8
    }
    if (E <= 8) return RWKV_ROUTER(8, false, 1);
    if (E <= 16) return RWKV_ROUTER(16, false, 1);
    if (E <= 32) return RWKV_ROUTER(32, false, 1);
    return RWKV_ROUTER(64, false, 1);
#undef RWKV_ROUTER
  };
  switch (dtype) {
    case 0: return go(float{}, float{});
    case 1: return gate32 ? go(f16{}, float{}) : go(f16{}, f16{});
    case 2: return gate32 ? go(bf16{}, float{}) : go(bf16{}, bf16{});
    default: return hipErrorInvalidValue;
  }
}

bool decode_front_ok(int N, int C, int F, int E, int dtype, bool gate32) {
  // (a bf16 layer with an fp32 gate is left to the many-token kernels: its
  // router and the key tiles together exceed the register file)
  // two workgroups per CU: each within half the LDS, W_gate staged
  // (the decode router stages W_gate in LDS: it must fit)
  const int tt = router_tile_tokens(N, C, E, dtype);
  const RouterSmem rs = gate32 ? router_smem<f16, float>(tt, C, E, true) : router_smem<f16, f16>(tt, C, E, true);
  return dtype != 0 && !(dtype == 2 && gate32) && N >= 1 && N <= kDecTok && F % kDecCols == 0 && C % 64 == 0 &&
         E <= 16 && decode_key_smem(C, 2) <= (size_t)kLdsBytes / 2 && rs.w_in_lds &&
         rs.total <= (size_t)kLdsBytes / 2;
}

size_t router_smem_bytes(int dtype, int N, int C, int E, bool gate32, bool ln) {
  const int TT = router_tile_tokens(N, C, E, dtype);
  if (dtype == 0) return router_smem<float, float>(TT, C, E, false, ln).total;  // the plan without W_gate
  if (gate32) return router_smem<f16, float>(TT, C, E, false, ln).total;
  return router_smem<f16, f16>(TT, C, E, false, ln).total;
}

bool router_fuses_adapters(int N, int C, int E, int r, int dtype) {
  // 16-bit types only: fp32 MFMA steps cover 8x fewer K per instruction, and
  // every workgroup would stream twice the bytes of A_all (key-GEMM adapter
  // tiles are cheaper then)
  return dtype != 0 && E * r <= kRouterKx && router_tile_tokens(N, C, E, dtype) == 16;
}

hipError_t launch_router_finalize(const LossJob& jb, hipStream_t s) {
  // a small launch while each thread's one batch of loads covers the blocks
  const int threads = jb.nb <= 1024 ? 256 : kFinThreads;
  launch_kernel(router_finalize_kernel, dim3(1), dim3(threads), 0, s, jb);
  return mark(hipGetLastError(), "router_finalize", s);
}

}  // namespace rwkvmoe
