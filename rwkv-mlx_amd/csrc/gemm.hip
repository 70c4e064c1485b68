// MFMA GEMMs of the ChannelMix path for gfx950.
//
// Both products are "NT": out(M,N) = A(M,K) · B(N,K)ᵀ with both operands
// K-contiguous, which is how the reference stores them:
//   key    h   = relu(xk · W_keyᵀ)²          A = xk (N_tok,C)  B = W_key (F,C)    model.py:260-262
//          U   = w ⊙ (x · A_allᵀ)            A = x  (N_tok,C)  B = A_all (Kx,C)   moe.py:140-144
//   value  out = h · W_valueᵀ [+ U · B_allᵀ]  A = h (N_tok,F)   B = W_value (C,F)  model.py:263, moe.py:139-147
// The adapter down-projection U (FUSED mode) rides in the key GEMM as Kx/BN
// extra column tiles that read x instead of xk and apply the gate mask
// w_e[t] (0 for experts t is not routed to) instead of relu².
// xk (the token-shift mix, model.py:67-75, 260-261) is produced once per
// token by the router pass or by shift_mix_kernel, not per output tile.
// relu² and the residual add run in the epilogue.
//
// Kernel structure (256 threads = 4 waves in a 2x2 grid, BM x BN tile):
//   * K is walked in 128-byte slices (64 fp16/bf16 or 32 fp32 elements) that
//     buffer_load_dwordx4 ... lds writes straight into an S-deep LDS ring.  LDS
//     rows are 128 bytes, unpadded, with the 16-byte chunk index XOR-swizzled
//     by row so the MFMA fragment reads are free of bank conflicts.
//   * Each wave computes (BM/2) x (BN/2) with v_mfma_f32_32x32x16_{f16,bf16}
//     (v_mfma_f32_32x32x2f32 for fp32).
//   * The epilogue converts the tile into its own LDS buffer, then writes it
//     out with 16-byte coalesced stores while the next tile's slices load.
//   * Workgroups are persistent (one per CU); each XCD owns a contiguous run
//     of tiles walked in groups of M-tiles (walk_group_m picks the group
//     size per launch), so its resident tiles share operands in that XCD's
//     L2.
#include <stdlib.h>

#include <type_traits>

#include "common.h"
#include "gemm_tile.h"
#include "internal.h"

namespace rwkvmoe {
namespace {

// Persistent GEMM.  gridDim.x workgroups; workgroup w runs on XCD w % 8 and
// walks a contiguous block of that XCD's logical tiles, so the tiles resident
// on one XCD at any time share A rows and B columns in its L2.
//
// K slices stream through an S-deep LDS ring filled by buffer_load_dwordx4
// ... lds (no VGPR staging): lane l of a wave instruction lands at byte 16*l of a
// 1 KB block (1024/RB rows of RB bytes), so each lane fetches the logical
// 16-byte chunk (l % CPR) ^ swz(row) of row l / CPR.  The TB blocks of a
// slice are dealt round-robin over the NW loading waves (block b to wave
// b % NW).  The ring runs across tile boundaries.
// Iteration g (global slice index over this workgroup's tiles):
//   wait for own loads of slice g, barrier (everyone's slice g is in LDS and
//   slice g-1 is no longer read) -> MFMAs on slot g%S, with this wave's loads
//   of slice g+S-1 (into slot (g-1)%S) issued between the MFMA k-steps, so the
//   cycles a wave spends waiting to issue them overlap matrix work -> at a
//   tile's last slice: epilogue.  Load-only waves (LW) just issue loads.
//
// The MFMA computes each block transposed (A operand = W rows, B operand =
// token rows), so a lane's accumulators hold 4 consecutive output columns of
// one token row: the epilogue writes them to LDS as one 8- (16-bit types) or
// 16-byte (fp32) store into a row-major tile whose rows are padded by 16
// bytes, then the tile leaves through coalesced 16-byte global stores.
//
// MX (a 16-bit base with fp32 adapters, EXT): at the first K-extension slice
// the accumulators, which then hold the base product, are rounded to T (the
// base's dtype, model.py:263); the extension [U_hi | 2^-11·U_hi | U_lo] ·
// [B_hi | B_lo' | B_hi] then adds the fp32 delta (moe.py:138-147), and the
// tile leaves in fp32 (out = base + delta in MLX's promoted dtype), with
// the residual added in fp32.
template <typename T, int BM, int BN, int WGM, int WGN, int S, int EPI, bool EXT, int MN, int LW, int RB, bool NTS,
          bool SPLIT, bool GRP, bool MX, bool GK = false>
__global__ __launch_bounds__(64 * (WGM * WGN + LW)) void gemm_kernel(GemmParams<T> p) {
  static_assert(!MX || (EXT && !SPLIT && !GRP && (EPI == EPI_STORE || EPI == EPI_RESID)), "mixed value product");
  static_assert(!GK || (!EXT && !SPLIT && !GRP && !MX && EPI == EPI_STORE), "grouped-K product");
  typedef typename std::conditional<MX, float, T>::type OT;  // output element
  using M = typename MmaSel<T, MN>::type;
  typedef typename M::frag frag;
  typedef typename M::acc accv;
  constexpr int NMW = WGM * WGN;        // MFMA waves, WGM x WGN grid over the tile
  constexpr int NW = NMW + LW;          // all waves issue loads; the last LW issue loads only
  constexpr int NT = 64 * NW;           // threads
  static_assert(NT >= kDispThreads, "a dispatch job block needs 256 threads");
  constexpr int VEC = 16 / sizeof(T);   // elements per 16-byte chunk
  constexpr int BK = RB / sizeof(T);    // elements per K slice (one RB-byte LDS row)
  constexpr int CPR = RB / 16;          // 16-byte chunks per row
  constexpr int RPB = 1024 / RB;        // rows per 1 KB DMA block
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int MI = WM / MN, NI = WN / MN;
  static_assert(MI * MN == WM && NI * MN == WN, "wave tile must be a multiple of the MFMA block");
  constexpr int A_BYTES = BM * RB, STAGE = (BM + BN) * RB;
  constexpr int TB = (BM + BN) / RPB;   // 1 KB DMA blocks per slice
  constexpr int DLO = TB / NW, NHI = TB % NW;  // waves < NHI issue DLO + 1 blocks per slice, the others DLO
  constexpr int DMAX = DLO + (NHI > 0 ? 1 : 0);
  constexpr int NKK = BK / M::KS;       // MFMA k-steps per slice
  constexpr bool OSW = out_swizzled<OT, BM, BN, S, RB>();  // unpadded output rows, chunk index swizzled
  static_assert(!OSW || BN * (int)sizeof(OT) / 16 >= 32, "the swizzle needs 32 chunks per output row");
  constexpr int OSTR = BN * (int)sizeof(OT) + (OSW ? 0 : 16);  // output tile row stride in LDS (bytes)
  constexpr int OUT_BYTES = BM * OSTR;
  // the output tile reuses the ring when it does not fit beside it (then the
  // workgroup has a single tile: the launcher guarantees it)
  constexpr bool OUT_IN_RING = out_in_ring<OT, BM, BN, S, RB>();
  constexpr int LDS_BYTES = OUT_IN_RING ? S * STAGE : S * STAGE + OUT_BYTES;
  static_assert(MI >= 1 && NI >= 1 && DMAX >= 1, "tile too small");
  static_assert(TB * RPB == BM + BN && BM % RPB == 0, "slice rows must fill whole DMA blocks");
  static_assert(LDS_BYTES <= 163840, "LDS budget");
  static_assert((S - 2) * DMAX < 64, "vmcnt range");
  static_assert(M::ACC % 4 == 0, "epilogue writes 4 accumulators at a time");

  __shared__ __attribute__((aligned(1024))) unsigned char lds[LDS_BYTES];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool mma_wave = wave < NMW;
  const int wm = mma_wave ? wave / WGN : 0, wn = mma_wave ? wave % WGN : 0;
  const int nblk = wave < NHI ? DLO + 1 : DLO;  // this wave's DMA blocks per slice

  const int ks = SPLIT && p.ksplit > 1 ? p.ksplit : 1;  // work items per tile (1 unless instantiated SPLIT)
  const int tiles_m = (p.m + BM - 1) / BM, tiles_n = p.n / BN;
  const int total = tiles_m * tiles_n * ks;
  const int G = gridDim.x, w = blockIdx.x;
  // work items of this workgroup: logical index base + i*step, i < count
  int base, step, count;
  if ((total & 7) == 0 && (G & 7) == 0) {
    const int per_xcd = total >> 3, wx = G >> 3, x = w & 7, j = w >> 3;
    base = x * per_xcd + j;
    step = wx;
    count = j < per_xcd ? (per_xcd - j + wx - 1) / wx : 0;
  } else {
    base = w;
    step = G;
    count = w < total ? (total - w + G - 1) / G : 0;
  }
  // grouped: one tile per workgroup; logical M-tile w / tiles_n is found in
  // the concatenation of the segments' tiles (ceil(rows / BM) each)
  int g_e = 0, g_m0 = 0, mlim = p.m;
  if constexpr (GRP) {
    const int mt = w / tiles_n;
    int acc = 0;
    bool found = false;
    for (int e = 0; e < p.grp_n; ++e) {
      const int lo = p.grp_off[e], hi = p.grp_off[e + 1];
      const int te = (hi - lo + BM - 1) / BM;
      if (!found && mt < acc + te) {
        g_e = e;
        g_m0 = lo + (mt - acc) * BM;
        mlim = hi;
        found = true;
      }
      acc += te;
    }
    base = w;
    step = G;
    count = found ? 1 : 0;  // not found: past the last segment's tiles
  }
  // grouped K: one tile per workgroup, output g_e = w / (tiles per output)
  int gk_k0 = 0, gk_nkt = 0;
  if constexpr (GK) {
    const int per = tiles_m * tiles_n;
    g_e = w / per;
    base = w - g_e * per;
    step = G;
    if (g_e < p.gk_n) {
      gk_k0 = p.gk_off[g_e];
      gk_nkt = (p.gk_off[g_e + 1] - gk_k0) / BK;
    }
    count = gk_nkt > 0 ? 1 : 0;  // (an empty range would leave its output unwritten: the caller pads)
  }
  // The router's loss reduction, run by the first workgroup to reach its
  // last tile's epilogue: thread 0 takes a ticket there (the atomic's latency
  // overlaps the epilogue), and after the tiles (LDS is free then) the
  // workgroup holding ticket 0 runs it.  Grouped launches leave it to their
  // workgroups past the last segment's tiles (there is at least one: the grid
  // holds ceil(m / BM) + grp_n M-tiles, the segments fewer), which are
  // dispatched last, into the launch's tail.
  int ticket = 1;
  auto take_ticket = [&]() {
    if (p.loss.losses != nullptr && tid == 0) ticket = atomicAdd(p.loss.claim, 1);
  };
  auto run_losses = [&]() {
    if (p.loss.losses == nullptr) return;
    static_assert(256 + loss_scratch_bytes(NT) <= LDS_BYTES, "loss scratch");
    __syncthreads();
    int* flag = (int*)lds;
    if (tid == 0) flag[0] = ticket;
    __syncthreads();
    const bool mine = flag[0] == 0;
    __syncthreads();
    if (mine) {
      double* sp = (double*)(lds + 256);
      long long* sc = (long long*)(sp + NT);
      reduce_losses(p.loss, sp, sc, (double*)(sc + NT));
    }
  };
  if (count == 0) {
    take_ticket();
    run_losses();
    dispatch_job_run(p.disp, (int*)lds + 1, (int*)(lds + 256));
    return;
  }
  // (with OUT_IN_RING, run() launches one workgroup per tile, so count <= 1)
  const int GROUP_M = p.group_m > 0 ? p.group_m : 8;
  const int in_group = GROUP_M * tiles_n;
  auto tile_of = [&](int i, int& m0, int& n0) {
    if constexpr (GRP) {
      m0 = g_m0;
      n0 = (base % tiles_n) * BN;
      return;
    }
    if constexpr (GK) {
      m0 = (base / tiles_n) * BM;
      n0 = (base % tiles_n) * BN;
      return;
    }
    const int l = ks > 1 ? (base + i * step) / ks : base + i * step;
    const int first_m = (l / in_group) * GROUP_M;
    const int gsize = min(tiles_m - first_m, GROUP_M);
    m0 = (first_m + (l % in_group) % gsize) * BM;
    n0 = ((l % in_group) / gsize) * BN;
  };

  auto split_of = [&](int i) { return ks > 1 ? (base + i * step) % ks : 0; };

  const int nk1 = p.k1 / BK;
  const int nkt = GK ? gk_nkt : (nk1 + (EXT ? p.k2 / BK : 0)) / ks;  // K slices per work item (the launcher checks ks divides)
  const int gtotal = count * nkt;

  // operand rows of slice g: A row m0 + i is A + i*lda + kb, B row j is B + j*ldb + kb
  struct Src {
    const T* A;
    const T* B;
    int lda, ldb, kb, m0;
  };
  // a workgroup with one work item (every launch but the persistent ones)
  // takes its tile from registers: no per-slice index arithmetic
  int m00 = 0, n00 = 0;
  tile_of(0, m00, n00);
  // the loads ask for slices in ascending order (one more per iteration), so
  // a persistent workgroup keeps the tile of its latest request and steps it
  // forward at a tile boundary instead of dividing on every slice
  int d_ti = 0, d_g0 = 0, d_m0 = m00, d_n0 = n00;
  auto slice_src = [&](int g) -> Src {
    if (count > 1)
      while (g >= d_g0 + nkt) {
        ++d_ti;
        d_g0 += nkt;
        tile_of(d_ti, d_m0, d_n0);
      }
    const int ti = d_ti;
    const int m0 = d_m0, n0 = d_n0;
    const int kt = split_of(ti) * nkt + (g - d_g0);
    const bool adapter = EPI == EPI_KEYAD && n0 >= p.n_key;
    const bool seg2 = EXT && kt >= nk1;
    Src r;
    r.A = seg2 ? p.a2 : (adapter ? p.a_ad : p.a1);
    r.B = seg2 ? p.b2 + (size_t)n0 * p.ldb2
               : (adapter ? p.b_ad + (size_t)(n0 - p.n_key) * p.ldb1
                          : p.b1 + (GRP ? (size_t)g_e * p.grp_bstride : 0) + (size_t)n0 * p.ldb1);
    r.lda = seg2 ? p.lda2 : p.lda1;
    r.ldb = seg2 ? p.ldb2 : p.ldb1;
    r.kb = gk_k0 + (seg2 ? kt - nk1 : kt) * BK;
    r.m0 = m0;
    return r;
  };

  // block i (< nblk) of this wave for the slice described by sr, into slot.
  // The buffer starts at the tile's first row (A) or column (B), so the
  // 32-bit offsets stay within BM (BN) rows of one operand; rows past the
  // end of A are clamped to its last row.
  auto dma_block = [&](const Src& sr, unsigned char* slot, int i) {
    const int blk = wave + i * NW;
    const bool is_a = blk < BM / RPB;
    const int rb = is_a ? blk : blk - BM / RPB;
    const int row = rb * RPB + lane / CPR;
    const int c = (lane % CPR) ^ swz<RB>(row);
    const T* base = is_a ? sr.A + (size_t)sr.m0 * sr.lda : sr.B;
    const int r = is_a ? min(sr.m0 + row, mlim - 1) - sr.m0 : row;
    const unsigned off =
        ((unsigned)r * (unsigned)(is_a ? sr.lda : sr.ldb) + (unsigned)(sr.kb + c * VEC)) * (unsigned)sizeof(T);
    buffer_load_lds16(buf_rsrc(base, 0x7FFFFFF0u), (lds_ptr_t)(slot + (is_a ? 0 : A_BYTES) + rb * 1024), off);
  };
  // all of this wave's loads of slice g_req (clamped to the last slice: a
  // clamped load lands in a slot no later iteration reads, and keeps the
  // per-wave load count of every iteration the same)
  auto dma_all = [&](int g_req) {
    const Src sr = slice_src(min(g_req, gtotal - 1));
    unsigned char* slot = lds + (g_req % S) * STAGE;
#pragma unroll
    for (int i = 0; i < DMAX; ++i)
      if (i < nblk) dma_block(sr, slot, i);
  };

  auto frag_at = [](const unsigned char* base_, int row, int k) -> const frag* {
    const int byte = k * (int)sizeof(T);
    return (const frag*)(base_ + row * RB + (((byte >> 4) ^ swz<RB>(row)) << 4) + (byte & 15));
  };

  accv acc[MI][NI];
  auto zero_acc = [&]() {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int v = 0; v < M::ACC; ++v) acc[i][j][v] = 0.f;
  };

  // MFMAs of slot `slot`; this wave's loads of slice g_dma go out between the
  // k-steps (block i after step (i * NKK) / DMAX)
  auto compute = [&](int slot, int g_dma) {
    const unsigned char* As = lds + slot * STAGE;
    const unsigned char* Bs = As + A_BYTES;
    const Src sr = slice_src(min(g_dma, gtotal - 1));
    unsigned char* dslot = lds + (g_dma % S) * STAGE;
    if constexpr (M::KV == 1) {
      // fp32 (one k value per lane and step): lane group q = lane / MN takes
      // k = q·KR + t at step t, the same in both operands, so its KR values
      // of the slice are contiguous and are read as 16-byte chunks ahead of
      // the MFMAs (one 4-byte read per step left every MFMA waiting on LDS)
      constexpr int KR = BK / (64 / MN);
      static_assert(KR == NKK && KR % 4 == 0, "fp32 slice split");
      const int k0 = (lane / MN) * KR;
      f32x4 av[MI][KR / 4], bv[NI][KR / 4];
#pragma unroll
      for (int c = 0; c < KR / 4; ++c) {
#pragma unroll
        for (int i = 0; i < MI; ++i) av[i][c] = *(const f32x4*)frag_at(As, wm * WM + i * MN + (lane % MN), k0 + 4 * c);
#pragma unroll
        for (int j = 0; j < NI; ++j) bv[j][c] = *(const f32x4*)frag_at(Bs, wn * WN + j * MN + (lane % MN), k0 + 4 * c);
      }
#pragma unroll
      for (int t = 0; t < NKK; ++t) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < NI; ++j) acc[i][j] = M::run(bv[j][t / 4][t % 4], av[i][t / 4][t % 4], acc[i][j]);
#pragma unroll
        for (int i = 0; i < DMAX; ++i)
          if ((i * NKK) / DMAX == t && i < nblk) dma_block(sr, dslot, i);
      }
      return;
    }
#pragma unroll
    for (int t = 0; t < NKK; ++t) {
      const int k = t * M::KS + (lane / MN) * M::KV;
      frag af[MI], bf[NI];
#pragma unroll
      for (int i = 0; i < MI; ++i) af[i] = *frag_at(As, wm * WM + i * MN + (lane % MN), k);
#pragma unroll
      for (int j = 0; j < NI; ++j) bf[j] = *frag_at(Bs, wn * WN + j * MN + (lane % MN), k);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = M::run(bf[j], af[i], acc[i][j]);
#pragma unroll
      for (int i = 0; i < DMAX; ++i)
        if ((i * NKK) / DMAX == t && i < nblk) dma_block(sr, dslot, i);
    }
  };

  unsigned char* ot = OUT_IN_RING ? lds : lds + S * STAGE;
  // byte offset of an output element within its row of the LDS tile
  auto ocol = [](int row, int byte) -> int { return OSW ? ((((byte >> 4) ^ (row & 31)) << 4) | (byte & 15)) : byte; };
  // epilogue, part 1 (MFMA waves): accumulators -> LDS tile
  auto epi_acc = [&](int ti) {
    int m0, n0;
    tile_of(ti, m0, n0);
    const bool adapter = EPI == EPI_KEYAD && n0 >= p.n_key;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int row = wm * WM + i * MN + (lane % MN);
#pragma unroll
        for (int v0 = 0; v0 < M::ACC; v0 += 4) {
          const int col = wn * WN + j * MN + acc_row_n<MN>(v0, lane);  // 4 consecutive columns
          unsigned char* dst = ot + row * OSTR + ocol(row, col * (int)sizeof(OT));
          if constexpr (MX) {  // fp32 out: the accumulators as they are
            *(f32x4*)dst = f32x4{acc[i][j][v0], acc[i][j][v0 + 1], acc[i][j][v0 + 2], acc[i][j][v0 + 3]};
            continue;
          }
          if constexpr ((EPI == EPI_KEY || EPI == EPI_KEYAD) && std::is_same<T, f16>::value) {
            if (!adapter) {
              *(unsigned long long*)dst = relu2_f16x4(acc[i][j][v0], acc[i][j][v0 + 1], acc[i][j][v0 + 2], acc[i][j][v0 + 3]);
              continue;
            }
          }
          float r[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) r[q] = rnd<T>(acc[i][j][v0 + q]);
          if constexpr (EPI == EPI_KEY || EPI == EPI_KEYAD) {
            if (!adapter) {
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const float z = r[q] > 0.f ? r[q] : 0.f;
                r[q] = z * z;  // relu(key(k)) ** 2 (model.py:262)
              }
            } else {
              adapter_scale4(p, min(m0 + row, p.m - 1), n0 - p.n_key + col, r);
            }
          }
          T o[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) o[q] = from_f<T>(r[q]);
          if constexpr (sizeof(T) == 4) {
            *(f32x4*)dst = f32x4{to_f(o[0]), to_f(o[1]), to_f(o[2]), to_f(o[3])};
          } else {
            union { T e[4]; unsigned long long u; } pk;
#pragma unroll
            for (int q = 0; q < 4; ++q) pk.e[q] = o[q];
            *(unsigned long long*)dst = pk.u;
          }
        }
      }
  };
  // epilogue, part 2 (every wave): LDS tile -> global, 16-byte coalesced stores
  auto epi_store = [&](int ti) {
    int m0, n0;
    tile_of(ti, m0, n0);
    const bool adapter = EPI == EPI_KEYAD && n0 >= p.n_key;
    constexpr int OVEC = 16 / (int)sizeof(OT);  // output elements per 16-byte chunk
    constexpr int OCPR = BN / OVEC;
#pragma unroll
    for (int it = 0; it < (BM * OCPR + NT - 1) / NT; ++it) {
      const int id = tid + it * NT;
      if (id >= BM * OCPR) break;
      const int row = id / OCPR, c = (id % OCPR) * OVEC;
      const int gm = m0 + row;
      if (gm >= mlim) continue;
      u32x4 v = *(const u32x4*)(ot + row * OSTR + ocol(row, c * (int)sizeof(OT)));
      if constexpr (MX) {
        // fp32 out (+ the residual, in dtype, added in fp32)
        if constexpr (EPI == EPI_RESID) {
          union { unsigned long long u; T e[4]; } rr;
          rr.u = *(const unsigned long long*)(p.resid + (size_t)gm * p.ldo + n0 + c);
          f32x4 o = __builtin_bit_cast(f32x4, v);
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = to_f(rr.e[e]) + o[e];
          v = __builtin_bit_cast(u32x4, o);
        }
        *(u32x4*)((float*)(void*)p.out + (size_t)gm * p.ldo + n0 + c) = v;
        continue;
      }
      if constexpr (EPI == EPI_RESID) {
        Chunk<T> o, rr;
        o.raw = v;
        rr.raw = *(const u32x4*)(p.resid + (size_t)gm * p.ldo + n0 + c);
#pragma unroll
        for (int e = 0; e < VEC; ++e) o.e[e] = from_f<T>(to_f(rr.e[e]) + to_f(o.e[e]));
        v = o.raw;
      }
      T* dstp = (EPI == EPI_KEYAD && adapter)
                    ? p.out_ad + (size_t)gm * (p.n - p.n_key) + (n0 - p.n_key) + c
                    : p.out + (GK ? (size_t)g_e * p.gk_ostride : 0) + (size_t)gm * p.ldo + n0 + c;
      if constexpr (NTS) __builtin_nontemporal_store(v, (u32x4*)dstp);
      else *(u32x4*)dstp = v;
    }
  };
  // split-K epilogue (MFMA waves): the raw fp32 accumulators of this work
  // item -> part[split], 4 consecutive columns per 16-byte store
  auto epi_partial = [&](int ti) {
    int m0, n0;
    tile_of(ti, m0, n0);
    float* dst = p.part + (size_t)split_of(ti) * p.m * p.n;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int gm = m0 + wm * WM + i * MN + (lane % MN);
        if (gm < p.m) {
#pragma unroll
          for (int v0 = 0; v0 < M::ACC; v0 += 4) {
            const int col = n0 + wn * WN + j * MN + acc_row_n<MN>(v0, lane);
            *(f32x4*)(dst + (size_t)gm * p.n + col) =
                f32x4{acc[i][j][v0], acc[i][j][v0 + 1], acc[i][j][v0 + 2], acc[i][j][v0 + 3]};
          }
        }
      }
  };
  // the output tile may overlay the ring: wait until no load into it is in flight
  auto ring_idle = [&]() {
    if constexpr (OUT_IN_RING) asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  };
  auto wait_slice = [&]() {
    if (wave < NHI) wait_vm_barrier<(S - 2) * (DLO + 1)>();
    else wait_vm_barrier<(S - 2) * DLO>();
  };

#pragma unroll
  for (int s = 0; s < S - 1; ++s) dma_all(s);
  // MFMA waves and load-only waves run separate loops with the same barrier
  // sequence (one per slice, two per tile epilogue)
  // launches with one tile per workgroup by construction never take the
  // multi-tile loop, which is then not compiled
  constexpr bool ONE_TILE = OUT_IN_RING || GRP || GK;
  if (mma_wave && (ONE_TILE || count == 1)) {
    // one work item: no tile boundary inside the K loop, so the accumulators
    // are only ever written by the MFMAs there (with a boundary in the loop
    // the compiler copied a 128x128 wave tile's 256 accumulators between
    // register files on every slice)
    zero_acc();
    wait_scalar_loads();
    for (int g = 0; g < gtotal; ++g) {
      wait_slice();
      if constexpr (MX) {
        if (g == nk1) {  // first K-extension slice: round the base product to T
#pragma unroll
          for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j)
#pragma unroll
              for (int v = 0; v < M::ACC; ++v) acc[i][j][v] = rnd<T>(acc[i][j][v]);
        }
      }
      compute(g % S, g + S - 1);
    }
    if (!GRP) take_ticket();
    if (ks > 1) {
      epi_partial(0);
    } else {
      ring_idle();
      epi_acc(0);
      wait_lds_barrier();
      epi_store(0);
    }
  } else if (mma_wave) {
    if constexpr (!ONE_TILE) {
    zero_acc();
    wait_scalar_loads();
    int ti = 0, kk = 0;  // work item of slice g and the slice's place in it
    for (int g = 0; g < gtotal; ++g) {
      wait_slice();
      if constexpr (MX) {
        // first K-extension slice: the base product is complete; round it to T
        if (kk == nk1) {
#pragma unroll
          for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j)
#pragma unroll
              for (int v = 0; v < M::ACC; ++v) acc[i][j][v] = rnd<T>(acc[i][j][v]);
        }
      }
      compute(g % S, g + S - 1);
      if (kk == nkt - 1) {
        if (!GRP && ti == count - 1) take_ticket();
        if (ks > 1) {
          epi_partial(ti);
        } else {
          ring_idle();
          epi_acc(ti);
          wait_lds_barrier();
          epi_store(ti);
        }
        zero_acc();
      }
      if (++kk == nkt) {
        kk = 0;
        ++ti;
      }
    }
    }
  } else {
    int ti = 0, kk = 0;
    for (int g = 0; g < gtotal; ++g) {
      wait_slice();
      dma_all(g + S - 1);
      if (kk == nkt - 1 && ks == 1) {
        ring_idle();
        wait_lds_barrier();
        epi_store(ti);
      }
      if (++kk == nkt) {
        kk = 0;
        ++ti;
      }
    }
  }
  // drain the trailing clamped loads before the workgroup's LDS is released
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  run_losses();
  // the SPARSE forward's dispatch scatter, block by block (after the tile:
  // the key product does not read it)
  dispatch_job_run(p.disp, (int*)lds + 1, (int*)(lds + 256));
}

// Split K: the fp32 partials part[0..ksplit) are summed in ascending split
// order, then the unsplit kernel's epilogue runs with the same rounding
// points: relu² on key columns, the gate mask on adapter columns, the
// residual add.  One thread per 4 output columns; the partial loads go out 8
// at a time.
template <typename T, int EPI>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmParams<T> p) {
  const int n4 = p.n / 4;
  const int id = blockIdx.x * 256 + threadIdx.x;
  if (id >= p.m * n4) return;
  const int gm = id / n4, gc = (id - gm * n4) * 4;
  const size_t plane = (size_t)p.m * p.n;
  const float* src = p.part + (size_t)gm * p.n + gc;
  f32x4 a = *(const f32x4*)src;
  for (int s0 = 1; s0 < p.ksplit; s0 += 8) {
    f32x4 b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] = *(const f32x4*)(src + (size_t)min(s0 + i, p.ksplit - 1) * plane);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (s0 + i < p.ksplit) a = f32x4{a[0] + b[i][0], a[1] + b[i][1], a[2] + b[i][2], a[3] + b[i][3]};
  }
  const bool adapter = EPI == EPI_KEYAD && gc >= p.n_key;
  float r[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) r[q] = rnd<T>(a[q]);
  if constexpr (EPI == EPI_KEY || EPI == EPI_KEYAD) {
    if (!adapter) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float z = r[q] > 0.f ? r[q] : 0.f;
        r[q] = z * z;  // relu(key(k)) ** 2 (model.py:262)
      }
    } else {
      adapter_scale4(p, gm, gc - p.n_key, r);
    }
  }
  T o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    o[q] = from_f<T>(r[q]);
    if constexpr (EPI == EPI_RESID) o[q] = from_f<T>(to_f(p.resid[(size_t)gm * p.ldo + gc + q]) + to_f(o[q]));
  }
  T* dst = adapter ? p.out_ad + (size_t)gm * (p.n - p.n_key) + (gc - p.n_key) : p.out + (size_t)gm * p.ldo + gc;
  if constexpr (sizeof(T) == 4) {
    *(f32x4*)dst = f32x4{to_f(o[0]), to_f(o[1]), to_f(o[2]), to_f(o[3])};
  } else {
    union { T e[4]; unsigned long long u; } pk;
#pragma unroll
    for (int q = 0; q < 4; ++q) pk.e[q] = o[q];
    *(unsigned long long*)dst = pk.u;
  }
}

// xk = x + (shift(x) - x) * x_k, each op rounded to T (model.py:260-261);
// shift(x)[t] = x[t-1], x_prev[b] or 0 at t = 0 of a sequence (model.py:73-75).
template <typename T>
__global__ __launch_bounds__(256) void shift_mix_kernel(const T* __restrict__ x, const T* __restrict__ xprev,
                                                        const T* __restrict__ mu, T* xk, int N, int T_, int C) {
  constexpr int VEC = 16 / sizeof(T);
  const int cpr = C / VEC;
  const size_t id = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (id >= (size_t)N * cpr) return;
  const int n = (int)(id / cpr), c = (int)(id % cpr) * VEC;
  const int t = n % T_;
  const u32x4 xv = *(const u32x4*)(x + (size_t)n * C + c);
  const u32x4 pv = t > 0 ? *(const u32x4*)(x + (size_t)(n - 1) * C + c)
                         : (xprev ? *(const u32x4*)(xprev + (size_t)(n / T_) * C + c) : zero4());
  *(u32x4*)(xk + (size_t)n * C + c) = shift_mix_chunk<T>(xv, pv, *(const u32x4*)(mu + c));
}


template <typename T, int BM, int BN, int WGM, int WGN, int S, int EPI, bool EXT, int MN = 32, int LW = 0, int RB = 128,
          bool NTS = false, bool SPLIT = false, bool GRP = false, bool MX = false, bool GK = false>
hipError_t run(const GemmParams<T>& p, hipStream_t s, bool persistent) {
  typedef typename std::conditional<MX, float, T>::type OT;
  constexpr int BK = RB / (int)sizeof(T);
  if (p.k1 % BK || (EXT && p.k2 % BK)) return hipErrorInvalidValue;
  if (p.n % BN) return hipErrorInvalidValue;
  const int ks = p.ksplit > 1 ? p.ksplit : 1;
  if (ks > 1 && (!SPLIT || !p.part || persistent)) return hipErrorInvalidValue;
  if ((p.k1 / BK + (EXT ? p.k2 / BK : 0)) % ks) return hipErrorInvalidValue;
  if (GRP && (ks > 1 || !p.grp_off || p.grp_n < 1)) return hipErrorInvalidValue;
  if (GK && (ks > 1 || !p.gk_off || p.gk_n < 1)) return hipErrorInvalidValue;
  // grouped: every segment may end in a partial tile, one more tile row each
  const int tiles = GK ? p.gk_n * ((p.m + BM - 1) / BM) * (p.n / BN)
                       : ((p.m + BM - 1) / BM + (GRP ? p.grp_n : 0)) * (p.n / BN) * ks;  // work items
  if (tiles == 0) return hipSuccess;
  int grid = tiles;
  if (GRP || GK) persistent = false;
  // an output tile staged in the ring leaves room for one tile per workgroup
  if (out_in_ring<OT, BM, BN, S, RB>()) persistent = false;
  if (persistent) {
    grid = num_cus();
    if (grid > tiles) grid = tiles;
    if (tiles % 8 == 0 && grid % 8) grid -= grid % 8;  // keep the XCD-contiguous mapping
  }
  GemmParams<T> q = p;
  if (!GRP && !GK && ks == 1) q.group_m = walk_group_m((p.m + BM - 1) / BM, p.n / BN, BM, BN);
  launch_kernel((gemm_kernel<T, BM, BN, WGM, WGN, S, EPI, EXT, MN, LW, RB, NTS, SPLIT, GRP, MX, GK>),
                     dim3(grid), dim3(64 * (WGM * WGN + LW)), 0, s, q);
  return hipGetLastError();
}

// Tile codes: 0 = automatic, 1 = 128x128 persistent, 2 = 128x64 persistent,
// 3 = 256x192 (8 waves), 5 = 256x128 (8 waves), 6 = 128x96 (16x16 MFMA),
// 7 = 64-row tiles with K split (as for small products), 8 = 64x16 tiles over
// the whole K (16-bit, at most 64 rows), 9 = 64x16 tiles with K split,
// 10 = 256x256 (8 waves of 128x64, 64-byte K slices, 5 stages; 16-bit; the
// relu² key products with 128-byte slices in 2 stages).
// Only a tuning build (-DRWKVMOE_TUNING) lets RWKVMOE_GEMM_TILE force a code;
// the library as built reads no environment and always plans automatically.
int tile_override() {
#ifdef RWKVMOE_TUNING
  static int v = [] {
    const char* s = getenv("RWKVMOE_GEMM_TILE");
    return s ? atoi(s) : 0;
  }();
  return v;
#else
  return 0;
#endif
}

// Whether the 256x192 and 128x96 tiles run in their VGPR-staged form
// (gemm_vs.hip).  Only a tuning build (-DRWKVMOE_TUNING) lets RWKVMOE_VS=0
// select the global_load_lds ring form instead, for A/B timing.
bool vs_enabled() {
#ifdef RWKVMOE_TUNING
  static int v = [] {
    const char* s = getenv("RWKVMOE_VS");
    return s ? atoi(s) : 1;
  }();
  return v != 0;
#else
  return true;
#endif
}

// Automatic choice (16-bit): the largest tile that still gives every CU a
// tile — operand traffic from L2 per FLOP falls as 1/BM + 1/BN, and L2->CU
// bandwidth, not MFMA issue, bounds these products.
//   256x256 (8 waves) when N % 256 == 0 and it yields >= 2 tiles per CU with
//   a last wave at least half full (the wide layers' products: 556 / 518
//   against 732 / 706 us for the 256x128 ring at 16384 x 8192 x 2048 and
//   16384 x 2048 x 8192 bf16),
//   256x192 (8 waves) when N % 192 == 0 and it yields >= 90% of a tile per CU,
//   256x128 (8 waves) when N % 128 == 0 and it yields >= 1 tile per CU,
//   128x96 (16x16 MFMA blocks, 256-byte K slices, 4 MFMA waves + 10 waves that
//   only issue loads: DMA throughput grows with the number of issuing waves)
//   when N % 96 == 0 and it yields ~1 tile per CU,
//   else persistent 128x128 (N % 128 == 0) or 128x64.
// When that leaves more than half of the CUs idle (decode batches, small
// layers): 64-row tiles (x128 for 16-bit types when N allows, else x64), and
// K split into the most work items per tile that keeps them within 1.25 per
// CU and at least 2 K slices each (the partials are reduced by
// splitk_reduce_kernel in a fixed order) — except 16-bit products of at most
// 64 rows whose 64x16 tiles give half a wave: those run unsplit.
struct TilePlan {
  int t;   // tile code (RWKVMOE_GEMM_TILE numbering)
  int bn;  // t == 7: tile width
  int ks;  // t == 7: work items per tile
};

TilePlan plan_tiles(int elem, int epi, int m, int n, int n_key, int k_total) {
  const int cus = num_cus();
  // a tile never straddles the key / adapter column boundary
  auto fits = [&](int bn) { return n % bn == 0 && (epi != EPI_KEYAD || n_key % bn == 0); };
  auto tiles = [&](int bm, int bn) { return ((m + bm - 1) / bm) * (n / bn); };
  TilePlan pl{tile_override(), 0, 1};
  const bool automatic = pl.t == 0;
  if (automatic) {
    // (the adapter epilogue's extra live values do not fit 256x192's register budget)
    // 256x256 for products of two or more waves of such tiles whose last wave
    // is at least half full: half the LDS reads per FLOP of the 64x64 wave
    // tiles (8 waves of 128x64)
    const int t256 = tiles(256, 256);
    if (elem == 2 && fits(256) && k_total % 32 == 0 && t256 >= 2 * cus && (t256 % cus == 0 || 2 * (t256 % cus) >= cus))
      pl.t = 10;
    else if (elem == 2 && epi != EPI_KEYAD && fits(192) && tiles(256, 192) * 10 >= cus * 9) pl.t = 3;
    else if (elem == 2 && fits(128) && tiles(256, 128) >= cus) pl.t = 5;
    else if (elem == 2 && fits(96) && tiles(128, 96) * 10 >= cus * 9) pl.t = 6;
    else pl.t = fits(128) ? 1 : 2;
    const int chosen = pl.t == 10 ? t256 : pl.t == 3 ? tiles(256, 192) : pl.t == 5 ? tiles(256, 128)
                     : pl.t == 6 ? tiles(128, 96) : pl.t == 1 ? tiles(128, 128) : tiles(128, 64);
    if (chosen * 2 <= cus) pl.t = 7;
  }
  if (pl.t == 7) {
    pl.bn = (elem == 2 && fits(128)) ? 128 : 64;
    const int nkt = k_total / (128 / elem);  // K slices of 128 bytes
    const int ts = tiles(64, pl.bn);
    if (ts * 2 <= cus)
      for (int c = 2; c <= nkt; ++c)
        if (nkt % c == 0 && nkt / c >= 2 && ts * c <= cus + cus / 4) pl.ks = c;
    // a few rows (decode batches): 64x16 tiles over the whole K when they
    // give at least half a wave, so no split partials and no reduction
    // launch; else 64x16 tiles with K split, which for the same fill write
    // 8x fewer partials than 64x128 tiles
    if (automatic && elem == 2 && m <= 64 && fits(16)) {
      const int t16 = tiles(64, 16);
      if (t16 * 2 >= cus) {
        pl.t = 8;
        pl.ks = 1;
      } else {
        int c16 = 1;
        for (int c = 2; c <= nkt; ++c)
          if (nkt % c == 0 && nkt / c >= 2 && t16 * c <= cus + cus / 4) c16 = c;
        if (c16 > 1) {
          pl.t = 9;
          pl.ks = c16;
        }
      }
    }
  }
  return pl;
}

// With `deferred`, a split product leaves its partials in p.part for the
// caller to reduce (in ascending split order) and reports the split count.
// LW: waves that only issue loads (more loads in flight per CU).
template <typename T, int BM, int BN, int EPI, bool EXT, int LW = 0, int WGM = 2, int WGN = 2, int MN = 32>
hipError_t run_small(GemmParams<T> p, int ks, hipStream_t s, int* deferred) {
  p.ksplit = ks;
  const hipError_t e = run<T, BM, BN, WGM, WGN, 3, EPI, EXT, MN, LW, 128, false, true>(p, s, false);
  if (deferred) *deferred = ks > 1 ? ks : 1;
  if (e != hipSuccess || ks <= 1 || deferred) return e;
  const int grid = (p.m * (p.n / 4) + 255) / 256;
  launch_kernel((splitk_reduce_kernel<T, EPI>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

// Tile codes a mixed value product (MX) runs: the unsplit 16-bit tiles.
bool mixed_tile_ok(int t) { return t == 1 || t == 2 || t == 3 || t == 5 || t == 6 || t == 10; }

template <typename T, int EPI, bool EXT, bool MX = false>
hipError_t dispatch_tile(const GemmParams<T>& p, hipStream_t s, const TilePlan* given = nullptr,
                         int* deferred = nullptr) {
  auto fits = [&](int bn) { return p.n % bn == 0 && (EPI != EPI_KEYAD || p.n_key % bn == 0); };
  const TilePlan pl = given ? *given : plan_tiles((int)sizeof(T), EPI, p.m, p.n, p.n_key, p.k1 + (EXT ? p.k2 : 0));
  const int t = pl.t;
  if (deferred) *deferred = 1;
  if (vs_enabled() && (t == 3 || t == 5 || t == 6)) {
    const hipError_t e = gemm_vs_run<T>(p, t, EPI, EXT, MX, s);
    if (e != hipErrorNotSupported) return e;
  }
  if constexpr (MX) {
    // fp32 out tiles: the 256-row tiles' fp32 output does not fit LDS beside
    // (or inside) their ring, so they give way to 128x128
    if constexpr (sizeof(T) == 2 && EXT && (EPI == EPI_STORE || EPI == EPI_RESID)) {
      if (t == 6 && fits(96)) {
        if (p.k1 % 128 == 0 && p.k2 % 128 == 0)
          return run<T, 128, 96, 2, 2, 2, EPI, EXT, 16, 10, 256, false, false, false, true>(p, s, false);
        return run<T, 128, 96, 2, 2, 4, EPI, EXT, 16, 3, 128, false, false, false, true>(p, s, true);
      }
      if ((t == 1 || t == 3 || t == 5 || t == 10) && fits(128))
        return run<T, 128, 128, 2, 2, 4, EPI, EXT, 32, 0, 128, false, false, false, true>(p, s, true);
      if (mixed_tile_ok(t) && fits(64))
        return run<T, 128, 64, 2, 2, 4, EPI, EXT, 32, 0, 128, false, false, false, true>(p, s, true);
    }
    return hipErrorInvalidValue;
  }
  if constexpr (sizeof(T) == 2)
    if (t == 9 && fits(16)) return run_small<T, 64, 16, EPI, EXT, 0, 4, 1, 16>(p, pl.ks, s, deferred);
  if (t == 7) {
    if (!fits(pl.bn)) return hipErrorInvalidValue;
    // plain products with long work items (8+ K slices each: the backward's
    // token-contracted products) are load-bound: 4 more waves issue loads
    if constexpr (EPI == EPI_STORE && !EXT) {
      const int items_k = p.k1 / (128 / (int)sizeof(T)) / (pl.ks > 1 ? pl.ks : 1);
      if (items_k >= 8) {
        if constexpr (sizeof(T) == 2)
          if (pl.bn == 128) return run_small<T, 64, 128, EPI, EXT, 4>(p, pl.ks, s, deferred);
        return run_small<T, 64, 64, EPI, EXT, 4>(p, pl.ks, s, deferred);
      }
    }
    if constexpr (sizeof(T) == 2)
      if (pl.bn == 128) return run_small<T, 64, 128, EPI, EXT>(p, pl.ks, s, deferred);
    return run_small<T, 64, 64, EPI, EXT>(p, pl.ks, s, deferred);
  }
  if constexpr (sizeof(T) == 2) {
    if (t == 8 && fits(16)) {
      if (p.k1 % 128 == 0 && (!EXT || p.k2 % 128 == 0)) return run<T, 64, 16, 4, 1, 3, EPI, EXT, 16, 0, 256>(p, s, false);
      return run<T, 64, 16, 4, 1, 3, EPI, EXT, 16, 0, 128>(p, s, false);
    }
    // the relu² products in 64-element slices, two 64 KB stages (the skewed
    // layer's key product 80.0 against 83.2 us, D=2048's 520 against 525;
    // the value products measured slower so: 510 against 485 us at D=2048)
    if constexpr (EPI == EPI_KEY)
      if (t == 10 && fits(256) && p.k1 % 64 == 0 && (!EXT || p.k2 % 64 == 0))
        return run<T, 256, 256, 2, 4, 2, EPI, EXT, 32, 0, 128>(p, s, false);
    if (t == 10 && fits(256) && p.k1 % 32 == 0 && (!EXT || p.k2 % 32 == 0))
      return run<T, 256, 256, 2, 4, 5, EPI, EXT, 32, 0, 64>(p, s, false);
    if constexpr (EPI != EPI_KEYAD)
      if (t == 3 && fits(192)) return run<T, 256, 192, 4, 2, 2, EPI, EXT>(p, s, false);
    if ((t == 5 || t == 10) && fits(128)) return run<T, 256, 128, 4, 2, 2, EPI, EXT>(p, s, false);
    if (t == 6 && fits(96)) {
      if (p.k1 % 128 == 0 && (!EXT || p.k2 % 128 == 0)) return run<T, 128, 96, 2, 2, 2, EPI, EXT, 16, 10, 256>(p, s, false);
      return run<T, 128, 96, 2, 2, 4, EPI, EXT, 16, 3>(p, s, true);
    }
    if (t == 1 && fits(128)) return run<T, 128, 128, 2, 2, 4, EPI, EXT>(p, s, true);
    if (!fits(64)) return hipErrorInvalidValue;
    return run<T, 128, 64, 2, 2, 4, EPI, EXT>(p, s, true);
  } else {
    if (t == 1 && fits(128)) return run<T, 128, 128, 2, 2, 3, EPI, EXT>(p, s, true);
    if (!fits(64)) return hipErrorInvalidValue;
    return run<T, 128, 64, 2, 2, 4, EPI, EXT>(p, s, true);
  }
}

template <typename T>
GemmParams<T> blank() {
  GemmParams<T> p;
  __builtin_memset(&p, 0, sizeof(p));
  return p;
}

}  // namespace

int num_cus() {
  static int v = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                 hipSuccess || n <= 0)
      n = 256;
    return n;
  }();
  return v;
}

bool value_plan_mixed_ok(int m, int n, int k_total) {
  return mixed_tile_ok(plan_tiles(2, EPI_STORE, m, n, n, k_total).t);
}

size_t gemm_partial_bytes(int dtype, int m, int n, int n_key, int k_total, bool keyad) {
  const TilePlan pl = plan_tiles(dtype == 0 ? 4 : 2, keyad ? EPI_KEYAD : EPI_KEY, m, n, n_key, k_total);
  return (pl.t == 7 || pl.t == 9) && pl.ks > 1 ? (size_t)pl.ks * m * n * sizeof(float) : 0;
}

hipError_t launch_shift_mix(int dtype, const void* x, const void* xprev, const void* mu, void* xk, int N, int T_,
                            int C, hipStream_t s) {
  RWKV_DISPATCH_DTYPE(dtype, T, {
    const size_t chunks = (size_t)N * (C / (16 / sizeof(T)));
    const int grid = (int)((chunks + 255) / 256);
    if (grid == 0) return hipSuccess;
    launch_kernel(shift_mix_kernel<T>, dim3(grid), dim3(256), 0, s, (const T*)x, (const T*)xprev, (const T*)mu,
                       (T*)xk, N, T_, C);
  });
  return mark(hipGetLastError(), "shift_mix", s);
}

// Whether the key product with adapter columns runs as two launches, the key
// columns alone and then the adapter columns alone (n_key = 0).  One launch
// rounds the combined tile count up to whole rounds of tiles over the CUs:
// at D=2048 (F = 8192, Kx = 512, 16384 tokens) 2176 tiles of 256x256 on 256
// CUs run as 9 rounds where the key columns alone fill 8 exactly.  Two
// launches round each product up on its own tiles (the adapter product takes
// smaller ones).  Tile area per round stands for time; only wide key
// products (256x256 tiles) are considered.
bool split_key_adapters(int elem, int N, int C, int F, int kx) {
  auto dims = [](int t, int& bm, int& bn) {
    switch (t) {
      case 10: bm = 256; bn = 256; return true;
      case 3: bm = 256; bn = 192; return true;
      case 5: bm = 256; bn = 128; return true;
      case 6: bm = 128; bn = 96; return true;
      case 1: bm = 128; bn = 128; return true;
      case 2: bm = 128; bn = 64; return true;
      default: return false;  // split-K and decode tiles
    }
  };
  const TilePlan k = plan_tiles(elem, EPI_KEY, N, F, F, C);
  const TilePlan c = plan_tiles(elem, EPI_KEYAD, N, F + kx, F, C);
  const TilePlan a = plan_tiles(elem, EPI_KEYAD, N, kx, 0, C);
  int bmk, bnk, bmc, bnc, bma, bna;
  if (k.t != 10 || !dims(k.t, bmk, bnk) || !dims(c.t, bmc, bnc) || !dims(a.t, bma, bna)) return false;
  const long long cus = num_cus();
  auto cost = [&](int bm, int bn, int n) {
    const long long tiles = (long long)((N + bm - 1) / bm) * (n / bn);
    return (tiles + cus - 1) / cus * bm * bn;
  };
  return cost(bmk, bnk, F) + cost(bma, bna, kx) < cost(bmc, bnc, F + kx);
}

hipError_t launch_cmix_key(int dtype, const void* xk, const void* wk, void* h, int N, int C, int F, const void* x,
                           const void* at, const void* gdense, int E, int r, int kx, void* u, const LossJob* loss,
                           float* part, hipStream_t s, const DispatchJob* disp) {
  RWKV_DISPATCH_DTYPE(dtype, T, {
    GemmParams<T> p = blank<T>();
    if (loss) p.loss = *loss;
    if (disp) p.disp = *disp;
    p.part = part;
    p.a1 = (const T*)xk; p.lda1 = C; p.b1 = (const T*)wk; p.ldb1 = C; p.k1 = C;
    p.m = N; p.n = F; p.out = (T*)h; p.ldo = F; p.n_key = F;
    if (u) {
      p.n = F + kx; p.a_ad = (const T*)x; p.b_ad = (const T*)at; p.out_ad = (T*)u;
      p.gmat = (const T*)gdense; p.n_experts = E; p.rank = r;
    }
    if (u && split_key_adapters((int)sizeof(T), N, C, F, kx)) {
      GemmParams<T> pk = p;  // the key columns (with the loss reduction)
      pk.n = F;
      const hipError_t e = mark(dispatch_tile<T, EPI_KEY, false>(pk, s), "cmix_key", s);
      if (e != hipSuccess) return e;
      GemmParams<T> pa = blank<T>();  // the adapter columns: every tile is an adapter tile
      pa.part = part;
      pa.a1 = (const T*)x; pa.lda1 = C; pa.b1 = (const T*)at; pa.ldb1 = C; pa.k1 = C;
      pa.m = N; pa.n = kx; pa.out = (T*)u; pa.ldo = kx; pa.n_key = 0;
      pa.a_ad = (const T*)x; pa.b_ad = (const T*)at; pa.out_ad = (T*)u;
      pa.gmat = (const T*)gdense; pa.n_experts = E; pa.rank = r;
      return mark(dispatch_tile<T, EPI_KEYAD, false>(pa, s), "cmix_adapters", s);
    }
    if (u) return mark(dispatch_tile<T, EPI_KEYAD, false>(p, s), "cmix_key_adapters", s);
    return mark(dispatch_tile<T, EPI_KEY, false>(p, s), "cmix_key", s);
  });
  return hipSuccess;
}

hipError_t launch_cmix_value(int dtype, const void* h, const void* wv, int F, const void* u, const void* bt, int kx,
                             const void* resid, void* out, int N, int C, float* part, hipStream_t s, bool mixed) {
  if (mixed) {
    // K-extension [U_hi | 2^-11·U_hi | U_lo] · [B_hi | B_lo' | B_hi]: 3·kx
    if (dtype != 1 || !u || !bt) return hipErrorInvalidValue;
    typedef f16 T;
    GemmParams<T> p = blank<T>();
    p.a1 = (const T*)h; p.lda1 = F; p.b1 = (const T*)wv; p.ldb1 = F; p.k1 = F;
    p.a2 = (const T*)u; p.lda2 = 3 * kx; p.b2 = (const T*)bt; p.ldb2 = 3 * kx; p.k2 = 3 * kx;
    p.m = N; p.n = C; p.out = (T*)out; p.ldo = C; p.resid = (const T*)resid;
    const hipError_t e = resid ? dispatch_tile<T, EPI_RESID, true, true>(p, s) : dispatch_tile<T, EPI_STORE, true, true>(p, s);
    return mark(e, "cmix_value_adapters", s);
  }
  RWKV_DISPATCH_DTYPE(dtype, T, {
    GemmParams<T> p = blank<T>();
    p.part = part;
    p.a1 = (const T*)h; p.lda1 = F; p.b1 = (const T*)wv; p.ldb1 = F; p.k1 = F;
    if (u && bt) { p.a2 = (const T*)u; p.lda2 = kx; p.b2 = (const T*)bt; p.ldb2 = kx; p.k2 = kx; }
    p.m = N; p.n = C; p.out = (T*)out; p.ldo = C; p.resid = (const T*)resid;
    hipError_t e;
    if (p.k2 > 0) e = resid ? dispatch_tile<T, EPI_RESID, true>(p, s) : dispatch_tile<T, EPI_STORE, true>(p, s);
    else e = resid ? dispatch_tile<T, EPI_RESID, false>(p, s) : dispatch_tile<T, EPI_STORE, false>(p, s);
    return mark(e, p.k2 > 0 ? "cmix_value_adapters" : "cmix_value", s);
  });
  return hipSuccess;
}

bool value_combine_fusable(int dtype, int N, int C, int F, int k) {
  if (dtype == 0 || k < 1 || k > kCombineMaxK || !vs_enabled()) return false;
  const TilePlan pl = plan_tiles(2, EPI_STORE, N, C, C, F);
  return (pl.t == 6 && F % 128 == 0 && C % 96 == 0) || (pl.t == 5 && F % 64 == 0 && C % 128 == 0);
}

hipError_t launch_cmix_value_combine(int dtype, const void* h, const void* wv, int F, const void* rows,
                                     const int* inds, const void* gates, const void* resid, void* out, int N, int C,
                                     int k, hipStream_t s) {
  if (!value_combine_fusable(dtype, N, C, F, k)) return hipErrorInvalidValue;
  const TilePlan pl = plan_tiles(2, EPI_STORE, N, C, C, F);
  auto go = [&](auto tag) {
    typedef decltype(tag) T;
    GemmParams<T> p = blank<T>();
    p.a1 = (const T*)h; p.lda1 = F; p.b1 = (const T*)wv; p.ldb1 = F; p.k1 = F;
    p.m = N; p.n = C; p.out = (T*)out; p.ldo = C; p.resid = (const T*)resid;
    p.cmb_rows = (const T*)rows; p.cmb_inds = inds; p.cmb_gates = (const T*)gates; p.cmb_k = k;
    return gemm_vs_run<T>(p, pl.t, EPI_COMBINE, false, false, s);
  };
  const hipError_t e = dtype == 1 ? go(f16{}) : go(bf16{});
  return mark(e, "cmix_value_combine", s);
}

bool value_sparse_fusable(int dtype, int N, int C, int F, int E, int r, int k, int kx) {
  if (dtype == 0 || k < 1 || k > kCombineMaxK || !vs_enabled()) return false;
  // one 128-column rank slice per routing rank (kx = 128, the VGPR-staged
  // 128x96 tile's 256-byte K slice), u chunks of 8 columns within one expert
  if (kx != 128 || E * r > kx || r % 8 || E > kSparseMaxE) return false;
  // (at least 3 base K slices: the rank slices' loads, two slices ahead, are
  // issued after the barrier that publishes the rank table)
  const TilePlan pl = plan_tiles(2, EPI_STORE, N, C, C, F + k * kx);
  return pl.t == 6 && F % 128 == 0 && F >= 3 * 128 && C % 96 == 0;
}

hipError_t launch_cmix_value_sparse(int dtype, const void* h, const void* wv, int F, const void* u, const void* bt,
                                    int kx, const int* inds, const void* gates, int E, int r, const void* resid,
                                    void* out, int N, int C, int k, hipStream_t s) {
  if (!value_sparse_fusable(dtype, N, C, F, E, r, k, kx)) return hipErrorInvalidValue;
  auto go = [&](auto tag) {
    typedef decltype(tag) T;
    GemmParams<T> p = blank<T>();
    p.a1 = (const T*)h; p.lda1 = F; p.b1 = (const T*)wv; p.ldb1 = F; p.k1 = F;
    p.a2 = (const T*)u; p.lda2 = kx; p.b2 = (const T*)bt; p.ldb2 = kx; p.k2 = k * kx;
    p.m = N; p.n = C; p.out = (T*)out; p.ldo = C; p.resid = (const T*)resid;
    p.cmb_inds = inds; p.cmb_gates = (const T*)gates; p.cmb_k = k;
    p.n_experts = E; p.rank = r;
    return gemm_vs_run<T>(p, 6, EPI_SPARSE, true, false, s);
  };
  const hipError_t e = dtype == 1 ? go(f16{}) : go(bf16{});
  return mark(e, "cmix_value_sparse", s);
}

// Grouped product: one tile per workgroup, no split K or persistent grid.
// The tile minimises waves x operand rows per tile (ceil(tiles / CUs) x
// (BM + BN)): these products are bound by each CU's operand loads, and a
// partial last wave costs as much as a full one.  Ties go to the larger
// tile.  Candidates (16-bit): 256x192, 256x128, 128x96 (K % 128 == 0),
// 128x128, 64x128, 64x64; fp32: 128x128, 64x64.
template <typename T, int EPI>
hipError_t dispatch_grouped(const GemmParams<T>& p, hipStream_t s) {
  auto fits = [&](int bn) { return p.n % bn == 0; };
  auto tiles = [&](int bm, int bn) { return ((p.m + bm - 1) / bm + p.grp_n) * (p.n / bn); };
  const int cus = num_cus();
  struct Cand { int bm, bn; bool ok; };
  const bool h = sizeof(T) == 2;
  const Cand cands[] = {{256, 192, h && fits(192)}, {256, 128, h && fits(128)},
                        {128, 96, h && fits(96) && p.k1 % 128 == 0}, {128, 128, fits(128)},
                        {64, 128, h && fits(128)}, {64, 64, fits(64)}};
  int best = -1;
  long long best_cost = 0;
  for (int i = 0; i < (int)(sizeof(cands) / sizeof(cands[0])); ++i) {
    if (!cands[i].ok) continue;
    const long long waves = (tiles(cands[i].bm, cands[i].bn) + cus - 1) / cus;
    const long long cost = waves * (cands[i].bm + cands[i].bn);
    if (best < 0 || cost < best_cost) {
      best = i;
      best_cost = cost;
    }
  }
  if (best < 0) return hipErrorInvalidValue;
  if constexpr (sizeof(T) == 2) {
    switch (best) {
      case 0: return run<T, 256, 192, 4, 2, 2, EPI, false, 32, 0, 128, false, false, true>(p, s, false);
      case 1: return run<T, 256, 128, 4, 2, 2, EPI, false, 32, 0, 128, false, false, true>(p, s, false);
      case 2: return run<T, 128, 96, 2, 2, 2, EPI, false, 16, 10, 256, false, false, true>(p, s, false);
      case 3: return run<T, 128, 128, 2, 2, 4, EPI, false, 32, 0, 128, false, false, true>(p, s, false);
      case 4: return run<T, 64, 128, 2, 2, 3, EPI, false, 32, 0, 128, false, false, true>(p, s, false);
      default: return run<T, 64, 64, 2, 2, 3, EPI, false, 32, 0, 128, false, false, true>(p, s, false);
    }
  } else {
    if (best == 3) return run<T, 128, 128, 2, 2, 3, EPI, false, 32, 0, 128, false, false, true>(p, s, false);
    return run<T, 64, 64, 2, 2, 3, EPI, false, 32, 0, 128, false, false, true>(p, s, false);
  }
}

// A given plan for the products of the backward (planned by
// backward_gemm_plan below), or the automatic one.
TilePlan gemm_nt_plan(int dtype, int m, int n, int k_total, int hint) {
  const int elem = dtype == 0 ? 4 : 2;
  TilePlan pl = plan_tiles(elem, EPI_STORE, m, n, n, k_total);
  // the hints replace only a split plan (products too small to fill the CUs)
  if (tile_override() != 0 || pl.t != 7) return pl;
  const int nkt = k_total / (128 / elem);
  if (hint == GEMM_HINT_NO_SPLIT && n % 64 == 0) {
    // short K (a few slices per tile): unsplit 128x64 tiles, no partials to reduce
    pl.t = 2;
    pl.ks = 1;
  } else if (hint == GEMM_HINT_SPLIT64 && n % 64 == 0) {
    // long K over a small output: 64x64 tiles, K split 8 ways (4 with fewer slices)
    pl.t = 7;
    pl.bn = 64;
    pl.ks = 1;
    for (int c : {8, 4, 2})
      if (nkt % c == 0 && nkt / c >= 2) {
        pl.ks = c;
        break;
      }
  }
  return pl;
}

hipError_t launch_grouped_gemm(int dtype, bool relu2, const void* a, int lda, const void* b, int ldb,
                               long long bstride, int k, int m, int n, const int* offsets, int n_groups, void* out,
                               int ldo, const char* name, hipStream_t s, const LossJob* loss) {
  RWKV_DISPATCH_DTYPE(dtype, T, {
    GemmParams<T> p = blank<T>();
    p.a1 = (const T*)a; p.lda1 = lda; p.b1 = (const T*)b; p.ldb1 = ldb; p.k1 = k;
    p.m = m; p.n = n; p.out = (T*)out; p.ldo = ldo; p.n_key = n;
    p.grp_off = offsets; p.grp_n = n_groups; p.grp_bstride = bstride;
    if (loss) p.loss = *loss;
    const hipError_t e = relu2 ? dispatch_grouped<T, EPI_KEY>(p, s) : dispatch_grouped<T, EPI_STORE>(p, s);
    return mark(e, name, s);
  });
  return hipSuccess;
}

hipError_t launch_gemm_grouped_k(int dtype, const void* a, int lda, const void* b, int ldb, const int* koff,
                                 int n_groups, int m, int n, void* out, int ldo, long long ostride, const char* name,
                                 hipStream_t s) {
  if (n % 64) return hipErrorInvalidValue;
  RWKV_DISPATCH_DTYPE(dtype, T, {
    GemmParams<T> p = blank<T>();
    p.a1 = (const T*)a; p.lda1 = lda; p.b1 = (const T*)b; p.ldb1 = ldb; p.k1 = 0;
    p.m = m; p.n = n; p.out = (T*)out; p.ldo = ldo; p.n_key = n;
    p.gk_off = koff; p.gk_n = n_groups; p.gk_ostride = ostride;
    hipError_t e;
    if (n % 128 == 0) {
      if constexpr (sizeof(T) == 2)
        e = run<T, 128, 128, 2, 2, 4, EPI_STORE, false, 32, 0, 128, false, false, false, false, true>(p, s, false);
      else
        e = run<T, 128, 128, 2, 2, 3, EPI_STORE, false, 32, 0, 128, false, false, false, false, true>(p, s, false);
    } else {
      e = run<T, 64, 64, 2, 2, 3, EPI_STORE, false, 32, 0, 128, false, false, false, false, true>(p, s, false);
    }
    return mark(e, name, s);
  });
  return hipSuccess;
}

size_t gemm_nt_partial_bytes(int dtype, int m, int n, int k_total, int hint) {
  const TilePlan pl = gemm_nt_plan(dtype, m, n, k_total, hint);
  return (pl.t == 7 || pl.t == 9) && pl.ks > 1 ? (size_t)pl.ks * m * n * sizeof(float) : 0;
}

hipError_t launch_gemm_nt(int dtype, const void* a1, int lda1, const void* b1, int ldb1, int k1, const void* a2,
                          int lda2, const void* b2, int ldb2, int k2, int m, int n, void* out, int ldo, float* part,
                          const char* name, hipStream_t s, int hint, int* deferred) {
  RWKV_DISPATCH_DTYPE(dtype, T, {
    GemmParams<T> p = blank<T>();
    p.part = part;
    p.a1 = (const T*)a1; p.lda1 = lda1; p.b1 = (const T*)b1; p.ldb1 = ldb1; p.k1 = k1;
    if (k2 > 0) { p.a2 = (const T*)a2; p.lda2 = lda2; p.b2 = (const T*)b2; p.ldb2 = ldb2; p.k2 = k2; }
    p.m = m; p.n = n; p.out = (T*)out; p.ldo = ldo; p.n_key = n;
    const TilePlan pl = gemm_nt_plan(dtype, m, n, k1 + (k2 > 0 ? k2 : 0), hint);
    const hipError_t e = k2 > 0 ? dispatch_tile<T, EPI_STORE, true>(p, s, &pl, deferred)
                                : dispatch_tile<T, EPI_STORE, false>(p, s, &pl, deferred);
    return mark(e, name, s);
  });
  return hipSuccess;
}

}  // namespace rwkvmoe
