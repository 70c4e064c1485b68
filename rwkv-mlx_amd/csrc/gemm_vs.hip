// VGPR-staged MFMA GEMM tiles for the layer's two large products (the key
// projection with relu², model.py:262, and the value projection with the
// adapter K-extension, model.py:263 / moe.py:139-147).
//
// Why a second form: a global_load_lds ring can only have as many K slices
// in flight as LDS holds free slots, and with two 57 KB slots a CU keeps
// one slice in flight while it computes the other — about 26 B/clk per CU
// at the loaded latency of a chip-wide stream.  Here load-only waves keep D
// slices in flight in their VGPRs (global_load_dwordx4) and write each one
// into a two-slot LDS ring (ds_write_b128) once its slot is free, so the
// bytes in flight no longer depend on LDS space.
//
// One tile per workgroup (the grid is the tile count, XCD-aware as in
// gemm.hip).  NMW = WGM·WGN MFMA waves, LW load waves.  K is walked in slices
// of RB bytes per row (BK = RB / sizeof(T) elements); a slice is the tile's BM
// A rows then BN B rows, NCH = (BM + BN)·RB / 16 chunks of 16 bytes, stored
// in LDS with the chunk index XOR-swizzled by row (swz<RB>) as the MFMA
// fragment reads expect.  Load-wave lane i (of LL = 64·LW) owns chunks
// i + j·LL, j < NPL.
//   load waves, iteration g: write slice g (held in registers) into slot
//     g % 2, issue the loads of slice g + D into the same registers, wait for
//     the LDS writes, barrier g;
//   MFMA waves, iteration g: barrier g, MFMAs on slot g % 2.
// Slot g % 2 is rewritten after barrier g - 1, which every MFMA wave reaches
// only after its reads of slice g - 2; its slice g is complete in LDS at
// barrier g.  Loads past the last slice are clamped to it (their values are
// never written), so every iteration has the same number of loads in
// flight.
#include <type_traits>

#include "common.h"
#include "gemm_tile.h"
#include "internal.h"

namespace rwkvmoe {
namespace {

template <typename T, int BM, int BN, int WGM, int WGN, int MN, int LW, int RB, int D, int EPI, bool EXT, bool MX>
__global__ __launch_bounds__(64 * (WGM * WGN + LW)) void gemm_vs_kernel(GemmParams<T> p) {
  static_assert(!MX || (EXT && (EPI == EPI_STORE || EPI == EPI_RESID)), "mixed value product");
  static_assert(EPI != EPI_COMBINE || (!EXT && !MX && sizeof(T) == 2), "fused combine: 16-bit SPARSE value product");
  static_assert(EPI != EPI_SPARSE || (EXT && !MX && sizeof(T) == 2), "rank slices: 16-bit SPARSE value product");
  constexpr bool SP = EPI == EPI_SPARSE;
  typedef typename std::conditional<MX, float, T>::type OT;  // output element
  using M = typename MmaSel<T, MN>::type;
  typedef typename M::frag frag;
  typedef typename M::acc accv;
  constexpr int NMW = WGM * WGN;
  constexpr int NT = 64 * (NMW + LW);
  static_assert(NT >= kDispThreads, "a dispatch job block needs 256 threads");
  constexpr int VEC = 16 / sizeof(T);
  constexpr int BK = RB / sizeof(T), CPR = RB / 16;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int MI = WM / MN, NI = WN / MN;
  constexpr int A_BYTES = BM * RB, STAGE = (BM + BN) * RB;
  constexpr int NCH = (BM + BN) * CPR, LL = 64 * LW, NPL = (NCH + LL - 1) / LL;
  constexpr int NKK = BK / M::KS;
  constexpr int OSTR = BN * (int)sizeof(OT) + 16;  // output tile row stride in LDS (bytes)
  constexpr int OUT_BYTES = BM * OSTR;
  constexpr bool OUT_IN_RING = 2 * STAGE + OUT_BYTES > 163840;
  constexpr int KM = kCombineMaxK;
  // EPI_SPARSE: gate of each tile row's rank ρ (fp32 [BM][KM]), then the
  // rank of each expert id < kSparseMaxE in the row (int8 [BM][kSparseMaxE],
  // -1: not routed)
  constexpr int GT_BYTES = SP ? BM * KM * 4 + BM * kSparseMaxE : 0;
  constexpr int LDS_BYTES = (OUT_IN_RING ? 2 * STAGE : 2 * STAGE + OUT_BYTES) + GT_BYTES;
  static_assert(MI >= 1 && NI >= 1 && MI * MN == WM && NI * MN == WN, "wave tile");
  static_assert(!OUT_IN_RING || 2 * STAGE >= OUT_BYTES, "output tile");
  static_assert(!SP || !OUT_IN_RING, "the rank slices keep the base in the output tile beside the ring");
  static_assert(LDS_BYTES <= 163840, "LDS budget");
  static_assert(256 + loss_scratch_bytes(NT) <= LDS_BYTES, "loss scratch");
  static_assert(D >= 2 && NPL * (D - 1) < 64, "loads in flight");
  static_assert(M::ACC % 4 == 0, "epilogue writes 4 accumulators at a time");

  __shared__ __attribute__((aligned(1024))) unsigned char lds[LDS_BYTES];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool mma_wave = wave < NMW;
  const int wm = mma_wave ? wave / WGN : 0, wn = mma_wave ? wave % WGN : 0;

  // this workgroup's tile: XCD x (= w % 8) owns a contiguous run of the
  // logical tiles, walked in groups of group_m M-tiles (walk_group_m)
  const int tiles_m = (p.m + BM - 1) / BM, tiles_n = p.n / BN;
  const int total = tiles_m * tiles_n, w = blockIdx.x;
  const int l = (total & 7) == 0 ? (w & 7) * (total >> 3) + (w >> 3) : w;
  const int GROUP_M = p.group_m > 0 ? p.group_m : 8;
  const int in_group = GROUP_M * tiles_n;
  const int first_m = (l / in_group) * GROUP_M;
  const int gsize = min(tiles_m - first_m, GROUP_M);
  const int m0 = (first_m + (l % in_group) % gsize) * BM;
  const int n0 = ((l % in_group) / gsize) * BN;
  const bool adapter = EPI == EPI_KEYAD && n0 >= p.n_key;

  const int nk1 = p.k1 / BK;
  const int G = nk1 + (EXT ? p.k2 / BK : 0);  // K slices (EPI_SPARSE: then one per rank)

  // EPI_SPARSE: rank of each routed slot of a row, by (expert id, slot) as
  // combine_chunk ranks them (unrouted slots, id < 0, take no rank)
  auto slot_ranks = [&](const int (&ex)[KM], int (&rk)[KM]) {
    const int K = p.cmb_k;
#pragma unroll
    for (int s = 0; s < KM; ++s) {
      rk[s] = -1;
      if (s < K && ex[s] >= 0) {
        rk[s] = 0;
#pragma unroll
        for (int q = 0; q < KM; ++q)
          rk[s] += (q < K && ex[q] >= 0 && (ex[q] < ex[s] || (ex[q] == ex[s] && q < s))) ? 1 : 0;
      }
    }
  };
  auto load_slots = [&](int gm, int (&ex)[KM], float (&gv)[KM]) {
    const int K = p.cmb_k;
#pragma unroll
    for (int s = 0; s < KM; ++s) {
      const size_t as = (size_t)gm * K + (s < K ? s : K - 1);
      ex[s] = p.cmb_inds[as];
      gv[s] = to_f(p.cmb_gates[as]);
    }
  };

  // ---- load waves ----------------------------------------------------------
  // A load lane's source rows, one per load and K segment, made once: a
  // slice's loads then only add its K offset (with the segments picked per
  // slice, the per-load address products stayed inside the loop and the
  // K-extension kernel ran ~1.4 us slower at 4096 x 768 x 3200)
  const T* src1[NPL];
  const T* src2[EXT ? NPL : 1];
  {
    const T* A = adapter ? p.a_ad : p.a1;
    const T* B = adapter ? p.b_ad + (size_t)(n0 - p.n_key) * p.ldb1 : p.b1 + (size_t)n0 * p.ldb1;
    const int lt = tid - 64 * NMW;
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int id = min(lt + j * LL, NCH - 1);
      const int row = id / CPR, c = id % CPR;
      const size_t ar = (size_t)min(m0 + row, p.m - 1);
      src1[j] = (row < BM ? A + ar * p.lda1 : B + (size_t)(row - BM) * p.ldb1) + c * VEC;
      if constexpr (EXT)
        src2[j] = (row < BM ? p.a2 + ar * p.lda2 : p.b2 + (size_t)(n0 + row - BM) * p.ldb2) + c * VEC;
    }
  }
  // EPI_SPARSE: a u chunk (8 columns, all of expert column / r: r is a
  // multiple of 8) enters rank slice ρ when its expert has rank ρ among the
  // row's routed slots (the rank table, written by the MFMA waves before
  // barrier 0; the rank slices' loads are issued after it); the routed
  // experts of a row are distinct (top-k), so a chunk enters at most one
  // rank slice.  Chunks outside their slice read 0 past the buffer's end.
  const float* gtab = (const float*)(lds + LDS_BYTES - GT_BYTES);
  const signed char* rtab = (const signed char*)(gtab + BM * KM);
  const __amdgpu_buffer_rsrc_t ubuf = buf_rsrc(SP ? (const void*)p.a2 : (const void*)p.a1,
                                               SP ? (unsigned)p.m * (unsigned)p.lda2 * (unsigned)sizeof(T) : 0u);
  auto issue = [&](u32x4 (&buf)[NPL], int g) {
    const bool seg2 = EXT && g >= nk1;
    if constexpr (SP) {
      // rank slice ρ: u chunks of rank ρ (others read 0 past the buffer's end)
      // and the tile's B_all columns, the same for every rank
      if (seg2) {
        const int rho = g - nk1;
        const int lt = tid - 64 * NMW;
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
          const int id = min(lt + j * LL, NCH - 1);
          const int row = id / CPR, c = id % CPR;
          if (row < BM) {
            const bool in = rtab[row * kSparseMaxE + c * VEC / p.rank] == rho;  // (rows past the last: -1)
            buf[j] = buf_load16(ubuf, in ? ((unsigned)(m0 + row) * (unsigned)p.lda2 + (unsigned)(c * VEC)) *
                                               (unsigned)sizeof(T)
                                         : kOOB);
          } else {
            buf[j] = *(const u32x4*)src2[j];
          }
        }
        return;
      }
    }
    const int kb = (seg2 ? g - nk1 : g) * BK;
#pragma unroll
    for (int j = 0; j < NPL; ++j) buf[j] = *(const u32x4*)((seg2 ? src2[EXT ? j : 0] : src1[j]) + kb);
  };
  auto put = [&](const u32x4 (&buf)[NPL], int slot) {
    const int lt = tid - 64 * NMW;
    unsigned char* base = lds + slot * STAGE;
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int id = lt + j * LL;
      if (NCH % LL == 0 || id < NCH) {
        const int row = id / CPR, c = id % CPR;
        const int r = row < BM ? row : row - BM;
        *(u32x4*)(base + (row < BM ? 0 : A_BYTES) + r * RB + ((c ^ swz<RB>(r)) << 4)) = buf[j];
      }
    }
  };

  // ---- MFMA waves ----------------------------------------------------------
  accv acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int v = 0; v < M::ACC; ++v) acc[i][j][v] = 0.f;
  auto frag_at = [](const unsigned char* base_, int row, int k) -> const frag* {
    const int byte = k * (int)sizeof(T);
    return (const frag*)(base_ + row * RB + (((byte >> 4) ^ swz<RB>(row)) << 4) + (byte & 15));
  };
  auto compute = [&](int slot) {
    const unsigned char* As = lds + slot * STAGE;
    const unsigned char* Bs = As + A_BYTES;
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
    }
  };

  // Both wave kinds run Gp = G rounded up to D iterations, one barrier each;
  // the last Gp - G move no data.  Every iteration of the load waves issues
  // the same loads, so the compiler's count of loads in flight is the same on
  // every path into the unrolled loop and its waits stay at (D - 1)·NPL.
  const int Gp = (G + D - 1) / D * D;
  if (!mma_wave) {
    u32x4 buf[D][NPL];
#pragma unroll
    for (int d = 0; d < D; ++d) issue(buf[d], min(d, G - 1));
    for (int g0 = 0; g0 < Gp; g0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const int g = g0 + d;
        if (g < G) put(buf[d], g & 1);
        issue(buf[d], min(g + D, G - 1));
        wait_lds_barrier();  // barrier g: slice g is in slot g % 2
      }
    }
  } else {
    // EPI_SPARSE: gate of each tile row's rank ρ (0 where the row has no
    // rank ρ) into LDS, read at the rank slices' ends; δ of this lane's
    // accumulator positions, packed as T
    float* gtw = (float*)(lds + LDS_BYTES - GT_BYTES);
    unsigned* rtw = (unsigned*)(gtw + BM * KM);
    unsigned long long dpk[SP ? MI : 1][SP ? NI : 1][SP ? M::ACC / 4 : 1];
    if constexpr (SP) {
      for (int row = tid; row < BM; row += 64 * NMW) {
        float gr[KM];
        int ex[KM], rk[KM];
#pragma unroll
        for (int q = 0; q < KM; ++q) {
          gr[q] = 0.f;
          rk[q] = -1;
        }
        if (m0 + row < p.m) {
          float gv[KM];
          load_slots(m0 + row, ex, gv);
          slot_ranks(ex, rk);
#pragma unroll
          for (int s = 0; s < KM; ++s)
#pragma unroll
            for (int q = 0; q < KM; ++q)
              if (rk[s] == q) gr[q] = gv[s];
        }
#pragma unroll
        for (int q = 0; q < KM; ++q) gtw[row * KM + q] = gr[q];
        // rank of each expert id in this row, 4 ids per word
#pragma unroll
        for (int w4 = 0; w4 < kSparseMaxE / 4; ++w4) {
          unsigned wv = 0;
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            int v = -1;
#pragma unroll
            for (int s = 0; s < KM; ++s)
              if (rk[s] >= 0 && ex[s] == w4 * 4 + b) v = rk[s];
            wv |= (unsigned)(v & 0xff) << (8 * b);
          }
          rtw[row * (kSparseMaxE / 4) + w4] = wv;
        }
      }
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
          for (int v = 0; v < M::ACC / 4; ++v) dpk[i][j][v] = 0ull;
    }
    for (int g = 0; g < Gp; ++g) {
      wait_lds_barrier();  // barrier g
      if (g >= G) continue;
      if constexpr (SP) {
        if (g == nk1) {
          // the base product is complete: round it to T into the output tile
          // (the epilogue's positions), then the accumulators start rank 0
          unsigned char* ot0 = lds + 2 * STAGE;
#pragma unroll
          for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j) {
              const int row = wm * WM + i * MN + (lane % MN);
#pragma unroll
              for (int v0 = 0; v0 < M::ACC; v0 += 4) {
                const int col = wn * WN + j * MN + acc_row_n<MN>(v0, lane);
                union { T e[4]; unsigned long long u; } pk;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                  pk.e[q] = from_f<T>(acc[i][j][v0 + q]);
                  acc[i][j][v0 + q] = 0.f;
                }
                *(unsigned long long*)(ot0 + row * OSTR + col * (int)sizeof(T)) = pk.u;
              }
            }
        }
      }
      if constexpr (MX) {
        // first K-extension slice: the base product is complete; round it to
        // T, the base's dtype (model.py:263), before the fp32 delta is added
        if (g == nk1) {
#pragma unroll
          for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j)
#pragma unroll
              for (int v = 0; v < M::ACC; ++v) acc[i][j][v] = rnd<T>(acc[i][j][v]);
        }
      }
      compute(g & 1);
      if constexpr (SP) {
        if (g >= nk1) {
          // end of rank slice ρ: a = round(x·A_e·B_e) (moe.py:142), then
          // δ = round(δ + round(g·a)) as combine_chunk adds it
          const int rho = g - nk1;
#pragma unroll
          for (int i = 0; i < MI; ++i) {
            const int row = wm * WM + i * MN + (lane % MN);
            const float gr = gtw[row * KM + rho];
#pragma unroll
            for (int j = 0; j < NI; ++j)
#pragma unroll
              for (int v0 = 0; v0 < M::ACC; v0 += 4) {
                union { T e[4]; unsigned long long u; } dd;
                dd.u = dpk[i][j][v0 / 4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                  const float a = rnd<T>(acc[i][j][v0 + q]);
                  dd.e[q] = from_f<T>(to_f(dd.e[q]) + rnd<T>(gr * a));
                  acc[i][j][v0 + q] = 0.f;
                }
                dpk[i][j][v0 / 4] = dd.u;
              }
          }
        }
      }
    }
    if constexpr (SP) {
      // out = round(base + δ) in the output tile, in place
      unsigned char* ot0 = lds + 2 * STAGE;
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) {
          const int row = wm * WM + i * MN + (lane % MN);
#pragma unroll
          for (int v0 = 0; v0 < M::ACC; v0 += 4) {
            const int col = wn * WN + j * MN + acc_row_n<MN>(v0, lane);
            unsigned long long* dst = (unsigned long long*)(ot0 + row * OSTR + col * (int)sizeof(T));
            union { T e[4]; unsigned long long u; } b, dd;
            b.u = *dst;
            dd.u = dpk[i][j][v0 / 4];
#pragma unroll
            for (int q = 0; q < 4; ++q) b.e[q] = from_f<T>(to_f(b.e[q]) + to_f(dd.e[q]));
            *dst = b.u;
          }
        }
    }
  }

  // ---- epilogue ------------------------------------------------------------
  int ticket = 1;
  if (p.loss.losses != nullptr && tid == 0) ticket = atomicAdd(p.loss.claim, 1);
  unsigned char* ot = OUT_IN_RING ? lds : lds + 2 * STAGE;
  if (OUT_IN_RING) wait_lds_barrier();  // every MFMA wave is done reading the ring
  if (mma_wave && !SP) {  // (EPI_SPARSE: the tile is already in LDS)
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int row = wm * WM + i * MN + (lane % MN);
#pragma unroll
        for (int v0 = 0; v0 < M::ACC; v0 += 4) {
          const int col = wn * WN + j * MN + acc_row_n<MN>(v0, lane);  // 4 consecutive columns
          unsigned char* dst = ot + row * OSTR + col * (int)sizeof(OT);
          if constexpr (MX) {  // fp32 out: the accumulators as they are
            *(f32x4*)dst = f32x4{acc[i][j][v0], acc[i][j][v0 + 1], acc[i][j][v0 + 2], acc[i][j][v0 + 3]};
          } else {
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
      }
  }
  wait_lds_barrier();
  {
    constexpr int OVEC = 16 / (int)sizeof(OT);  // output elements per 16-byte chunk
    constexpr int OCPR = BN / OVEC;
#pragma unroll
    for (int it = 0; it < (BM * OCPR + NT - 1) / NT; ++it) {
      const int id = tid + it * NT;
      if (id >= BM * OCPR) break;
      const int row = id / OCPR, c = (id % OCPR) * OVEC;
      const int gm = m0 + row;
      if (gm >= p.m) continue;
      u32x4 v = *(const u32x4*)(ot + row * OSTR + c * (int)sizeof(OT));
      if constexpr (MX) {
        if constexpr (EPI == EPI_RESID) {  // the residual (dtype T) added in fp32
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
      if constexpr (EPI == EPI_RESID || EPI == EPI_SPARSE) {
        if (EPI == EPI_RESID || p.resid) {
        Chunk<T> o, rr;
        o.raw = v;
        rr.raw = *(const u32x4*)(p.resid + (size_t)gm * p.ldo + n0 + c);
#pragma unroll
        for (int e = 0; e < VEC; ++e) o.e[e] = from_f<T>(to_f(rr.e[e]) + to_f(o.e[e]));
        v = o.raw;
        }
      }
      if constexpr (EPI == EPI_COMBINE) v = combine_chunk(p, gm, n0 + c, v);
      T* dstp = adapter ? p.out_ad + (size_t)gm * (p.n - p.n_key) + (n0 - p.n_key) + c
                        : p.out + (size_t)gm * p.ldo + n0 + c;
      *(u32x4*)dstp = v;
    }
  }
  // the router's loss reduction, by the workgroup that took ticket 0
  if (p.loss.losses != nullptr) {
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
  }
  // the SPARSE forward's dispatch scatter, block by block (after the tile:
  // the key product does not read it)
  dispatch_job_run(p.disp, (int*)lds + 1, (int*)(lds + 256));
}

template <typename T, int BM, int BN, int WGM, int WGN, int MN, int LW, int RB, int D, int EPI, bool EXT, bool MX>
hipError_t run_vs(const GemmParams<T>& p, hipStream_t s) {
  constexpr int BK = RB / (int)sizeof(T);
  if (p.k1 % BK || (EXT && p.k2 % BK) || p.n % BN || p.m < 1) return hipErrorInvalidValue;
  const int tiles = ((p.m + BM - 1) / BM) * (p.n / BN);
  GemmParams<T> q = p;
  q.group_m = walk_group_m((p.m + BM - 1) / BM, p.n / BN, BM, BN);
  launch_kernel((gemm_vs_kernel<T, BM, BN, WGM, WGN, MN, LW, RB, D, EPI, EXT, MX>), dim3(tiles),
                     dim3(64 * (WGM * WGN + LW)), 0, s, q);
  return hipGetLastError();
}

}  // namespace

// 256x128: 8 MFMA waves (4x2, 32x32 blocks), 8 load waves, 128-byte slices,
// two slices in flight per load lane.
template <typename T>
hipError_t run_vs_256x128(const GemmParams<T>& p, int epi, bool ext, hipStream_t s) {
  if (ext) {
    if (epi == EPI_RESID) return run_vs<T, 256, 128, 4, 2, 32, 8, 128, 2, EPI_RESID, true, false>(p, s);
    if (epi == EPI_STORE) return run_vs<T, 256, 128, 4, 2, 32, 8, 128, 2, EPI_STORE, true, false>(p, s);
    return hipErrorNotSupported;
  }
  if (epi == EPI_RESID) return run_vs<T, 256, 128, 4, 2, 32, 8, 128, 2, EPI_RESID, false, false>(p, s);
  if (epi == EPI_STORE) return run_vs<T, 256, 128, 4, 2, 32, 8, 128, 2, EPI_STORE, false, false>(p, s);
  if (epi == EPI_COMBINE) return run_vs<T, 256, 128, 4, 2, 32, 8, 128, 2, EPI_COMBINE, false, false>(p, s);
  if (epi == EPI_KEY) return run_vs<T, 256, 128, 4, 2, 32, 8, 128, 2, EPI_KEY, false, false>(p, s);
  if (epi == EPI_KEYAD) return run_vs<T, 256, 128, 4, 2, 32, 8, 128, 2, EPI_KEYAD, false, false>(p, s);
  return hipErrorNotSupported;
}

// Variant of a tile code (gemm.hip's numbering) in the VGPR-staged form;
// hipErrorNotSupported when there is none (the caller keeps the ring form).
//   6: 128x96, 4 MFMA waves (2x2, 16x16 blocks), 12 load waves, 256-byte slices
//      (the value product: 26.9 against 30.9 us in the ring form at 4096 x 768
//      x 3072; the 256x192 key tile measured slower in this form, 30.6
//      against 29.3 us, and keeps the ring).  Two slices in flight per load
//      lane: with the adapter K-extension at 4096 x 768 x 3200, 28.7-29.4 us
//      against 30.0-30.3 us with three, 30.6-31.1 with four and 30.6-31.5
//      with five; 8 load waves or 8 MFMA waves measured slower (30.9-37.4);
//      the fp32-adapter product too (30.5 against 31.2-32.0 us with three)
//   5: 256x128, 8 MFMA waves, 8 load waves (run_vs_256x128; against the ring
//      form: 615 / 554 against 732 / 706 us for the plain key / value products
//      at 16384 x 8192 x 2048 and 16384 x 2048 x 8192 bf16, 99 / 78 against
//      108 / 85 us at 8192 x 4096 x 1024 and 8192 x 1024 x 4096 fp16)
template <typename T>
hipError_t gemm_vs_run(const GemmParams<T>& p, int tile, int epi, bool ext, bool mx, hipStream_t s) {
  if constexpr (sizeof(T) != 2) {
    return hipErrorNotSupported;
  } else {
    if (tile == 5 && !mx && p.k1 % 64 == 0 && (!ext || p.k2 % 64 == 0)) return run_vs_256x128<T>(p, epi, ext, s);
    if (tile == 6 && (p.k1 % 128 == 0) && (!ext || p.k2 % 128 == 0)) {
      if (mx) {
        if (epi == EPI_RESID) return run_vs<T, 128, 96, 2, 2, 16, 12, 256, 2, EPI_RESID, true, true>(p, s);
        if (epi == EPI_STORE) return run_vs<T, 128, 96, 2, 2, 16, 12, 256, 2, EPI_STORE, true, true>(p, s);
        return hipErrorNotSupported;
      }
      if (ext) {
        if (epi == EPI_SPARSE) return run_vs<T, 128, 96, 2, 2, 16, 12, 256, 2, EPI_SPARSE, true, false>(p, s);
        if (epi == EPI_RESID) return run_vs<T, 128, 96, 2, 2, 16, 12, 256, 2, EPI_RESID, true, false>(p, s);
        if (epi == EPI_STORE) return run_vs<T, 128, 96, 2, 2, 16, 12, 256, 2, EPI_STORE, true, false>(p, s);
        return hipErrorNotSupported;
      }
      if (epi == EPI_RESID) return run_vs<T, 128, 96, 2, 2, 16, 12, 256, 2, EPI_RESID, false, false>(p, s);
      if (epi == EPI_STORE) return run_vs<T, 128, 96, 2, 2, 16, 12, 256, 2, EPI_STORE, false, false>(p, s);
      if (epi == EPI_COMBINE) return run_vs<T, 128, 96, 2, 2, 16, 12, 256, 2, EPI_COMBINE, false, false>(p, s);
    }
    return hipErrorNotSupported;
  }
}

template hipError_t gemm_vs_run<f16>(const GemmParams<f16>&, int, int, bool, bool, hipStream_t);
template hipError_t gemm_vs_run<bf16>(const GemmParams<bf16>&, int, int, bool, bool, hipStream_t);
template hipError_t gemm_vs_run<float>(const GemmParams<float>&, int, int, bool, bool, hipStream_t);

}  // namespace rwkvmoe
