// Expert adapters: operand preparation, grouped LoRA over routed rows,
// gate-weighted combine and the orthogonality loss
// (rwkv_mlx/moe.py:121-125, 138-147, 149-163).
#include <type_traits>

#include "common.h"
#include "internal.h"

namespace rwkvmoe {
namespace {

// ---- operand preparation ---------------------------------------------------
// A_all (Kx,C):  A_all[e*r + j][c] = lora_A[e][c][j]   (rows >= E*r are zero)
// B_all (C,Kx):  B_all[c][e*r + j] = lora_B[e][j][c]   (cols >= E*r are zero)
// Both put the reduction index innermost, the layout the MFMA operand loads
// want.  Each is a transpose of a (rows x cols) matrix viewed per expert
// ((C x r) -> (r x C) for A, (r x C) -> (C x r) for B) done through 32x32
// LDS tiles so reads and writes are both row-contiguous.
constexpr int kTp = 32;

// One launch prepares both operands: blockIdx.z == 0 writes A_all, 1 writes
// B_all, each 32x32 tile through LDS.
//   A_all[n][c] (n < kx, c < C) from A viewed as (E, C, r): A[(n/r)*C*r + c*r + n%r]
//   B_all[c][n] (c < C, n < kx) from B viewed as (E*r, C): B[n*C + c]
// MX (fp32 adapters, fp16 operands): every value v becomes the pair
// (hi, lo') of split_f16.  A_all then holds 2·kx rows, hi then lo' (in
// fragment order, the two passes of a K-step side by side: frag_pos2), and
// B_all has 3·kx columns [hi | lo' | hi]: with A-side operands
// [U_hi | 2^-11·U_hi | U_lo] the K-extension Σ U·B comes out as
// U_hi·B_hi + U_hi·(B - B_hi) + (U - U_hi)·B_hi.
template <typename TI, typename TO, bool MX>
__global__ __launch_bounds__(256) void lora_prep_kernel(const TI* __restrict__ A, const TI* __restrict__ B, int E,
                                                        int C, int r, int kx, int frag, TO* at, TO* bt) {
  __shared__ float tile[kTp][kTp + 1];
  const int c0 = blockIdx.x * kTp, n0 = blockIdx.y * kTp;
  const int tx = threadIdx.x % kTp, ty = threadIdx.x / kTp;  // 32 x 8
  if (blockIdx.z == 0) {
    for (int yy = ty; yy < kTp; yy += 8) {  // read: row c, column n (n contiguous within an expert)
      const int c = c0 + yy, n = n0 + tx;
      float v = 0.f;
      if (c < C && n < E * r) v = to_f(A[((size_t)(n / r) * C + c) * r + (n % r)]);
      tile[yy][tx] = v;
    }
    __syncthreads();
    for (int yy = ty; yy < kTp; yy += 8) {  // write: row n, column c
      const int n = n0 + yy, c = c0 + tx;
      if (n < kx && c < C) {
        if constexpr (MX) {
          f16 hi, lo;
          split_f16(tile[tx][yy], hi, lo);
          at[frag ? frag_pos2(n, c, C, 0) : (size_t)n * C + c] = hi;
          at[frag ? frag_pos2(n, c, C, 1) : (size_t)(kx + n) * C + c] = lo;
        } else {
          at[frag ? frag_pos(n, c, C) : (size_t)n * C + c] = from_f<TO>(tile[tx][yy]);
        }
      }
    }
  } else {
    for (int yy = ty; yy < kTp; yy += 8) {  // read: row n, column c (c contiguous)
      const int n = n0 + yy, c = c0 + tx;
      float v = 0.f;
      if (n < E * r && c < C) v = to_f(B[(size_t)n * C + c]);
      tile[yy][tx] = v;
    }
    __syncthreads();
    for (int yy = ty; yy < kTp; yy += 8) {  // write: row c, column n
      const int c = c0 + yy, n = n0 + tx;
      if (c < C && n < kx) {
        if constexpr (MX) {
          f16 hi, lo;
          split_f16(tile[tx][yy], hi, lo);
          TO* row = bt + (size_t)c * 3 * kx;
          row[n] = hi;
          row[kx + n] = lo;
          row[2 * kx + n] = hi;
        } else {
          bt[(size_t)c * kx + n] = from_f<TO>(tile[tx][yy]);
        }
      }
    }
  }
}

// ---- grouped LoRA -------------------------------------------------------------
// One workgroup (4 waves) per 32 routed rows of one expert e (rows j of perm
// order), reproducing the rounding points of (x @ A_e) @ B_e (moe.py:142):
//   0. every wave finds (e, first row) from offsets with one load per lane
//      and a wave-wide scan of the per-expert tile counts; the 32 token ids
//      (perm) are loaded before anything else, so the gathered x rows can be
//      requested after a single memory round trip;
//   1. u = round(x[perm[j]/k] · A_e)   (32 x r): the rows are staged in LDS
//      (KC columns at a time; one chunk covers d_model <= KC) with coalesced
//      16-byte loads while this wave's A_e fragments are already in flight;
//      the MFMA K-steps of a chunk are dealt round-robin over the 4 waves and
//      the 4 partial 32x32 blocks are added in wave order (a fixed order, so
//      the result does not depend on timing); columns n >= r are padding;
//   2. a = round(u · B_e)               (32 x C): each wave takes a contiguous
//      quarter of the columns, in passes of up to 6 32x32 MFMA blocks over
//      K = r (zero-padded to the MFMA depth) whose B_e fragments were loaded
//      at the start (later passes: during the previous pass's stores); a pass
//      is staged in the wave's own LDS and leaves as whole row segments with
//      coalesced 16-byte stores.
// LDS: the x chunk, then (reused) the 4 partial blocks, then (reused) the
// per-wave output staging; about 54 KB, so two workgroups fit on a CU.
constexpr int kLoraRows = 32;
constexpr int kLoraThreads = 256;

RWKV_DEV void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// MX (an fp16 layer with fp32 adapters, moe.py:124-125): A_all holds the
// fp16 pairs of A (2·kx rows: hi, then lo') and B_all those of B (3·kx
// columns: hi | lo' | hi).  Stage 1 adds (2^-11·x)·A_lo' to x·A_hi in the
// same fp32 accumulator, so u = x·A_e to about 22 bits (MLX: fp32); u is
// staged as [u_hi | 2^-11·u_hi | u - u_hi] and stage 2 runs over those three
// K-blocks against [B_hi | B_lo' | B_hi], so a = u·B_e comes out in fp32
// and the rows are written in fp32 (the delta's promoted dtype).
template <typename T, bool MX>
__global__ __launch_bounds__(kLoraThreads) void lora_grouped_kernel(const T* __restrict__ x,
                                                                    const T* __restrict__ at,
                                                                    const T* __restrict__ bt,
                                                                    const int* __restrict__ perm,
                                                                    const int* __restrict__ offsets, int N, int C,
                                                                    int E, int k, int r, int kx,
                                                                    typename std::conditional<MX, float, T>::type* ag) {
  static_assert(!MX || std::is_same<T, f16>::value, "fp16 pairs need an fp16 layer");
  typedef typename std::conditional<MX, float, T>::type OT;  // adapter rows
  using M = Mma32<T>;
  typedef typename M::frag frag;
  constexpr int KV = M::KV, KS = M::KS, VEC = 16 / sizeof(T), OVEC = 16 / sizeof(OT);
  constexpr int NP = MX ? 2 : 1;                   // A fragments per K-step (hi, lo')
  constexpr int KC = 1536 / sizeof(T);             // x columns staged per chunk (1.5 KB rows)
  constexpr int CPR = KC / VEC;                    // 16-byte chunks per staged row
  constexpr int XL = kLoraRows * CPR / kLoraThreads;  // x loads per thread per chunk
  constexpr int NSTEP = (KC / KS + 3) / 4;         // K-steps of a chunk per wave
  constexpr int XS = KC + VEC;                     // staged x row stride (elements)
  constexpr int UB = MX ? 3 : 1;                   // K-blocks of staged u (MX: hi, 2^-11·hi, lo)
  constexpr int US = UB * 32 + VEC;                // u row stride (elements)
  constexpr int PBLK = MX ? 3 : (sizeof(T) == 2 ? 6 : 3);  // 32-column blocks per stage-2 pass
  constexpr int NQ = 32 / KS;                      // most MFMA K-steps over r <= 32
  constexpr int OS = PBLK * 32 + OVEC;             // staged output row stride (elements)
  constexpr int X_BYTES = kLoraRows * XS * (int)sizeof(T);
  constexpr int R_BYTES = 4 * 32 * 33 * 4;
  constexpr int O_BYTES = 4 * kLoraRows * OS * (int)sizeof(OT);
  constexpr int BIG = X_BYTES > O_BYTES ? (X_BYTES > R_BYTES ? X_BYTES : R_BYTES) : (O_BYTES > R_BYTES ? O_BYTES : R_BYTES);
  static_assert(XL * kLoraThreads == kLoraRows * CPR, "x chunk loads");
  __shared__ __attribute__((aligned(16))) unsigned char big[BIG];
  __shared__ __attribute__((aligned(16))) T us[kLoraRows * US];
  __shared__ int tk[kLoraRows];
  __shared__ int ta[kLoraRows];  // the rows' assignment ids (where each row is stored)
  T* xs = (T*)big;      // stage 1
  float* red = (float*)big;  // stage 1 partials (after the MFMAs)
  OT* os = (OT*)big;    // stage 2

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nk = N * k;
  // 0. (expert, row block): lane ee holds expert ee's tile count; inclusive scan
  int e, row0, nrow;
  {
    int lo = 0, hi = 0;
    if (lane < E) {
      lo = offsets[lane];
      hi = offsets[lane + 1];
      lo = lo < 0 ? 0 : (lo > nk ? nk : lo);
      hi = hi < lo ? lo : (hi > nk ? nk : hi);
    }
    const int tiles = (hi - lo + kLoraRows - 1) / kLoraRows;
    int incl = tiles;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int v = __shfl_up(incl, d);
      if (lane >= d) incl += v;
    }
    const unsigned long long hit = __ballot((int)blockIdx.x < incl);
    if (hit == 0ull) return;  // the grid's spare workgroups
    const int ee = __builtin_ctzll(hit);
    e = __builtin_amdgcn_readfirstlane(ee);
    const int excl = __shfl(incl - tiles, e), elo = __shfl(lo, e), ehi = __shfl(hi, e);
    row0 = __builtin_amdgcn_readfirstlane(elo + ((int)blockIdx.x - excl) * kLoraRows);
    nrow = __builtin_amdgcn_readfirstlane(min(kLoraRows, ehi - row0));
  }
  const int lr = lane & 31, kh = lane >> 5;

  // token ids first: everything else waits behind them in the load queue
  int tok = -1, asg = -1;
  if (tid < kLoraRows && tid < nrow) {
    const int a = perm[row0 + tid];
    asg = (a >= 0 && a < nk) ? a : -1;
    tok = asg >= 0 ? a / k : -1;
  }

  // A_e fragments of this wave for the chunk at c0 (K-steps wave, wave+4, ...;
  // MX: hi rows e·r + n, then lo' rows kx + e·r + n)
  const bool n_ok = lr < r;
  const T* arow = at + (size_t)(e * r + (n_ok ? lr : 0)) * C;
  frag abuf[NSTEP][NP];
  auto load_a = [&](int c0) {
    const int kc = min(KC, C - c0);
#pragma unroll
    for (int i = 0; i < NSTEP; ++i) {
      const int sk = (wave + 4 * i) * KS;
#pragma unroll
      for (int q = 0; q < NP; ++q)
        abuf[i][q] = (n_ok && sk < kc) ? *(const frag*)(arow + (size_t)q * kx * C + c0 + sk + kh * KV) : frag{};
    }
  };
  // stage-2 B_e fragments (B_all rows c, columns e*r + kb ..; MX: and the lo'
  // block at kx + e*r + kb) for one pass
  const int rpad = (r + KS - 1) / KS * KS, nq = rpad / KS;
  const int cq = (C / 32 + 3) / 4 * 32;  // columns per wave (multiple of 32)
  const int cbeg = wave * cq, cend = min(C, cbeg + cq);
  const int ldb = MX ? 3 * kx : kx;
  frag bbuf[PBLK][NQ][NP];
  auto load_b = [&](int cb) {
#pragma unroll
    for (int b = 0; b < PBLK; ++b)
#pragma unroll
      for (int q = 0; q < NQ; ++q)
#pragma unroll
        for (int h = 0; h < NP; ++h) {
          union { frag f; T e[KV]; } fb;
          fb.f = frag{};
          const int c = cb + b * 32 + lr, kb = q * KS + kh * KV;
          if (q < nq && cb + b * 32 < cend) {
            const T* brow = bt + (size_t)c * ldb + h * kx + e * r;
            if (kb + KV <= r && ((e * r + kb) % KV) == 0) {
              fb.f = *(const frag*)(brow + kb);
            } else {
#pragma unroll
              for (int i = 0; i < KV; ++i) fb.e[i] = (kb + i < r) ? brow[kb + i] : from_f<T>(0.f);
            }
          }
          bbuf[b][q][h] = fb.f;
        }
  };
  load_a(0);
  if (cbeg < cend) load_b(cbeg);
  if (tid < kLoraRows) {
    tk[tid] = tok;  // -1: padding row (reads zeros, not stored)
    ta[tid] = asg;
  }
  lds_sync();

  // 1. u = x_rows · A_e
  f32x16 acc;
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] = 0.f;
  for (int c0 = 0; c0 < C; c0 += KC) {
    const int kc = min(KC, C - c0);
    if (c0 > 0) lds_sync();  // every wave is done with the previous chunk
    u32x4 xv[XL];
#pragma unroll
    for (int j = 0; j < XL; ++j) {
      const int i = tid + j * kLoraThreads, row = i / CPR, cc = (i % CPR) * VEC;
      const int t = tk[row];
      xv[j] = (t >= 0 && cc < kc) ? *(const u32x4*)(x + (size_t)t * C + c0 + cc) : zero4();
    }
#pragma unroll
    for (int j = 0; j < XL; ++j) {
      const int i = tid + j * kLoraThreads, row = i / CPR, cc = (i % CPR) * VEC;
      *(u32x4*)(xs + row * XS + cc) = xv[j];
    }
    lds_sync();
#pragma unroll
    for (int i = 0; i < NSTEP; ++i) {
      const int sk = (wave + 4 * i) * KS;
      if (sk < kc) {
        const frag xf = *(const frag*)(xs + lr * XS + sk + kh * KV);
        acc = M::run(xf, abuf[i][0], acc);
        if constexpr (MX) acc = M::run(xf * (T)kLoUnscale, abuf[i][1], acc);
      }
    }
    if (c0 + KC < C) load_a(c0 + KC);
  }
  lds_sync();  // every wave is done with xs: the partials reuse it
#pragma unroll
  for (int v = 0; v < 16; ++v) red[wave * 32 * 33 + acc_row(v, lane) * 33 + lr] = acc[v];
  lds_sync();
  for (int i = tid; i < kLoraRows * 32; i += kLoraThreads) {
    const int row = i >> 5, n = i & 31;
    const float sum = ((red[row * 33 + n] + red[32 * 33 + row * 33 + n]) + red[2 * 32 * 33 + row * 33 + n]) +
                      red[3 * 32 * 33 + row * 33 + n];
    const float uv = n < r ? sum : 0.f;  // columns >= r: zero K padding for step 2
    if constexpr (MX) {
      const T hi = (T)uv;
      us[row * US + n] = hi;
      us[row * US + 32 + n] = (T)((float)hi * kLoUnscale);
      us[row * US + 64 + n] = (T)(uv - (float)hi);
    } else {
      us[row * US + n] = from_f<T>(uv);
    }
  }
  lds_sync();  // u ready; the staging area is free for stage 2

  // 2. a = u · B_e, passes of PBLK column blocks per wave
  OT* ow = os + wave * kLoraRows * OS;
  for (int cb = cbeg; cb < cend; cb += PBLK * 32) {
    const int ob = min(PBLK * 32, cend - cb);
#pragma unroll
    for (int b = 0; b < PBLK; ++b) {
      if (b * 32 < ob) {
        f32x16 o;
#pragma unroll
        for (int v = 0; v < 16; ++v) o[v] = 0.f;
        // transposed block (B_e columns x rows): a lane holds 4 consecutive
        // output columns of row lr per accumulator group -> one 8-byte (16-bit
        // types) or 16-byte (fp32) LDS store each
#pragma unroll
        for (int q = 0; q < NQ; ++q)
          if (q < nq) {
            const T* ur = &us[lr * US + q * KS + kh * KV];
            o = M::run(bbuf[b][q][0], *(const frag*)ur, o);
            if constexpr (MX) {
              o = M::run(bbuf[b][q][1], *(const frag*)(ur + 32), o);  // (2^-11·u_hi)·B_lo'
              o = M::run(bbuf[b][q][0], *(const frag*)(ur + 64), o);  // (u - u_hi)·B_hi
            }
          }
#pragma unroll
        for (int v0 = 0; v0 < 16; v0 += 4) {
          union { OT e[4]; typename std::conditional<sizeof(OT) == 2, unsigned long long, u32x4>::type u; } pk;
#pragma unroll
          for (int q = 0; q < 4; ++q) pk.e[q] = from_f<OT>(o[v0 + q]);
          *(decltype(pk.u)*)(ow + lr * OS + b * 32 + acc_row(v0, lane)) = pk.u;
        }
      }
    }
    if (cb + PBLK * 32 < cend) load_b(cb + PBLK * 32);  // next pass's fragments in flight during the stores
    // the wave's staged rows -> global; the region is this wave's own, so
    // waiting for its LDS writes (and fencing the compiler) is enough
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const int cpw = ob / OVEC;  // chunks per staged row
    for (int i = lane; i < nrow * cpw; i += 64) {
      const int row = i / cpw, cc = (i % cpw) * OVEC, a = ta[row];
      if (a >= 0) *(u32x4*)(ag + (size_t)a * C + cb + cc) = *(const u32x4*)(ow + row * OS + cc);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the next pass overwrites
  }
}

// ---- grouped LoRA on the vector ALUs ------------------------------------------
// The same product and rounding points as lora_grouped_kernel (u =
// round(x[perm[j]/k] · A_e), a = round(u · B_e)) with dot products on the
// VALUs instead of MFMA blocks (r <= 32 pads to 32-wide MFMA blocks there):
// 16-bit operands take v_dot2_f32_{f16,bf16} (two products per instruction
// into an fp32 accumulator), fp32 ones fmaf.  A workgroup of 4 waves takes
// 32 routed rows of one expert:
//   1. u: thread (row = tid / 8, jg = tid % 8) holds u[row][jg + 8i]; x rows
//      and A_e rows are staged in LDS KC columns at a time; each thread walks
//      its columns in ascending order;
//   2. a: B_e is staged in LDS as column pairs of j (Bp[j/2][c][j%2]), so a
//      16-byte read gives 4 columns for two j; a thread writes 8 consecutive
//      columns of its row per 16-byte store, chunks cc = tid % 8 + 8i.
// Padding rows read zeros and are not written.
template <typename T>
__global__ __launch_bounds__(kLoraThreads) void lora_grouped_valu_kernel(const T* __restrict__ x,
                                                                         const T* __restrict__ at,
                                                                         const T* __restrict__ bt,
                                                                         const int* __restrict__ perm,
                                                                         const int* __restrict__ offsets, int N,
                                                                         int C, int E, int k, int r, int kx,
                                                                         T* __restrict__ ag) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr bool H = sizeof(T) == 2;
  constexpr int KC = 768 / sizeof(T);            // staged columns per chunk (768 B rows)
  constexpr int XS = KC + VEC;                   // staged row stride (elements)
  constexpr int CW = KC;                         // stage-2 columns per B_e chunk
  __shared__ __attribute__((aligned(16))) T xs[kLoraRows * XS];
  __shared__ __attribute__((aligned(16))) T as_[32 * XS];
  __shared__ float us[kLoraRows][33];
  __shared__ int tk[kLoraRows];
  __shared__ int ta[kLoraRows];  // the rows' assignment ids (where each row is stored)
  T* bp = as_;  // stage 2: Bp[j/2][c][2] over CW columns (16 · CW · 2 elements fit A_e's staging)
  static_assert(16 * CW * 2 <= 32 * XS, "stage-2 staging");

  const int tid = threadIdx.x, lane = tid & 63;
  const int nk = N * k;
  int e, row0, nrow;
  {  // (expert, row block) from the per-expert tile counts, as lora_grouped_kernel
    int lo = 0, hi = 0;
    if (lane < E) {
      lo = offsets[lane];
      hi = offsets[lane + 1];
      lo = lo < 0 ? 0 : (lo > nk ? nk : lo);
      hi = hi < lo ? lo : (hi > nk ? nk : hi);
    }
    const int tiles = (hi - lo + kLoraRows - 1) / kLoraRows;
    int incl = tiles;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int v = __shfl_up(incl, d);
      if (lane >= d) incl += v;
    }
    const unsigned long long hit = __ballot((int)blockIdx.x < incl);
    if (hit == 0ull) return;  // the grid's spare workgroups
    const int ee = __builtin_ctzll(hit);
    e = __builtin_amdgcn_readfirstlane(ee);
    const int excl = __shfl(incl - tiles, e), elo = __shfl(lo, e), ehi = __shfl(hi, e);
    row0 = __builtin_amdgcn_readfirstlane(elo + ((int)blockIdx.x - excl) * kLoraRows);
    nrow = __builtin_amdgcn_readfirstlane(min(kLoraRows, ehi - row0));
  }
  if (tid < kLoraRows) {
    int asg = -1;
    if (tid < nrow) {
      const int a = perm[row0 + tid];
      asg = (a >= 0 && a < nk) ? a : -1;
    }
    tk[tid] = asg >= 0 ? asg / k : -1;
    ta[tid] = asg;
  }
  __syncthreads();

  // 1. u = x_rows · A_e
  const int row = tid >> 3, jg = tid & 7;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  const int cpr = KC / VEC;
  for (int c0 = 0; c0 < C; c0 += KC) {
    const int kc = min(KC, C - c0);
    if (c0 > 0) __syncthreads();  // every thread is done with the previous chunk
    for (int i = tid; i < kLoraRows * cpr; i += kLoraThreads) {
      const int rr = i / cpr, cc = (i % cpr) * VEC, t = tk[rr];
      *(u32x4*)(xs + rr * XS + cc) = (t >= 0 && cc < kc) ? *(const u32x4*)(x + (size_t)t * C + c0 + cc) : zero4();
    }
    for (int i = tid; i < r * cpr; i += kLoraThreads) {
      const int j = i / cpr, cc = (i % cpr) * VEC;
      *(u32x4*)(as_ + j * XS + cc) = cc < kc ? *(const u32x4*)(at + (size_t)(e * r + j) * C + c0 + cc) : zero4();
    }
    __syncthreads();
    const T* xr = xs + row * XS;
    for (int c = 0; c < kc; c += VEC) {
      Chunk<T> xv;
      xv.raw = *(const u32x4*)(xr + c);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j = jg + 8 * q;
        if (j >= r) break;
        Chunk<T> av;
        av.raw = *(const u32x4*)(as_ + j * XS + c);
        if constexpr (H) {
#pragma unroll
          for (int v = 0; v < VEC; v += 2) {
            typedef T t2 __attribute__((ext_vector_type(2)));
            const t2 xa = {xv.e[v], xv.e[v + 1]}, aa = {av.e[v], av.e[v + 1]};
            if constexpr (std::is_same<T, f16>::value) acc[q] = __builtin_amdgcn_fdot2(xa, aa, acc[q], false);
            else acc[q] = __builtin_amdgcn_fdot2_f32_bf16(xa, aa, acc[q], false);
          }
        } else {
#pragma unroll
          for (int v = 0; v < VEC; ++v) acc[q] = __builtin_fmaf(to_f(xv.e[v]), to_f(av.e[v]), acc[q]);
        }
      }
    }
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int j = jg + 8 * q;
    if (j < r) us[row][j] = rnd<T>(acc[q]);
  }
  const int rp = (r + 1) / 2;  // j pairs (the last padded with 0 for odd r)
  if (tid < kLoraRows && (r & 1)) us[tid][r] = 0.f;

  // 2. a = u · B_e, B_e staged as j pairs over CW columns at a time
  for (int cb = 0; cb < C; cb += CW) {
    const int cw = min(CW, C - cb);
    __syncthreads();  // u complete / the previous B chunk no longer read
    for (int i = tid; i < cw * rp; i += kLoraThreads) {
      const int c = i / rp, jp = i % rp;
      const T* br = bt + (size_t)(cb + c) * kx + e * r;
      const int j0 = 2 * jp;
      bp[(jp * CW + c) * 2] = br[j0];
      bp[(jp * CW + c) * 2 + 1] = j0 + 1 < r ? br[j0 + 1] : from_f<T>(0.f);
    }
    __syncthreads();
    const int nch = cw / VEC;
    for (int ch = jg; ch < nch; ch += 8) {
      float o[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) o[v] = 0.f;
      for (int jp = 0; jp < rp; ++jp) {
        const float u0 = us[row][2 * jp], u1 = us[row][2 * jp + 1];
        const T* bq = bp + ((size_t)jp * CW + ch * VEC) * 2;
        // 2·VEC elements: VEC columns x (j0, j0 + 1)
#pragma unroll
        for (int h = 0; h < 2 * VEC; h += VEC) {
          Chunk<T> bv;
          bv.raw = *(const u32x4*)(bq + h);
#pragma unroll
          for (int v = 0; v < VEC; v += 2) {
            const int col = (h + v) / 2;
            if constexpr (H) {
              typedef T t2 __attribute__((ext_vector_type(2)));
              const t2 uu = {from_f<T>(u0), from_f<T>(u1)}, bb = {bv.e[v], bv.e[v + 1]};
              if constexpr (std::is_same<T, f16>::value) o[col] = __builtin_amdgcn_fdot2(uu, bb, o[col], false);
              else o[col] = __builtin_amdgcn_fdot2_f32_bf16(uu, bb, o[col], false);
            } else {
              o[col] = __builtin_fmaf(u0, to_f(bv.e[v]), o[col]);
              o[col] = __builtin_fmaf(u1, to_f(bv.e[v + 1]), o[col]);
            }
          }
        }
      }
      if (row < nrow && ta[row] >= 0) {
        Chunk<T> ov;
#pragma unroll
        for (int v = 0; v < VEC; ++v) ov.e[v] = from_f<T>(o[v]);
        *(u32x4*)(ag + (size_t)ta[row] * C + cb + ch * VEC) = ov.raw;
      }
    }
  }
}

// ---- combine -----------------------------------------------------------------
// out[t] = round(base[t] + δ[t]) (+ residual), δ accumulated over the token's
// experts in ascending id: δ = round(δ + round(w_e · a_e)) (moe.py:138-147).
// T: base, gates and residual; OT: adapter rows, δ and out (fp32 for an fp16
// layer with fp32 adapters, MLX's promoted dtype; else T).
// One thread per 16-byte chunk of an output row, K (= top-k) a template
// argument so every slot is unrolled.  BY_ASSIGN: the rows of assignment
// t·K + s sit at that index (the grouped LoRA's layout), so the base and
// residual chunks, the token's routing and all K row chunks are requested
// together: one memory round trip.  Otherwise (the full-expert layer's rows,
// in perm order) the rows sit at inv[t·K + s], which is requested with the
// base first, then the K row chunks (clamped addresses, zeroed afterwards
// if the slot is not routed): two round trips whatever K is.
template <typename X, int NV>
struct Elems {  // NV elements of X loaded / stored as one 8- or 16-byte access
  static constexpr int BYTES = NV * (int)sizeof(X);
  typedef typename std::conditional<BYTES == 16, u32x4, unsigned long long>::type raw_t;
  union {
    raw_t raw;
    X e[NV];
  };
  RWKV_DEV void load(const X* p) { raw = *(const raw_t*)p; }
  RWKV_DEV void zero() { raw = raw_t{}; }
};

template <typename T, typename OT, int K, bool BY_ASSIGN>
__global__ __launch_bounds__(256) void combine_kernel(const T* __restrict__ base, const OT* __restrict__ ag,
                                                      const int* __restrict__ inds, const T* __restrict__ gates,
                                                      const int* __restrict__ inv, const T* __restrict__ resid,
                                                      OT* out, int N, int C) {
  constexpr int VEC = 16 / sizeof(OT);
  const int cpr = C / VEC;
  const int chunk = blockIdx.x * blockDim.x + threadIdx.x;  // N * cpr < 2^31 (checked by the caller)
  if (chunk >= N * cpr) return;
  const int t = chunk / cpr, c = (chunk - t * cpr) * VEC;
  const int nk = N * K;

  Elems<T, VEC> b, rc;
  if (base) b.load(base + (size_t)t * C + c);  // no base: the full-expert layer
  else b.zero();
  if (resid) rc.load(resid + (size_t)t * C + c);
  int ex[K], pos[K];
  float g[K];
#pragma unroll
  for (int s = 0; s < K; ++s) {
    ex[s] = inds[(size_t)t * K + s];
    pos[s] = BY_ASSIGN ? t * K + s : inv[(size_t)t * K + s];
    g[s] = to_f(gates[(size_t)t * K + s]);
  }
  Elems<OT, VEC> a[K];
  bool ok[K];
#pragma unroll
  for (int s = 0; s < K; ++s) {
    ok[s] = BY_ASSIGN ? ex[s] >= 0 : (pos[s] >= 0 && pos[s] < nk);  // (a negative id: an unrouted slot)
    a[s].load(ag + (size_t)(BY_ASSIGN || ok[s] ? pos[s] : 0) * C + c);
  }
  // rank of each routed slot in ascending (expert, slot) order
  int rk[K];
#pragma unroll
  for (int s = 0; s < K; ++s) {
    rk[s] = 0;
#pragma unroll
    for (int q = 0; q < K; ++q)
      rk[s] += (ok[q] && (ex[q] < ex[s] || (ex[q] == ex[s] && q < s))) ? 1 : 0;
  }
  float d[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) d[i] = 0.f;
#pragma unroll
  for (int j = 0; j < K; ++j) {
    // the slot of rank j (if any)
    Elems<OT, VEC> aj;
    aj.zero();
    float gj = 0.f;
    bool any = false;
#pragma unroll
    for (int s = 0; s < K; ++s)
      if (ok[s] && rk[s] == j) {
        aj = a[s];
        gj = g[s];
        any = true;
      }
    if (any) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) d[i] = rnd<OT>(d[i] + rnd<OT>(gj * to_f(aj.e[i])));
    }
  }
  Elems<OT, VEC> o;
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    float v = rnd<OT>(to_f(b.e[i]) + d[i]);
    if (resid) v = to_f(rc.e[i]) + v;
    o.e[i] = from_f<OT>(v);
  }
  *(u32x4*)(out + (size_t)t * C + c) = o.raw;
}

// ---- orthogonality loss ------------------------------------------------------
// part[p] = Σ_{a,b} round(round((A_iᵀA_j)[a,b])²) for pair p = (i<j), one
// workgroup per pair; the final sum runs over pairs in (i, j) order.
template <typename T>
__global__ __launch_bounds__(256) void ortho_pair_kernel(const T* __restrict__ A, int E, int C, int r, float* part) {
  __shared__ float sq[256];
  int p = blockIdx.x, i = 0;
  while (p >= E - 1 - i) { p -= E - 1 - i; ++i; }
  const int j = i + 1 + p;
  const T* Ai = A + (size_t)i * C * r;
  const T* Aj = A + (size_t)j * C * r;
  float local = 0.f;
  for (int ab = threadIdx.x; ab < r * r; ab += 256) {
    const int a = ab / r, b = ab % r;
    float s = 0.f;
    for (int c = 0; c < C; ++c) s += to_f(Ai[(size_t)c * r + a]) * to_f(Aj[(size_t)c * r + b]);
    const float cr = rnd<T>(s);
    local += rnd<T>(cr * cr);
  }
  sq[threadIdx.x] = local;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.f;
    for (int t = 0; t < 256; ++t) s += sq[t];
    part[blockIdx.x] = s;
  }
}

__global__ void ortho_final_kernel(const float* part, int np, float* out) {
  if (threadIdx.x == 0) {
    float s = 0.f;
    for (int p = 0; p < np; ++p) s += part[p];
    out[0] = s;
  }
}

}  // namespace

int lora_kx(int E, int r) { return (E * r + 127) / 128 * 128; }

hipError_t launch_lora_prep(int dtype, const void* A, const void* B, int E, int C, int r, int kx, void* at, void* bt,
                            hipStream_t s, bool frag, bool mixed) {
  if (frag && (dtype == 0 || kx % 16 || C % 32)) return hipErrorInvalidValue;
  if (mixed && dtype != 1) return hipErrorInvalidValue;
  const dim3 grid((C + kTp - 1) / kTp, (kx + kTp - 1) / kTp, 2);
  if (mixed) {
    launch_kernel((lora_prep_kernel<float, f16, true>), grid, dim3(256), 0, s, (const float*)A, (const float*)B, E,
                       C, r, kx, frag ? 1 : 0, (f16*)at, (f16*)bt);
    return mark(hipGetLastError(), "lora_prep", s);
  }
  RWKV_DISPATCH_DTYPE(dtype, T, {
    launch_kernel((lora_prep_kernel<T, T, false>), grid, dim3(256), 0, s, (const T*)A, (const T*)B, E, C, r, kx,
                       frag ? 1 : 0, (T*)at, (T*)bt);
  });
  return mark(hipGetLastError(), "lora_prep", s);
}

hipError_t launch_lora_grouped(int dtype, const void* x, const void* at, const void* bt, const int* perm,
                               const int* offsets, int N, int C, int E, int k, int r, int kx, void* ag, hipStream_t s,
                               bool mixed, bool valu) {
  const int grid = (N * k + kLoraRows - 1) / kLoraRows + E;  // Σ_e ceil(n_e/32) <= this
  if (valu) {
    if (mixed || r > 32) return hipErrorInvalidValue;
    RWKV_DISPATCH_DTYPE(dtype, T, {
      launch_kernel(lora_grouped_valu_kernel<T>, dim3(grid), dim3(kLoraThreads), 0, s, (const T*)x, (const T*)at,
                         (const T*)bt, perm, offsets, N, C, E, k, r, kx, (T*)ag);
    });
    return mark(hipGetLastError(), "lora_grouped", s);
  }
  if (mixed) {
    if (dtype != 1) return hipErrorInvalidValue;
    launch_kernel((lora_grouped_kernel<f16, true>), dim3(grid), dim3(kLoraThreads), 0, s, (const f16*)x,
                       (const f16*)at, (const f16*)bt, perm, offsets, N, C, E, k, r, kx, (float*)ag);
    return mark(hipGetLastError(), "lora_grouped", s);
  }
  RWKV_DISPATCH_DTYPE(dtype, T, {
    launch_kernel((lora_grouped_kernel<T, false>), dim3(grid), dim3(kLoraThreads), 0, s, (const T*)x,
                       (const T*)at, (const T*)bt, perm, offsets, N, C, E, k, r, kx, (T*)ag);
  });
  return mark(hipGetLastError(), "lora_grouped", s);
}

namespace {
template <typename T, typename OT>
hipError_t combine_k(const void* base, const void* ag, const int* inds, const void* gates, const int* inv,
                     const void* resid, void* out, int N, int C, int k, hipStream_t s) {
  const size_t chunks = (size_t)N * (C / (16 / sizeof(OT)));
  const int grid = (int)((chunks + 255) / 256);
  if (grid == 0) return hipSuccess;
  auto go = [&](auto kern) {
    launch_kernel(kern, dim3(grid), dim3(256), 0, s, (const T*)base, (const OT*)ag, inds, (const T*)gates, inv,
                       (const T*)resid, (OT*)out, N, C);
  };
  // inv == NULL: rows in assignment order (the grouped LoRA's)
  auto pick = [&](auto kk) {
    constexpr int K = decltype(kk)::value;
    if (inv) go(combine_kernel<T, OT, K, false>);
    else go(combine_kernel<T, OT, K, true>);
  };
  switch (k) {
    case 1: pick(std::integral_constant<int, 1>{}); break;
    case 2: pick(std::integral_constant<int, 2>{}); break;
    case 3: pick(std::integral_constant<int, 3>{}); break;
    case 4: pick(std::integral_constant<int, 4>{}); break;
    case 5: pick(std::integral_constant<int, 5>{}); break;
    case 6: pick(std::integral_constant<int, 6>{}); break;
    case 7: pick(std::integral_constant<int, 7>{}); break;
    case 8: pick(std::integral_constant<int, 8>{}); break;
    default: return hipErrorInvalidValue;
  }
  return hipSuccess;
}
}  // namespace

hipError_t launch_combine(int dtype, const void* base, const void* ag, const int* inds, const void* gates,
                          const int* inv, const void* resid, void* out, int N, int C, int k, hipStream_t s,
                          bool mixed) {
  hipError_t e;
  if (mixed) {
    if (dtype == 1) e = combine_k<f16, float>(base, ag, inds, gates, inv, resid, out, N, C, k, s);
    else if (dtype == 2) e = combine_k<bf16, float>(base, ag, inds, gates, inv, resid, out, N, C, k, s);
    else return hipErrorInvalidValue;
  } else {
    switch (dtype) {
      case 0: e = combine_k<float, float>(base, ag, inds, gates, inv, resid, out, N, C, k, s); break;
      case 1: e = combine_k<f16, f16>(base, ag, inds, gates, inv, resid, out, N, C, k, s); break;
      case 2: e = combine_k<bf16, bf16>(base, ag, inds, gates, inv, resid, out, N, C, k, s); break;
      default: return hipErrorInvalidValue;
    }
  }
  if (e != hipSuccess) return e;
  return mark(hipGetLastError(), "combine", s);
}

namespace {
// y = fp32(x), n elements (n % 8 == 0), 16-bit x: exact
template <typename T>
__global__ __launch_bounds__(256) void widen_kernel(const T* __restrict__ x, float* __restrict__ y, size_t n8) {
  const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i >= n8) return;
  Chunk<T> c;
  c.raw = *(const u32x4*)(x + i * 8);
  f32x4 a, b;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a[j] = to_f(c.e[j]);
    b[j] = to_f(c.e[4 + j]);
  }
  *(f32x4*)(y + i * 8) = a;
  *(f32x4*)(y + i * 8 + 4) = b;
}
}  // namespace

hipError_t launch_widen(int dtype, const void* x, float* y, size_t n, hipStream_t s) {
  if (n % 8 || n == 0) return n == 0 ? hipSuccess : hipErrorInvalidValue;
  const size_t n8 = n / 8;
  const dim3 grid((unsigned)((n8 + 255) / 256));
  if (dtype == 1)
    launch_kernel(widen_kernel<f16>, grid, dim3(256), 0, s, (const f16*)x, y, n8);
  else if (dtype == 2)
    launch_kernel(widen_kernel<bf16>, grid, dim3(256), 0, s, (const bf16*)x, y, n8);
  else
    return hipErrorInvalidValue;
  return mark(hipGetLastError(), "widen", s);
}

hipError_t launch_ortho(int dtype, const void* A, int E, int C, int r, float* part, float* out, hipStream_t s) {
  const int np = E * (E - 1) / 2;
  RWKV_DISPATCH_DTYPE(dtype, T, {
    if (np > 0) {
      launch_kernel(ortho_pair_kernel<T>, dim3(np), dim3(256), 0, s, (const T*)A, E, C, r, part);
      const hipError_t e = mark(hipGetLastError(), "ortho_pairs", s);
      if (e != hipSuccess) return e;
    }
  });
  launch_kernel(ortho_final_kernel, dim3(1), dim3(64), 0, s, part, np, out);
  return mark(hipGetLastError(), "ortho_final", s);
}

}  // namespace rwkvmoe
