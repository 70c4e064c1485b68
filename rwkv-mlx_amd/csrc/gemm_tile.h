// Pieces shared by the GEMM kernels of gemm.hip and gemm_vs.hip: the
// parameter block, the LDS row swizzle, the wait/barrier forms and the rule
// for where the output tile is staged.
#pragma once

#include "common.h"
#include "dispatch.h"
#include "losses.h"

namespace rwkvmoe {

// Epilogues: plain store; relu² (key); relu² on key columns and the gate mask
// on adapter columns n >= n_key (key with adapter tiles); residual add.
// EPI_COMBINE (SPARSE value product): out = round(base + δ) (+ residual)
// with δ the gate-weighted adapter rows of the token's experts, added in
// ascending expert id, each term rounded as combine_kernel rounds it
// (moe.py:138-147); the tile's base never leaves the chip.
// EPI_SPARSE (SPARSE value product with the adapters on chip): the same
// result with a_s itself computed in the launch: after the base's K slices,
// one K-extension slice per routing rank ρ (the token's ρ-th smallest expert
// id e) multiplies u = round(x·A_all) — the router's unscaled adapter
// product, masked to e's r columns — by B_all's columns of the tile, so the
// slice's accumulators hold x·A_e·B_e's fp32 sum, which is rounded
// (moe.py:142) and combined as above.
enum { EPI_STORE = 0, EPI_KEY = 1, EPI_RESID = 2, EPI_KEYAD = 3, EPI_COMBINE = 4, EPI_SPARSE = 5 };
// Slots per token the fused combine handles (top-k up to this).
constexpr int kCombineMaxK = 4;
// Experts the EPI_SPARSE rank slices handle (E·r within one 128-column slice
// with r >= 8).
constexpr int kSparseMaxE = 16;

template <typename T>
struct GemmParams {
  const T* a1; const T* b1; int k1; int lda1; int ldb1;   // segment 1
  const T* a2; const T* b2; int k2; int lda2; int ldb2;   // segment 2 (EXT only)
  int m, n;
  T* out; int ldo;
  const T* resid;   // (M, N) with stride ldo, EPI_RESID
  // EPI_KEYAD adapter tiles: columns n >= n_key
  int n_key;
  const T* a_ad;    // x (M, k1)
  const T* b_ad;    // A_all (n - n_key, k1)
  T* out_ad;        // U (M, n - n_key)
  const T* gmat;    // (M, n_experts) dense gates
  int n_experts, rank;
  LossJob loss;     // loss.losses != nullptr: the first workgroup to finish reduces the router's loss partials
  DispatchJob disp; // disp.nblk > 0: workgroups run the dispatch scatter's blocks by ticket after their tiles
  // split K: ksplit > 1 work items per tile, item s covering K slices
  // [s·nkt/ksplit, (s+1)·nkt/ksplit); each writes its fp32 partial tile to
  // part[s][m][n] and splitk_reduce_kernel sums them and applies the epilogue
  int ksplit;
  float* part;
  // grouped (GRP instances): rows are expert-contiguous segments
  // [grp_off[e], grp_off[e+1]) and segment e multiplies B + e·grp_bstride;
  // m is an upper bound on the rows (the launch covers every segment's tiles)
  const int* grp_off;
  int grp_n;
  long long grp_bstride;
  // grouped K (GK instances): output e (m x n at out + e·gk_ostride) sums
  // over the operand columns [gk_off[e], gk_off[e+1]), a multiple of the K
  // slice each and never empty; gk_n outputs
  const int* gk_off;
  int gk_n;
  long long gk_ostride;
  // rows of tiles per group of the XCD walk (0: 8), from walk_group_m
  int group_m;
  // EPI_COMBINE: the adapter rows of assignment t·cmb_k + s (N·k x n, row
  // stride ldo, the grouped LoRA's assignment order), the routing inds and
  // gates (N x k); resid, when set, is added after.  EPI_SPARSE reads the
  // same inds and gates (and rank = the LoRA rank r)
  const T* cmb_rows;
  const int* cmb_inds;
  const T* cmb_gates;
  int cmb_k;
};

// Rows of tiles per group of the XCD-contiguous tile walk.  The c tiles one
// XCD runs at once (c = its share of the tiles, at most one per CU of its
// 32) cover g row blocks x c/g column blocks, so its L2 fills g·BM + (c/g)·BN
// operand rows of K each; g minimises that (the larger g on a tie).
inline int walk_group_m(int tiles_m, int tiles_n, int BM, int BN) {
  const int total = tiles_m * tiles_n;
  if (total % 8) return 8;
  const int c = total / 8 < 32 ? total / 8 : 32;
  int best = 8, cost = 0x7fffffff;
  for (int g = 32; g >= 1; g >>= 1) {
    if (g > tiles_m || c % g || c / g > tiles_n) continue;
    const int f = g * BM + (c / g) * BN;
    if (f < cost) {
      cost = f;
      best = g;
    }
  }
  return best;
}

// The EPI_KEYAD adapter epilogue on 4 consecutive adapter columns n..n+3 of
// row gm (n a multiple of 4): U[gm, n+q] = w_e · r[q] with e = (n+q) / rank
// (moe.py:142-145), 0 on columns past the last expert.  With rank a multiple
// of 4 the 4 columns share one expert: one division and one gate load.
template <typename T>
RWKV_DEV void adapter_scale4(const GemmParams<T>& p, int gm, int n, float (&r)[4]) {
  const T* g = p.gmat + (size_t)gm * p.n_experts;
  if (p.rank % 4 == 0) {
    const int e = n / p.rank;
    const bool ok = e < p.n_experts;
    const float w = ok ? to_f(g[e]) : 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) r[q] = ok ? w * r[q] : 0.f;
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = (n + q) / p.rank;
      r[q] = e < p.n_experts ? to_f(g[e]) * r[q] : 0.f;
    }
  }
}

// relu² (model.py:262) of four fp32 accumulators of an fp16 key product,
// as four packed fp16: the accumulators rounded to fp16 in pairs (round to
// nearest even), max with 0, squared with one fp16 rounding.  These are the
// values of rounding each step through fp32 (the product of two fp16 values
// is exact in fp32, and fp16 subnormals are kept), at a third of the vector
// instructions of that form.
RWKV_DEV unsigned long long relu2_f16x4(float a0, float a1, float a2, float a3) {
  h16x2 lo = __builtin_convertvector((f32x2){a0, a1}, h16x2);
  h16x2 hi = __builtin_convertvector((f32x2){a2, a3}, h16x2);
  lo = __builtin_elementwise_max(lo, (h16x2){(f16)0, (f16)0});
  hi = __builtin_elementwise_max(hi, (h16x2){(f16)0, (f16)0});
  lo = lo * lo;
  hi = hi * hi;
  union {
    h16x2 v[2];
    unsigned long long u;
  } pk;
  pk.v[0] = lo;
  pk.v[1] = hi;
  return pk.u;
}

// The fused combine of one 16-byte output chunk (VEC elements of row gm at
// column col): out = round(base + δ), δ = round(δ + round(g_s · a_s)) over
// the routed slots s in ascending (expert, slot) order (combine_kernel's
// arithmetic), then the residual when p.resid is set.  The routing and the
// slots' row chunks are requested together: one memory round trip.
template <typename T>
RWKV_DEV u32x4 combine_chunk(const GemmParams<T>& p, int gm, int col, u32x4 base_raw) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int KM = kCombineMaxK;
  const int K = p.cmb_k;
  int ex[KM];
  float g[KM];
  Chunk<T> a[KM], rc;
#pragma unroll
  for (int s = 0; s < KM; ++s) {
    const int ss = s < K ? s : K - 1;  // (slots past k load slot k-1 and are dropped below)
    const size_t as = (size_t)gm * K + ss;
    ex[s] = p.cmb_inds[as];
    g[s] = to_f(p.cmb_gates[as]);
    a[s].raw = *(const u32x4*)(p.cmb_rows + as * p.ldo + col);
  }
  if (p.resid) rc.raw = *(const u32x4*)(p.resid + (size_t)gm * p.ldo + col);
  bool ok[KM];
#pragma unroll
  for (int s = 0; s < KM; ++s) ok[s] = s < K && ex[s] >= 0;  // (a negative id: an unrouted slot)
  int rk[KM];
#pragma unroll
  for (int s = 0; s < KM; ++s) {
    rk[s] = 0;
#pragma unroll
    for (int q = 0; q < KM; ++q) rk[s] += (ok[q] && (ex[q] < ex[s] || (ex[q] == ex[s] && q < s))) ? 1 : 0;
  }
  float d[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) d[i] = 0.f;
#pragma unroll
  for (int j = 0; j < KM; ++j) {
    Chunk<T> aj;
    aj.raw = zero4();
    float gj = 0.f;
    bool any = false;
#pragma unroll
    for (int s = 0; s < KM; ++s)
      if (ok[s] && rk[s] == j) {
        aj = a[s];
        gj = g[s];
        any = true;
      }
    if (any) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) d[i] = rnd<T>(d[i] + rnd<T>(gj * to_f(aj.e[i])));
    }
  }
  Chunk<T> b, o;
  b.raw = base_raw;
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    float v = rnd<T>(to_f(b.e[i]) + d[i]);
    if (p.resid) v = to_f(rc.e[i]) + v;
    o.e[i] = from_f<T>(v);
  }
  return o.raw;
}

// 16-byte chunk swizzle of an LDS row of RB bytes (RB/16 chunks); the result
// is always < RB/16.  Rows of 64 B: the 16 (row % 4, chunk) pairs of 16
// consecutive rows are distinct; rows of 128 B: distinct for rows r and r+8
// and for rows of either parity; rows of 256 B (a full 64-bank sweep each):
// distinct over any 16 consecutive rows.  Either way the 16 lanes of one LDS
// read phase hit distinct banks.
template <int RB>
RWKV_DEV int swz(int row) {
  static_assert(RB == 64 || RB == 128 || RB == 256, "LDS row size");
  if constexpr (RB == 64) return (row >> 2) & 3;
  else if constexpr (RB == 128) return (row ^ (row >> 3)) & 7;
  else return row & 15;
}

// Wait until at most n vector-memory operations of this wave are outstanding,
// then barrier.  Written as one asm statement with a memory clobber: the
// compiler may not move LDS accesses across it, and no workgroup fence (which
// would wait for every outstanding load) is emitted.
template <int N>
RWKV_DEV void wait_vm_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}
RWKV_DEV void wait_lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Asynchronous 16-byte copy per lane from the buffer r into LDS
// (buffer_load_dwordx4 ... lds): lane i's bytes land at dst + 16·i.  The
// MUBUF form is used rather than global_load_lds because the compiler counts
// that FLAT instruction against both the vector-memory and the LDS counters
// while it is outstanding, and then waits for every LDS read (lgkmcnt(0))
// before each MFMA that needs one; with the MUBUF form it waits for just the
// fragments an MFMA reads.  (The builtin sits in this non-template function:
// called directly from a kernel template's lambda, it made the host pass drop
// that kernel's launch stub.)
RWKV_DEV void buffer_load_lds16(__amdgpu_buffer_rsrc_t r, lds_ptr_t dst, unsigned off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, off, 0, 0, 0);
}

// s_waitcnt lgkmcnt(0) in the form the compiler's wait placement reads (an
// inline-asm wait is opaque to it): placed before a K loop, it keeps a scalar
// load still in flight from the prologue out of the loop's first LDS wait,
// which would otherwise have to be lgkmcnt(0) (scalar loads return out of
// order).  vmcnt and expcnt fields at their maximum: no wait on them.
RWKV_DEV void wait_scalar_loads() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Whether a tile config's output tile (elements of OT) is staged in LDS
// with unpadded rows, its 16-byte chunk index XOR-swizzled by row & 31 (for
// bank spread), instead of rows padded by 16 bytes: when only the unpadded
// tile fits in the operand ring (256x256 tiles with two 64 KB stages).
template <typename OT, int BM, int BN, int S, int RB>
constexpr bool out_swizzled() {
  constexpr int RING = S * (BM + BN) * RB;
  constexpr int PADDED = BM * (BN * (int)sizeof(OT) + 16);
  return RING < PADDED && RING >= BM * BN * (int)sizeof(OT) && RING + PADDED > 163840;
}

// Whether a tile config stages its output tile in the operand ring (the
// ring and a separate output tile would exceed 160 KB of LDS).  Such a
// workgroup can hold only one tile: the ring is overwritten by the epilogue.
template <typename OT, int BM, int BN, int S, int RB>
constexpr bool out_in_ring() {
  constexpr int RING = S * (BM + BN) * RB;
  constexpr int PADDED = BM * (BN * (int)sizeof(OT) + 16);
  return out_swizzled<OT, BM, BN, S, RB>() || (RING >= PADDED && RING + PADDED > 163840);
}

// The VGPR-staged form of tile code `tile` (gemm_vs.hip), or
// hipErrorNotSupported when that tile has none.
template <typename T>
hipError_t gemm_vs_run(const GemmParams<T>& p, int tile, int epi, bool ext, bool mx, hipStream_t s);

}  // namespace rwkvmoe
