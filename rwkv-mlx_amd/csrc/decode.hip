// Decode value launch: the value projection of a few tokens (N <= 64, a
// decode step of a batch of sequences) with the FUSED adapter K-extension,
//   out = h · W_valueᵀ + U · B_allᵀ (+ residual)        model.py:263, moe.py:139-147
//   U[t, e·r + j] = w_{t,e} · u[t, e·r + j],  u = x · A_allᵀ (decode front)
// in one launch with no workspace of its own.
//
// A workgroup computes one 16-token x 16-column output tile over the whole
// K = F + Kx: its 16 waves take the K-steps in turn (wave w: steps w, w+16,
// ...), each with up to kVCh steps of fragments in flight straight from
// global memory, and the 16 fp32 partial blocks are summed through LDS in
// ascending wave order — a fixed order, so results do not depend on timing —
// then rounded once to the element type, with the residual added after.  For
// the adapter steps the gate is applied to u as its fragment arrives
// (rounded as the FUSED router's U: round(w · u)); the router writes the
// gate of every adapter column in u's layout, so it arrives the same way.  The token blocks of one
// column tile get workgroup ids of one residue mod 8, i.e. one XCD under
// round-robin dispatch, so that XCD's L2 serves their shared W_value rows
// (placement affects speed only).  One more workgroup, past the tiles,
// reduces the router's loss partials (complete: the router ran in the
// previous launch).
//
// Operand layouts: h and u come from the decode front in fragment order
// (frag_pos: one 1 KB block per 16 rows and K-step, a wave's load is one
// contiguous KB); W_value is read in fragment order too when the caller has
// laid it out once (rwkvmoe_prepare_base), else as fragments of the
// row-major matrix (16 rows per load: about half the load throughput).
#include "common.h"
#include "internal.h"
#include "losses.h"

namespace rwkvmoe {
namespace {

constexpr int kVWaves = 16, kVThreads = 64 * kVWaves, kVCh = 8;

template <typename T>
struct DecodeValue {
  const T* h;      // (16·nb, F) fragment order
  const T* wv;     // (C, F) row-major, or fragment order with `wpk`
  const T* u;      // (16·nb, kx) x · A_allᵀ, fragment order
  const T* g;      // (16·nb, kx) the gate of each adapter column, fragment order (rows < N)
  const T* bt;     // (C, kx)
  const T* resid;  // (N, C) or null
  T* out;          // (N, C)
  int N, C, F, kx, nb, nct, wpk;  // nb token blocks, nct column tiles
  int ntile;                             // workgroups of the tile mapping (the loss workgroup follows)
  LossJob loss;
};

// One 16-bit matrix (R x K, row-major, R % 16 == 0, K % 32 == 0) to fragment
// order (frag_pos); thread i moves the 16 bytes that land at 16·i.
template <typename T>
__global__ __launch_bounds__(256) void frag_pack_kernel(const T* __restrict__ src, T* __restrict__ dst, int R, int K) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t n = (size_t)R * K / 8;
  if (i >= n) return;
  const int lane = (int)(i & 63);
  const size_t blk = i >> 6, nks = K / 32;
  const int row = (int)(blk / nks) * 16 + (lane & 15);
  const int col = (int)(blk % nks) * 32 + (lane >> 4) * 8;
  *(u32x4*)(dst + i * 8) = *(const u32x4*)(src + (size_t)row * K + col);
}

template <typename T>
__global__ __launch_bounds__(kVThreads) void decode_value_kernel(DecodeValue<T> p) {
  using M = Mma16<T>;
  typedef typename M::frag frag;
  __shared__ f32x4 red[kVWaves][64];
  // the argument lines at offsets 0x00 (h), 0x40 (kx), 0x80 (loss.claim)
  RWKV_KERNARG_LINES("s"(p.h), "s"(p.kx), "s"(p.loss.claim));
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = blockIdx.x, rr = b >> 3;
  if (b >= p.ntile) {  // the loss workgroup
    __shared__ double sp_[kVThreads];
    __shared__ long long sc_[kVThreads];
    __shared__ double fe_[kLossMaxE + 1];
    reduce_losses(p.loss, sp_, sc_, fe_);
    return;
  }
  const int tb = rr % p.nb, ct = (rr / p.nb) * 8 + (b & 7);
  if (ct >= p.nct) return;  // padding of the id mapping; the whole workgroup
  const int c0 = ct * 16, t0 = tb * 16;
  const int wrow = c0 + (lane & 15);                      // W_value / B_all row (output column)
  const int kh = (lane >> 4) * M::KV;
  const int nk1 = p.F / M::KS, nku = p.kx / M::KS, steps = nk1 + nku;
  const bool tok_ok = t0 + (lane & 15) < p.N;  // rows past N: U is 0 whatever the gate rows hold
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = wave; s0 < steps; s0 += kVWaves * kVCh) {
    frag wf[kVCh], xf[kVCh], gf[kVCh];
#pragma unroll
    for (int j = 0; j < kVCh; ++j) {
      const int ks = min(s0 + j * kVWaves, steps - 1);  // steps past the end load in bounds, add nothing
      const bool ad = ks >= nk1;
      const int kk = (ad ? ks - nk1 : ks) * M::KS + kh;
      const T* wsrc = ad ? p.bt + (size_t)wrow * p.kx + kk
                         : (p.wpk ? p.wv + (((size_t)ct * nk1 + ks) * 64 + lane) * 8 : p.wv + (size_t)wrow * p.F + kk);
      wf[j] = *(const frag*)wsrc;
      const size_t xo = ad ? (((size_t)tb * nku + ks - nk1) * 64 + lane) * 8 : (((size_t)tb * nk1 + ks) * 64 + lane) * 8;
      xf[j] = *(const frag*)((ad ? p.u : p.h) + xo);
      if (ad) gf[j] = *(const frag*)(p.g + xo);
    }
#pragma unroll
    for (int j = 0; j < kVCh; ++j) {
      const int ks = s0 + j * kVWaves;
      if (ks < steps) {
        if (ks >= nk1) {
          // U = w_e · u for the 8 adapter columns of this lane
          union { frag f; T e[M::KV]; } v, g;
          v.f = xf[j];
          g.f = gf[j];
#pragma unroll
          for (int i = 0; i < M::KV; ++i) v.e[i] = tok_ok ? from_f<T>(to_f(g.e[i]) * to_f(v.e[i])) : T(0.f);
          xf[j] = v.f;
        }
        acc = M::run(wf[j], xf[j], acc);
      }
    }
  }
  // lane: token t0 + lane%16, columns c0 + 4*(lane/16) + 0..3
  red[wave][lane] = acc;
  __syncthreads();
  if (tid < 64) {
    f32x4 a = red[0][tid];
#pragma unroll
    for (int w = 1; w < kVWaves; ++w) {
      const f32x4 q = red[w][tid];
      a = f32x4{a[0] + q[0], a[1] + q[1], a[2] + q[2], a[3] + q[3]};
    }
    const int t = t0 + (tid & 15), col = c0 + 4 * (tid >> 4);
    if (t < p.N) {
      union { T e[4]; unsigned long long u; } pk, rs;
      if (p.resid) rs.u = *(const unsigned long long*)(p.resid + (size_t)t * p.C + col);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        T o = from_f<T>(a[v]);
        if (p.resid) o = from_f<T>(to_f(rs.e[v]) + to_f(o));
        pk.e[v] = o;
      }
      *(unsigned long long*)(p.out + (size_t)t * p.C + col) = pk.u;
    }
  }
}

}  // namespace

hipError_t launch_frag_pack(int dtype, const void* src, void* dst, int R, int K, hipStream_t s) {
  if (R % 16 || K % 32 || dtype == 0) return hipErrorInvalidValue;
  const size_t n = (size_t)R * K / 8;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (dtype == 1) launch_kernel(frag_pack_kernel<f16>, grid, dim3(256), 0, s, (const f16*)src, (f16*)dst, R, K);
  else launch_kernel(frag_pack_kernel<bf16>, grid, dim3(256), 0, s, (const bf16*)src, (bf16*)dst, R, K);
  return mark(hipGetLastError(), "frag_pack", s);
}

hipError_t launch_decode_value(int dtype, const void* h, const void* wv, bool wv_packed, const void* u,
                               const void* g, const void* bt, const void* resid, void* out, int N, int C, int F,
                               int kx, const LossJob* loss, hipStream_t s) {
  if (N < 1 || N > 64 || C % 16 || F % 32 || kx % 32) return hipErrorInvalidValue;
  const int nb = (N + 15) / 16, nct = C / 16;
  const int ntile = (nct + 7) / 8 * 8 * nb;
  const int grid = ntile + (loss ? 1 : 0);
  auto go = [&](auto tag) -> hipError_t {
    typedef decltype(tag) T;
    DecodeValue<T> p{(const T*)h, (const T*)wv, (const T*)u, (const T*)g, (const T*)bt, (const T*)resid, (T*)out,
                     N, C, F, kx, nb, nct, wv_packed ? 1 : 0, ntile, LossJob{}};
    if (loss) p.loss = *loss;
    launch_kernel(decode_value_kernel<T>, dim3(grid), dim3(kVThreads), 0, s, p);
    return mark(hipGetLastError(), "decode_value", s);
  };
  switch (dtype) {
    case 1: return go(f16{});
    case 2: return go(bf16{});
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rwkvmoe
