// MFMA GEMMs of the ChannelMix path for gfx950.
//
// All three products are "NT": out(M,N) = A(M,K) · B(N,K)ᵀ with both operands
// K-contiguous, which is how the reference stores them:
//   key    h   = relu(xk · W_keyᵀ)²        A = xk (N_tok,C)  B = W_key (F,C)     model.py:260-262
//   value  out = h · W_valueᵀ [+ U · B_allᵀ] A = h (N_tok,F)   B = W_value (C,F)   model.py:263, moe.py:139-147
//   down   U   = gate ⊙ (x · A_allᵀ)       A = x (N_tok,C)   B = A_all (Kx,C)    moe.py:140-144
// The token shift (model.py:67-75, 260-261) is applied while the A tile is
// staged into LDS, and relu², the gate mask and the residual add run in the
// epilogue, so no elementwise pass touches HBM.
//
// Tiling: a 256-thread workgroup (4 waves, 2x2) owns a BM x BN output tile;
// each wave computes (BM/2) x (BN/2) with v_mfma_f32_32x32x16_{f16,bf16}
// (v_mfma_f32_32x32x2f32 for fp32).  K is walked in 128-byte slices staged
// through double-buffered, padded LDS; the next slice's global loads are in
// flight while the current slice feeds the MFMAs.
#include "common.h"
#include "internal.h"

namespace rwkvmoe {
namespace {

enum { PRO_NONE = 0, PRO_SHIFT = 1 };
enum { EPI_STORE = 0, EPI_RELU2 = 1, EPI_GATE = 2, EPI_RESID = 3 };

template <typename T>
struct GemmParams {
  const T* a1; const T* b1; int k1; int lda1; int ldb1;   // segment 1
  const T* a2; const T* b2; int k2; int lda2; int ldb2;   // segment 2 (k2 may be 0)
  int m, n;
  T* out; int ldo;
  const T* mu;      // (K1) token-shift mix, PRO_SHIFT
  const T* xprev;   // (M/seq_len, K1) state before t = 0, or null
  int seq_len;
  const T* gmat;    // (M, E) dense gates, EPI_GATE
  int n_experts, rank;
  const T* resid;   // (M, N), EPI_RESID
};

constexpr int kThreads = 256;

template <typename T, int BM, int BN, int PRO, int EPI, bool EXT>
__global__ __launch_bounds__(kThreads) void gemm_nt_kernel(GemmParams<T> p) {
  using M = Mma32<T>;
  typedef typename M::frag frag;
  constexpr int VEC = 16 / sizeof(T);   // elements per 16-byte chunk
  constexpr int BK = 128 / sizeof(T);   // elements per 128-byte K slice
  constexpr int LDS = BK + VEC;         // padded row stride (elements)
  constexpr int CPR = BK / VEC;         // chunks per row (8)
  constexpr int AC = BM * CPR / kThreads;
  constexpr int BC = BN * CPR / kThreads;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int MI = WM / 32, NI = WN / 32;
  static_assert(AC >= 1 && BC >= 1 && MI >= 1 && NI >= 1, "tile too small");

  __shared__ __attribute__((aligned(16))) T As[2][BM * LDS];
  __shared__ __attribute__((aligned(16))) T Bs[2][BN * LDS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Tile order: workgroups are dealt round-robin to the 8 XCDs, so give each
  // XCD a contiguous run of logical tiles, then walk tiles in groups of 8
  // M-tiles so neighbours share A rows and B columns in the XCD's L2.
  const int tiles_m = (p.m + BM - 1) / BM, tiles_n = p.n / BN;
  const int total = tiles_m * tiles_n;
  int pid = blockIdx.x;
  if ((total & 7) == 0) pid = (pid & 7) * (total >> 3) + (pid >> 3);
  constexpr int GROUP_M = 8;
  const int in_group = GROUP_M * tiles_n;
  const int first_m = (pid / in_group) * GROUP_M;
  const int gsize = min(tiles_m - first_m, GROUP_M);
  const int tm = first_m + (pid % in_group) % gsize;
  const int tn = (pid % in_group) / gsize;
  const int m0 = tm * BM, n0 = tn * BN;

  const int nk1 = p.k1 / BK, nkt = nk1 + (EXT ? p.k2 / BK : 0);

  u32x4 ra[AC], rb[BC];
  u32x4 rp[PRO == PRO_SHIFT ? AC : 1];
  u32x4 rmu;

  auto load = [&](int kt) {
    const bool seg2 = EXT && kt >= nk1;
    const T* A = seg2 ? p.a2 : p.a1;
    const T* B = seg2 ? p.b2 : p.b1;
    const int lda = seg2 ? p.lda2 : p.lda1, ldb = seg2 ? p.ldb2 : p.ldb1;
    const int kb = (seg2 ? kt - nk1 : kt) * BK;
#pragma unroll
    for (int i = 0; i < AC; ++i) {
      const int id = tid + i * kThreads, row = id / CPR, c = (id % CPR) * VEC;
      const int gm = m0 + row;
      ra[i] = gm < p.m ? *(const u32x4*)(A + (size_t)gm * lda + kb + c) : zero4();
      if constexpr (PRO == PRO_SHIFT) {
        u32x4 pv = zero4();
        if (gm < p.m) {
          const int t = gm % p.seq_len;
          if (t > 0)
            pv = *(const u32x4*)(A + (size_t)(gm - 1) * lda + kb + c);
          else if (p.xprev)
            pv = *(const u32x4*)(p.xprev + (size_t)(gm / p.seq_len) * lda + kb + c);
        }
        rp[i] = pv;
      }
    }
    if constexpr (PRO == PRO_SHIFT) rmu = *(const u32x4*)(p.mu + kb + (tid % CPR) * VEC);
#pragma unroll
    for (int i = 0; i < BC; ++i) {
      const int id = tid + i * kThreads, row = id / CPR, c = (id % CPR) * VEC;
      rb[i] = *(const u32x4*)(B + (size_t)(n0 + row) * ldb + kb + c);
    }
  };

  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < AC; ++i) {
      const int id = tid + i * kThreads, row = id / CPR, c = (id % CPR) * VEC;
      u32x4 v = ra[i];
      if constexpr (PRO == PRO_SHIFT) {
        // xx = shift(x) - x ; xk = x + xx * x_k, each op rounded to T (model.py:260-261)
        Chunk<T> xc, pc, mc, o;
        xc.raw = ra[i]; pc.raw = rp[i]; mc.raw = rmu;
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          const float xf = to_f(xc.e[j]);
          const float xx = rnd<T>(to_f(pc.e[j]) - xf);
          const float t1 = rnd<T>(xx * to_f(mc.e[j]));
          o.e[j] = from_f<T>(xf + t1);
        }
        v = o.raw;
      }
      *(u32x4*)(&As[buf][row * LDS + c]) = v;
    }
#pragma unroll
    for (int i = 0; i < BC; ++i) {
      const int id = tid + i * kThreads, row = id / CPR, c = (id % CPR) * VEC;
      *(u32x4*)(&Bs[buf][row * LDS + c]) = rb[i];
    }
  };

  f32x16 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nkt; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nkt) load(kt + 1);
#pragma unroll
    for (int kk = 0; kk < BK; kk += M::KS) {
      frag af[MI], bf[NI];
#pragma unroll
      for (int i = 0; i < MI; ++i)
        af[i] = *(const frag*)(&As[buf][(wm * WM + i * 32 + (lane & 31)) * LDS + kk + (lane >> 5) * M::KV]);
#pragma unroll
      for (int j = 0; j < NI; ++j)
        bf[j] = *(const frag*)(&Bs[buf][(wn * WN + j * 32 + (lane & 31)) * LDS + kk + (lane >> 5) * M::KV]);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = M::run(af[i], bf[j], acc[i][j]);
    }
    if (kt + 1 < nkt) store(buf ^ 1);
    __syncthreads();
  }

  // Epilogue.
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int col = n0 + wn * WN + j * 32 + (lane & 31);
      int e = 0;
      if constexpr (EPI == EPI_GATE) e = col / p.rank;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * WM + i * 32 + acc_row(v, lane);
        if (row >= p.m) continue;
        float r = rnd<T>(acc[i][j][v]);
        if constexpr (EPI == EPI_RELU2) {
          r = r > 0.f ? r : 0.f;
          r = r * r;  // relu(key(k)) ** 2 (model.py:262)
        } else if constexpr (EPI == EPI_GATE) {
          // U[:, e*r + j] = w_e ⊙ (x·A_e)[:, j]; w_e = 0 when e is not routed (moe.py:144)
          const float g = e < p.n_experts ? to_f(p.gmat[(size_t)row * p.n_experts + e]) : 0.f;
          r = g * r;
        } else if constexpr (EPI == EPI_RESID) {
          r = to_f(p.resid[(size_t)row * p.ldo + col]) + r;
        }
        p.out[(size_t)row * p.ldo + col] = from_f<T>(r);
      }
    }
}

template <typename T, int BM, int BN, int PRO, int EPI, bool EXT>
hipError_t run(const GemmParams<T>& p, hipStream_t s) {
  const int tiles = ((p.m + BM - 1) / BM) * (p.n / BN);
  if (tiles == 0) return hipSuccess;
  hipLaunchKernelGGL((gemm_nt_kernel<T, BM, BN, PRO, EPI, EXT>), dim3(tiles), dim3(kThreads), 0, s, p);
  return hipGetLastError();
}

// EXT: a second K segment follows the first (the fused adapter columns).
template <typename T, int PRO, int EPI, bool EXT = false>
hipError_t run_n(const GemmParams<T>& p, hipStream_t s) {
  if (p.n % 128 == 0) return run<T, 128, 128, PRO, EPI, EXT>(p, s);
  return run<T, 128, 64, PRO, EPI, EXT>(p, s);
}

template <typename T>
GemmParams<T> blank() {
  GemmParams<T> p;
  __builtin_memset(&p, 0, sizeof(p));
  p.seq_len = 1;
  p.rank = 1;
  return p;
}

}  // namespace

hipError_t launch_cmix_key(int dtype, const void* x, const void* xprev, const void* mu, const void* wk, void* h,
                           int N, int T_, int C, int F, hipStream_t s) {
  RWKV_DISPATCH_DTYPE(dtype, T, {
    GemmParams<T> p = blank<T>();
    p.a1 = (const T*)x; p.lda1 = C; p.b1 = (const T*)wk; p.ldb1 = C; p.k1 = C;
    p.m = N; p.n = F; p.out = (T*)h; p.ldo = F;
    p.mu = (const T*)mu; p.xprev = (const T*)xprev; p.seq_len = T_;
    return run_n<T, PRO_SHIFT, EPI_RELU2>(p, s);
  });
  return hipSuccess;
}

hipError_t launch_cmix_value(int dtype, const void* h, const void* wv, int F, const void* u, const void* bt, int kx,
                             const void* resid, void* out, int N, int C, hipStream_t s) {
  RWKV_DISPATCH_DTYPE(dtype, T, {
    GemmParams<T> p = blank<T>();
    p.a1 = (const T*)h; p.lda1 = F; p.b1 = (const T*)wv; p.ldb1 = F; p.k1 = F;
    if (u && bt) { p.a2 = (const T*)u; p.lda2 = kx; p.b2 = (const T*)bt; p.ldb2 = kx; p.k2 = kx; }
    p.m = N; p.n = C; p.out = (T*)out; p.ldo = C; p.resid = (const T*)resid;
    if (p.k2 > 0) {
      if (resid) return run_n<T, PRO_NONE, EPI_RESID, true>(p, s);
      return run_n<T, PRO_NONE, EPI_STORE, true>(p, s);
    }
    if (resid) return run_n<T, PRO_NONE, EPI_RESID>(p, s);
    return run_n<T, PRO_NONE, EPI_STORE>(p, s);
  });
  return hipSuccess;
}

hipError_t launch_lora_down(int dtype, const void* x, const void* at, const void* gdense, int N, int C, int kx, int E,
                            int r, void* u, hipStream_t s) {
  RWKV_DISPATCH_DTYPE(dtype, T, {
    GemmParams<T> p = blank<T>();
    p.a1 = (const T*)x; p.lda1 = C; p.b1 = (const T*)at; p.ldb1 = C; p.k1 = C;
    p.m = N; p.n = kx; p.out = (T*)u; p.ldo = kx;
    p.gmat = (const T*)gdense; p.n_experts = E; p.rank = r;
    return run_n<T, PRO_NONE, EPI_GATE>(p, s);
  });
  return hipSuccess;
}

}  // namespace rwkvmoe
