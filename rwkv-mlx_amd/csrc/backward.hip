// Backward (VJP) of the LoRA-MoE ChannelMix layer with respect to x,
// lora_A, lora_B and router.gate.weight — what MLX autodiff computes for the
// reference's training step (rwkv_mlx/finetune_moe.py:215-232 over
// moe.py:129-147).  The base output is under stop_gradient (moe.py:131), so
// only the router and the adapters carry gradient.
//
// The sparse per-expert sums are evaluated densely over the Kx = E·r (padded)
// adapter columns, so that every product runs on the MFMA GEMM of gemm.hip:
//   S  = x  · A_allᵀ              (N, Kx)  s_e = x·A_e for every expert
//   G  = dO · B_rowsᵀ             (N, Kx)  dO·B_eᵀ, B_rows[e·r+i] = B[e][i]
//   bwd_route_kernel, per token:  gates from the saved logits, dg_j = <s_e, G_e>
//       (= <dO, a_e>), the softmax / aux / z terms of dℓ, and
//       DSd[t, e·r+i] = g_j·G (ds_e), SGd = g_j·S (zero off the selected experts)
//   O        = xᵀ · [DSd | dℓ]     (C, Kx + Ep)  K = tokens: dA_all_T and dW_gateᵀ
//   dB_rows  = SGdᵀ · dO          (E·r, C) = dB in its (E, r, C) layout
//   dx       = DSd · A_allᵀᵀ + dℓ · W_gate   (one K-extended GEMM)
// Products whose K runs over tokens take operands transposed once
// (transpose_pad_kernel: token-contiguous rows, zero-padded to Np tokens).
#include "common.h"
#include "internal.h"

namespace rwkvmoe {
namespace {

// dst (W rows x Rp columns) = srcᵀ for src (R rows x W columns, row stride
// lds); columns R..Rp-1 of dst are zero.  W, lds and Rp are multiples of 64:
// 64x64 tiles, 16-byte loads along src rows and 16-byte stores along dst
// rows, through LDS (float holds every element type exactly).
template <typename T>
__global__ __launch_bounds__(256) void transpose_pad_kernel(const T* __restrict__ src, int R, int W, int lds,
                                                            T* __restrict__ dst, int Rp) {
  constexpr int VEC = 16 / sizeof(T), CPR = 64 / VEC;  // elements per 16 B, chunks per 64-wide row
  __shared__ float tile[64][65];
  const int w0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
  for (int i = threadIdx.x; i < 64 * CPR; i += 256) {
    const int rl = i / CPR, q = i - rl * CPR, r = r0 + rl;
    Chunk<T> c;
    c.raw = r < R ? *(const u32x4*)(src + (size_t)r * lds + w0 + q * VEC) : zero4();
#pragma unroll
    for (int j = 0; j < VEC; ++j) tile[rl][q * VEC + j] = to_f(c.e[j]);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * CPR; i += 256) {
    const int wl = i / CPR, q = i - wl * CPR;
    Chunk<T> c;
#pragma unroll
    for (int j = 0; j < VEC; ++j) c.e[j] = from_f<T>(tile[q * VEC + j][wl]);
    *(u32x4*)(dst + (size_t)(w0 + wl) * Rp + r0 + q * VEC) = c.raw;
  }
}

// The backward's weight re-layouts in one launch (16-bit or fp32 elements):
//   A_all  (kx, C):  A_all[e·r+i][c] = A[e][c][i]   (rows >= E·r zero)
//   A_T    (C, kx):  A_T[c][e·r+i]   = A[e][c][i]   (columns >= E·r zero)
//   B_rows (kx, C):  B_rows[e·r+i][c] = B[e][i][c]  (rows >= E·r zero)
//   WgT    (C, ep):  WgT[c][e] = W_gate[e][c]       (columns >= E zero)
// B_rows and WgT are skipped when their pointers are null.
template <typename T>
__global__ __launch_bounds__(256) void bwd_prep_kernel(const T* __restrict__ A, const T* __restrict__ B,
                                                       const T* __restrict__ wg, int E, int C, int r, int kx, int ep,
                                                       T* __restrict__ a_all, T* __restrict__ a_t,
                                                       T* __restrict__ b_rows, T* __restrict__ wgt) {
  const size_t i = blockIdx.x * (size_t)256 + threadIdx.x;
  const size_t n1 = (size_t)kx * C;
  const int er = E * r;
  if (i < n1) {
    const int row = (int)(i / C), c = (int)(i - (size_t)row * C);
    a_all[i] = row < er ? A[(size_t)(row / r) * C * r + (size_t)c * r + row % r] : from_f<T>(0.f);
  } else if (i < 2 * n1) {
    const size_t j = i - n1;
    const int c = (int)(j / kx), col = (int)(j - (size_t)c * kx);
    a_t[j] = col < er ? A[(size_t)(col / r) * C * r + (size_t)c * r + col % r] : from_f<T>(0.f);
  } else if (i < 3 * n1) {
    if (!b_rows) return;
    const size_t j = i - 2 * n1;
    const int row = (int)(j / C), c = (int)(j - (size_t)row * C);
    b_rows[j] = row < er ? B[(size_t)row * C + c] : from_f<T>(0.f);
  } else if (i < 3 * n1 + (size_t)C * ep) {
    if (!wgt) return;
    const size_t j = i - 3 * n1;
    const int c = (int)(j / ep), e = (int)(j - (size_t)c * ep);
    wgt[j] = e < E ? wg[(size_t)e * C + c] : from_f<T>(0.f);
  }
}

// Gradient of orthogonal_loss (moe.py:149-163): dA_i = 2 Σ_{j≠i} A_j·(A_jᵀA_i)
// is dA_T = A_T · Gm with Gm = 2·d_ortho·(A_all·A_allᵀ) off the diagonal
// r x r blocks (and zero past E·r).  This kernel turns the Gram matrix into
// Gm in place.
template <typename T>
__global__ __launch_bounds__(256) void ortho_mask_kernel(T* __restrict__ gram, int er, int r, int kx,
                                                         const float* __restrict__ d_ortho) {
  const size_t i = blockIdx.x * (size_t)256 + threadIdx.x;
  if (i >= (size_t)kx * kx) return;
  const int row = (int)(i / kx), col = (int)(i - (size_t)row * kx);
  const float d = d_ortho ? d_ortho[0] : 1.f;
  const bool keep = row < er && col < er && row / r != col / r;
  gram[i] = from_f<T>(keep ? 2.f * d * to_f(gram[i]) : 0.f);
}

// Tokens routed to each expert (the counts f_e of the aux loss,
// moe.py:80-83); one workgroup, LDS integer atomics (order-independent).
__global__ __launch_bounds__(1024) void bwd_count_kernel(const int* __restrict__ inds, int nk, int E,
                                                         int* __restrict__ cnt) {
  __shared__ int h[64];
  if (threadIdx.x < 64) h[threadIdx.x] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < nk; i += blockDim.x) {
    const int e = inds[i];
    if (e >= 0 && e < E) atomicAdd(&h[e], 1);
  }
  __syncthreads();
  if ((int)threadIdx.x < E) cnt[threadIdx.x] = h[threadIdx.x];
}

constexpr int kRouteTok = 16;   // tokens per workgroup
constexpr int kRouteThreads = kRouteTok * 8;
constexpr int kBwdMaxK = 8;

// Routing gradient, 16 tokens per workgroup (8 threads per token for the
// routing math).  The tile's logits, selections and the expert counts are
// staged in LDS first, so the routing phases wait on no memory.  From the
// saved logits ℓ and selection: the gates g̃ = softmax(ℓ[I]) and their dtype
// cast g (the forward's values), dg_j = Σ_i S·G over the slot's expert
// columns, then
//   dℓ[I_j] += g̃_j (dg_j − Σ_i g̃_i dg_i)
//   dℓ      += d_aux·(E/N)·P ⊙ (f − <P, f>) + d_z·(2 lse / N)·P
// with P = softmax(ℓ), lse = log Σ exp ℓ, f = counts / (N k); the 8 threads
// of a token each compute the gates (in slot order, as the forward does),
// thread j takes slot j's dot product, and every 8th expert's terms, combined
// with shuffles.  Then, in 64-column chunks: DSd = g·G and SGd = g·S on the
// selected experts' columns (0 elsewhere), written row-major (DSd, tokens
// < N) and, through an LDS tile, transposed with 16-byte stores (DSdᵀ, SGdᵀ;
// zero for padding tokens N..Np-1).  dℓ goes out row-major (N x ep) and
// transposed into the rows kx..kx+ep-1 of the same transposed array as DSdᵀ.
//
// FUSED (16-bit, Kx <= 128, C <= 768): S = x·A_allᵀ and G = dO·B_rowsᵀ for
// the tile are computed here rather than read from memory: the tile's x and
// dO rows go to LDS with the logits, then each of the 8 waves takes its
// 16-column blocks of S and G (both blocks' B fragments loaded together from
// A_all / B_rows in L2) with v_mfma_f32_16x16x32, rounding to the element
// type as the GEMM's epilogue does; the routing phases read S and G from LDS.
constexpr int kFusedThreads = 512;
constexpr int kFusedMaxKx = 128, kFusedMaxC = 768;  // 2 Kx/16 blocks <= 2 per wave

template <typename T, bool FUSED>
__global__ __launch_bounds__(FUSED ? kFusedThreads : kRouteThreads) void bwd_route_kernel(
    const float* __restrict__ logits, const int* __restrict__ inds, const T* __restrict__ S,
    const T* __restrict__ G, const int* __restrict__ cnt, const float* __restrict__ dloss, int N, int E, int k, int r,
    int kx, int ep, int np, T* __restrict__ dsd, T* __restrict__ dl, T* __restrict__ rT, T* __restrict__ sgdT,
    const T* __restrict__ x, const T* __restrict__ dO, const T* __restrict__ a_all, const T* __restrict__ b_rows,
    int C) {
  constexpr int VEC = 16 / sizeof(T), CPR = 64 / VEC, TPR = kRouteTok / VEC;
  constexpr int NT = FUSED ? kFusedThreads : kRouteThreads;
  __shared__ float dls[kRouteTok][65];
  __shared__ float lgs[kRouteTok][65];  // the tile's logits
  __shared__ int ids[kRouteTok][kBwdMaxK], cnts[64];
  __shared__ float gs[kRouteTok][kBwdMaxK], gts[kRouteTok][kBwdMaxK], dgs[kRouteTok][kBwdMaxK];
  __shared__ int es[kRouteTok][kBwdMaxK];
  __shared__ T tD[64][kRouteTok + VEC], tS[64][kRouteTok + VEC];
  extern __shared__ __attribute__((aligned(16))) unsigned char dyn[];
  const int t0 = blockIdx.x * kRouteTok, tid = threadIdx.x;
  const int tl = (tid >> 3) & (kRouteTok - 1), sub = tid & 7, t = t0 + tl;
  const bool rthread = tid < kRouteThreads;  // the routing phases: 8 threads per token
  const bool live = rthread && t < N;
  // S and G of the tile: rows tl of (Sb, Gb) with row stride ss
  const T* Sb = S + (size_t)t0 * kx;
  const T* Gb = G + (size_t)t0 * kx;
  int ss = kx;

  // logits, selections and counts of the tile -> LDS (loads issued before the
  // x / dO rows, so they come back first)
  {
    const int nt = min(kRouteTok, N - t0);
    for (int i = tid; i < kRouteTok * E; i += NT) {
      const int rl = i / E, e = i - rl * E;
      lgs[rl][e] = rl < nt ? logits[(size_t)(t0 + rl) * E + e] : 0.f;
    }
    for (int i = tid; i < kRouteTok * k; i += NT) {
      const int rl = i / k, j = i - rl * k;
      ids[rl][j] = rl < nt ? inds[(size_t)(t0 + rl) * k + j] : -1;
    }
    for (int e = tid; e < E; e += NT) cnts[e] = cnt[e];
  }
  if constexpr (FUSED) {
    const int XSS = C + 8, KXS = kx + 8;  // LDS row strides (16-byte aligned rows)
    T* xs = (T*)dyn;
    T* os = xs + kRouteTok * XSS;
    T* sS = os + kRouteTok * XSS;
    T* sG = sS + kRouteTok * KXS;
    // x and dO rows of the tile (zeros past N), all loads of a thread in flight together
    {
      const int cpr = C / VEC, per = kRouteTok * cpr;
      constexpr int LB = 2 * kRouteTok * (kFusedMaxC / VEC) / kFusedThreads;
      u32x4 v[LB];
#pragma unroll
      for (int j = 0; j < LB; ++j) {
        const int i = tid + j * NT;
        const int which = i >= per ? 1 : 0, rem = i - which * per;
        const int rl = rem / cpr, c = (rem - rl * cpr) * VEC, tt = t0 + rl;
        const bool ok = i < 2 * per && tt < N;
        const T* src = which ? dO : x;
        const u32x4 w = *(const u32x4*)(src + (size_t)(ok ? tt : 0) * C + (ok ? c : 0));
        v[j] = ok ? w : zero4();
      }
#pragma unroll
      for (int j = 0; j < LB; ++j) {
        const int i = tid + j * NT;
        if (i < 2 * per) {
          const int which = i >= per ? 1 : 0, rem = i - which * per;
          const int rl = rem / cpr, c = (rem - rl * cpr) * VEC;
          *(u32x4*)((which ? os : xs) + rl * XSS + c) = v[j];
        }
      }
    }
    // this wave's S / G blocks (column blocks of 16; at most two per wave):
    // both blocks' B fragments are loaded before the tile's rows are awaited
    using UM = Mma16<T>;
    typedef typename UM::frag ufrag;
    const int wave = tid >> 6, lane = tid & 63;
    const int nb = kx / 16, nks = C / UM::KS;
    constexpr int MAXKS = kFusedMaxC / UM::KS, NW = kFusedThreads / 64;
    ufrag bf[2][MAXKS];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int b = wave + q * NW;
      if (b < 2 * nb) {
        const bool isG = b >= nb;
        const int col0 = (isG ? b - nb : b) * 16;
        const T* wrow = (isG ? b_rows : a_all) + (size_t)(col0 + (lane & 15)) * C + (lane >> 4) * UM::KV;
#pragma unroll
        for (int j = 0; j < MAXKS; ++j)
          if (j < nks) bf[q][j] = *(const ufrag*)(wrow + j * UM::KS);
      }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int b = wave + q * NW;
      if (b < 2 * nb) {
        const bool isG = b >= nb;
        const int col0 = (isG ? b - nb : b) * 16;
        const T* arow = (isG ? os : xs) + (lane & 15) * XSS + (lane >> 4) * UM::KV;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < MAXKS; ++j)
          if (j < nks) acc = UM::run(*(const ufrag*)(arow + j * UM::KS), bf[q][j], acc);
        T* dst = isG ? sG : sS;
#pragma unroll
        for (int v = 0; v < 4; ++v) dst[((lane >> 4) * 4 + v) * KXS + col0 + (lane & 15)] = from_f<T>(acc[v]);
      }
    }
    Sb = sS;
    Gb = sG;
    ss = KXS;
  }
  __syncthreads();
  // gates (every thread of the token, in slot order) and dg (thread j: slot j)
  if (rthread) {
    float m = 0.f, den = 0.f, ex[kBwdMaxK];
    int ej[kBwdMaxK];
    es[tl][sub] = -1;
    gs[tl][sub] = gts[tl][sub] = dgs[tl][sub] = 0.f;
    if (live) {
      for (int j = 0; j < k; ++j) {
        const int raw = ids[tl][j];
        ej[j] = raw >= 0 && raw < E ? raw : -1;  // the forward writes only valid ids; others carry no gradient
        const float l = lgs[tl][ej[j] >= 0 ? ej[j] : 0];
        if (j == 0) m = l;
        ex[j] = expf(l - m);
        den += ex[j];
      }
      if (sub < k) {
        const float gt = ex[sub] / den;
        const int e = ej[sub];
        float acc = 0.f;
        if (e >= 0) {
          const T* sr = Sb + (size_t)tl * ss + e * r;
          const T* gr = Gb + (size_t)tl * ss + e * r;
          for (int i = 0; i < r; ++i) acc += to_f(sr[i]) * to_f(gr[i]);
        }
        es[tl][sub] = e;
        gs[tl][sub] = rnd<T>(gt);
        gts[tl][sub] = gt;
        dgs[tl][sub] = acc;
      }
    }
  }
  __syncthreads();
  // softmax, lse and <P, f> over the experts, 8 threads per token
  if (rthread) {
    const float* lr = lgs[tl];
    float mx = -INFINITY;
    for (int e = sub; e < E; e += 8) mx = fmaxf(mx, lr[e]);
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 8));
    const float inv_nk = 1.f / ((float)N * (float)k);
    float sp = 0.f, se = 0.f, pf = 0.f;
    for (int e = sub; e < E; e += 8) {
      const float p = expf(lr[e] - mx);
      sp += p;
      se += expf(lr[e]);
      pf += p * ((float)cnts[e] * inv_nk);
    }
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) {
      sp += __shfl_xor(sp, off, 8);
      se += __shfl_xor(se, off, 8);
      pf += __shfl_xor(pf, off, 8);
    }
    pf /= sp;
    const float lse = logf(se);
    const float daux = dloss ? dloss[0] : 0.f, dz = dloss ? dloss[1] : 0.f;
    const float caux = daux * (float)E / (float)N, cz = dz * 2.f * lse / (float)N;
    float sdg = 0.f;
    for (int j = 0; j < kBwdMaxK; ++j) sdg += gts[tl][j] * dgs[tl][j];
    for (int e = sub; e < 64; e += 8) {
      float v = 0.f;
      if (live && e < E) {
        const float P = expf(lr[e] - mx) / sp;
        v = caux * P * ((float)cnts[e] * inv_nk - pf) + cz * P;
        for (int j = 0; j < kBwdMaxK; ++j)
          if (es[tl][j] == e) v += gts[tl][j] * (dgs[tl][j] - sdg);
      }
      dls[tl][e] = v;
    }
  }
  __syncthreads();
  // DSd / SGd in 64-column chunks
  for (int c0 = 0; c0 < kx; c0 += 64) {
    for (int i = tid; i < kRouteTok * CPR; i += NT) {
      const int rl = i / CPR, q = i - rl * CPR, tt = t0 + rl, col0 = c0 + q * VEC;
      Chunk<T> cs, cg, od, os;
      cs.raw = cg.raw = zero4();
      if (tt < N) {
        cs.raw = *(const u32x4*)(Sb + (size_t)rl * ss + col0);
        cg.raw = *(const u32x4*)(Gb + (size_t)rl * ss + col0);
      }
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const int col = col0 + j, e = col / r;
        float g = 0.f;
        if (col < E * r)
          for (int s = 0; s < kBwdMaxK; ++s)
            if (es[rl][s] == e) g = gs[rl][s];
        od.e[j] = from_f<T>(g * to_f(cg.e[j]));
        os.e[j] = from_f<T>(g * to_f(cs.e[j]));
        tD[q * VEC + j][rl] = od.e[j];
        tS[q * VEC + j][rl] = os.e[j];
      }
      if (tt < N) *(u32x4*)(dsd + (size_t)tt * kx + col0) = od.raw;
    }
    __syncthreads();
    for (int i = tid; i < 64 * TPR; i += NT) {
      const int cl = i / TPR, q = i - cl * TPR;
      Chunk<T> od, os;
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        od.e[j] = tD[cl][q * VEC + j];
        os.e[j] = tS[cl][q * VEC + j];
      }
      *(u32x4*)(rT + (size_t)(c0 + cl) * np + t0 + q * VEC) = od.raw;
      *(u32x4*)(sgdT + (size_t)(c0 + cl) * np + t0 + q * VEC) = os.raw;
    }
    __syncthreads();
  }
  // dℓ: row-major (tokens < N) and transposed (rows kx.. of rT)
  for (int i = tid; i < kRouteTok * (ep / VEC); i += NT) {
    const int rl = i / (ep / VEC), q = i - rl * (ep / VEC), tt = t0 + rl;
    if (tt >= N) continue;
    Chunk<T> c;
#pragma unroll
    for (int j = 0; j < VEC; ++j) c.e[j] = from_f<T>(q * VEC + j < 64 ? dls[rl][q * VEC + j] : 0.f);
    *(u32x4*)(dl + (size_t)tt * ep + q * VEC) = c.raw;
  }
  for (int i = tid; i < ep * TPR; i += NT) {
    const int e = i / TPR, q = i - e * TPR;
    Chunk<T> c;
#pragma unroll
    for (int j = 0; j < VEC; ++j) c.e[j] = from_f<T>(e < 64 ? dls[q * VEC + j][e] : 0.f);
    *(u32x4*)(rT + (size_t)(kx + e) * np + t0 + q * VEC) = c.raw;
  }
}

// dA[e][c][i] = O[c][e·r+i] and dW_gate[e][c] = O[c][kx+e] for the merged
// product O = xᵀ · [DSd | dℓ] (C x (kx + ep)); either output may be null.
template <typename T>
__global__ __launch_bounds__(256) void relayout_dawg_kernel(const T* __restrict__ o, int E, int C, int r, int kx,
                                                            int ep, T* __restrict__ dA, T* __restrict__ dwg) {
  const size_t i = blockIdx.x * (size_t)256 + threadIdx.x;
  const size_t na = dA ? (size_t)E * C * r : 0;
  const size_t nw = dwg ? (size_t)E * C : 0;
  const int ow = kx + ep;
  if (i < na) {
    const int e = (int)(i / ((size_t)C * r));
    const int rem = (int)(i - (size_t)e * C * r);
    const int c = rem / r, j = rem - c * r;
    dA[i] = o[(size_t)c * ow + e * r + j];
  } else if (i < na + nw) {
    const size_t w = i - na;
    const int e = (int)(w / C), c = (int)(w - (size_t)e * C);
    dwg[w] = o[(size_t)c * ow + kx + e];
  }
}

}  // namespace

hipError_t launch_transpose_pad(int dtype, const void* src, int R, int W, int lds, void* dst, int Rp, hipStream_t s) {
  if (W % 64 || Rp % 64 || lds % 8) return hipErrorInvalidValue;
  const dim3 grid(W / 64, Rp / 64);
  RWKV_DISPATCH_DTYPE(dtype, T, {
    hipLaunchKernelGGL(transpose_pad_kernel<T>, grid, dim3(256), 0, s, (const T*)src, R, W, lds, (T*)dst, Rp);
  });
  return mark(hipGetLastError(), "bwd_transpose", s);
}

hipError_t launch_bwd_prep(int dtype, const void* A, const void* B, const void* wg, int E, int C, int r, int kx,
                           int ep, void* a_all, void* a_t, void* b_rows, void* wgt, hipStream_t s) {
  const size_t total = 3 * (size_t)kx * C + (size_t)C * ep;
  const dim3 grid((unsigned)((total + 255) / 256));
  RWKV_DISPATCH_DTYPE(dtype, T, {
    hipLaunchKernelGGL(bwd_prep_kernel<T>, grid, dim3(256), 0, s, (const T*)A, (const T*)B, (const T*)wg, E, C, r, kx,
                       ep, (T*)a_all, (T*)a_t, (T*)b_rows, (T*)wgt);
  });
  return mark(hipGetLastError(), "bwd_prep", s);
}

hipError_t launch_ortho_mask(int dtype, void* gram, int er, int r, int kx, const float* d_ortho, hipStream_t s) {
  const dim3 grid((unsigned)(((size_t)kx * kx + 255) / 256));
  RWKV_DISPATCH_DTYPE(dtype, T, {
    hipLaunchKernelGGL(ortho_mask_kernel<T>, grid, dim3(256), 0, s, (T*)gram, er, r, kx, d_ortho);
  });
  return mark(hipGetLastError(), "ortho_mask", s);
}

hipError_t launch_bwd_count(const int* inds, int nk, int E, int* cnt, hipStream_t s) {
  hipLaunchKernelGGL(bwd_count_kernel, dim3(1), dim3(1024), 0, s, inds, nk, E, cnt);
  return mark(hipGetLastError(), "bwd_count", s);
}

hipError_t launch_bwd_route(int dtype, const float* logits, const int* inds, const void* S, const void* G,
                            const int* cnt, const float* dloss, int N, int E, int k, int r, int kx, int ep, int np,
                            void* dsd, void* dl, void* rT, void* sgdT, hipStream_t s, const void* x, const void* dO,
                            const void* a_all, const void* b_rows, int C) {
  if (k > kBwdMaxK || E > 64 || ep < 64 || ep % 64 || kx % 64 || np % kRouteTok) return hipErrorInvalidValue;
  const dim3 grid(np / kRouteTok);
  const bool fused = x != nullptr;
  if (fused && !bwd_route_fuses(dtype, kx, C)) return hipErrorInvalidValue;
  RWKV_DISPATCH_DTYPE(dtype, T, {
    if constexpr (sizeof(T) == 2) {
      if (fused) {
        const size_t smem = (size_t)2 * kRouteTok * ((C + 8) + (kx + 8)) * sizeof(T);
        auto kern = bwd_route_kernel<T, true>;
        if (smem > 65536) {
          const hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   (int)smem);
          if (e != hipSuccess) return e;
        }
        hipLaunchKernelGGL(kern, grid, dim3(kFusedThreads), smem, s, logits, inds, (const T*)nullptr,
                           (const T*)nullptr, cnt, dloss, N, E, k, r, kx, ep, np, (T*)dsd, (T*)dl, (T*)rT, (T*)sgdT,
                           (const T*)x, (const T*)dO, (const T*)a_all, (const T*)b_rows, C);
        return mark(hipGetLastError(), "bwd_route_fused", s);
      }
    }
    hipLaunchKernelGGL((bwd_route_kernel<T, false>), grid, dim3(kRouteThreads), 0, s, logits, inds, (const T*)S,
                       (const T*)G, cnt, dloss, N, E, k, r, kx, ep, np, (T*)dsd, (T*)dl, (T*)rT, (T*)sgdT,
                       (const T*)nullptr, (const T*)nullptr, (const T*)nullptr, (const T*)nullptr, C);
  });
  return mark(hipGetLastError(), "bwd_route", s);
}

bool bwd_route_fuses(int dtype, int kx, int C) {
  return dtype != 0 && kx <= kFusedMaxKx && C <= kFusedMaxC && C % 32 == 0;
}

hipError_t launch_relayout_dawg(int dtype, const void* o, int E, int C, int r, int kx, int ep, void* dA, void* dwg,
                                hipStream_t s) {
  const size_t total = (dA ? (size_t)E * C * r : 0) + (dwg ? (size_t)E * C : 0);
  if (total == 0) return hipSuccess;
  const dim3 grid((unsigned)((total + 255) / 256));
  RWKV_DISPATCH_DTYPE(dtype, T, {
    hipLaunchKernelGGL(relayout_dawg_kernel<T>, grid, dim3(256), 0, s, (const T*)o, E, C, r, kx, ep, (T*)dA,
                       (T*)dwg);
  });
  return mark(hipGetLastError(), "bwd_relayout", s);
}

}  // namespace rwkvmoe
