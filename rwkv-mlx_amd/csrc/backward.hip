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
#include <algorithm>

#include "common.h"
#include "internal.h"

namespace rwkvmoe {
namespace {

// dst (W rows x Rp columns) = srcᵀ for src (R rows x W columns, row stride
// lds); columns R..Rp-1 of dst are zero.  W, lds and Rp are multiples of 64:
// 64x64 tiles, 16-byte loads along src rows and 16-byte stores along dst
// rows, through LDS (float holds every element type exactly).  Matrix z of
// a batch (blockIdx.z) is src + z·sstride -> dst + z·dstride.
template <typename T>
__global__ __launch_bounds__(256) void transpose_pad_kernel(const T* __restrict__ src, int R, int W, int lds,
                                                            T* __restrict__ dst, int Rp, long long sstride,
                                                            long long dstride) {
  constexpr int VEC = 16 / sizeof(T), CPR = 64 / VEC;  // elements per 16 B, chunks per 64-wide row
  __shared__ float tile[64][65];
  const int w0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
  src += blockIdx.z * sstride;
  dst += blockIdx.z * dstride;
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
// B_rows and WgT are skipped when their pointers are null.  With `frag`,
// A_all and B_rows are written in fragment order (frag_coords) for the fused
// routing-gradient kernel instead of row-major.
//
// Fragment order of a (rows x C) 16-bit matrix, rows a multiple of 16 and
// C of 32: the v_mfma_f32_16x16x32 operand of 16-row block b, k-step j and
// lane l — the 8 elements (b·16 + l % 16, j·32 + (l / 16)·8 + 0..7) — sits at
// position ((b·C/32 + j)·64 + l)·8, so one wave's fragment is 1 KB contiguous.
RWKV_DEV void frag_coords(size_t p, int C, int& row, int& c) {
  const int i = (int)(p & 7), l = (int)((p >> 3) & 63);
  const size_t bj = p >> 9;
  const int nks = C / 32, b = (int)(bj / nks), j = (int)(bj - (size_t)b * nks);
  row = b * 16 + (l & 15);
  c = j * 32 + (l >> 4) * 8 + i;
}

template <typename T>
__global__ __launch_bounds__(256) void bwd_prep_kernel(const T* __restrict__ A, const T* __restrict__ B,
                                                       const T* __restrict__ wg, int E, int C, int r, int kx, int ep,
                                                       int frag, T* __restrict__ a_all, T* __restrict__ a_t,
                                                       T* __restrict__ b_rows, T* __restrict__ wgt,
                                                       const int* __restrict__ inds, int nk, int* __restrict__ cnt) {
  // workgroup 0 (when cnt is given; dispatched first, so it overlaps the
  // rest): tokens routed to each expert (the counts f_e of the aux loss,
  // moe.py:80-83), 32 loads per thread in flight, LDS integer atomics
  if (cnt && blockIdx.x == 0) {
    __shared__ int h[64];
    if (threadIdx.x < 64) h[threadIdx.x] = 0;
    __syncthreads();
    const __amdgpu_buffer_rsrc_t ri = buf_rsrc(inds, (unsigned)nk * 4);
    for (int b0 = 0; b0 < nk; b0 += 256 * 32) {
      unsigned v[32];
#pragma unroll
      for (int u = 0; u < 32; ++u) {
        const int j = b0 + u * 256 + (int)threadIdx.x;
        v[u] = buf_load4(ri, j < nk ? (unsigned)j * 4u : kOOB);
      }
#pragma unroll
      for (int u = 0; u < 32; ++u) {
        const int j = b0 + u * 256 + (int)threadIdx.x, e = (int)v[u];
        if (j < nk && e >= 0 && e < E) atomicAdd(&h[e], 1);
      }
    }
    __syncthreads();
    if ((int)threadIdx.x < E) cnt[threadIdx.x] = h[threadIdx.x];
    return;
  }
  const size_t i = (blockIdx.x - (cnt ? 1 : 0)) * (size_t)256 + threadIdx.x;
  const size_t n1 = (size_t)kx * C;
  const int er = E * r;
  if (i < n1) {
    int row, c;
    if (frag) {
      frag_coords(i, C, row, c);
    } else {
      row = (int)(i / C);
      c = (int)(i - (size_t)row * C);
    }
    a_all[i] = row < er ? A[(size_t)(row / r) * C * r + (size_t)c * r + row % r] : from_f<T>(0.f);
  } else if (i < 2 * n1) {
    const size_t j = i - n1;
    const int c = (int)(j / kx), col = (int)(j - (size_t)c * kx);
    a_t[j] = col < er ? A[(size_t)(col / r) * C * r + (size_t)c * r + col % r] : from_f<T>(0.f);
  } else if (i < 3 * n1) {
    if (!b_rows) return;
    const size_t j = i - 2 * n1;
    int row, c;
    if (frag) {
      frag_coords(j, C, row, c);
    } else {
      row = (int)(j / C);
      c = (int)(j - (size_t)row * C);
    }
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

constexpr int kRouteTok = 16;   // tokens per workgroup
constexpr int kRouteThreads = kRouteTok * 8;
constexpr int kBwdMaxK = 8;

// Routing gradient from S and G in memory, 16 tokens per workgroup, 8
// threads per token.  The tile's logits, selections and the expert counts
// are staged in LDS first, so the routing phases wait on no memory.  From
// the saved logits ℓ and selection: the gates g̃ = softmax(ℓ[I]) and their
// dtype cast g (the forward's values), dg_j = Σ_i S·G over the slot's expert
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
template <typename T>
__global__ __launch_bounds__(kRouteThreads) void bwd_route_kernel(
    const float* __restrict__ logits, const int* __restrict__ inds, const T* __restrict__ S,
    const T* __restrict__ G, const int* __restrict__ cnt, const float* __restrict__ dloss, int N, int E, int k, int r,
    int kx, int ep, int np, T* __restrict__ dsd, T* __restrict__ dl, T* __restrict__ rT, T* __restrict__ sgdT,
    T* __restrict__ sgd, unsigned long long* __restrict__ emask, int g16) {
  constexpr int VEC = 16 / sizeof(T), CPR = 64 / VEC, TPR = kRouteTok / VEC;
  constexpr int NT = kRouteThreads;
  __shared__ float dls[kRouteTok][65];
  __shared__ float lgs[kRouteTok][65];  // the tile's logits
  __shared__ int ids[kRouteTok][kBwdMaxK], cnts[64];
  __shared__ float gs[kRouteTok][kBwdMaxK], gts[kRouteTok][kBwdMaxK], dgs[kRouteTok][kBwdMaxK];
  __shared__ int es[kRouteTok][kBwdMaxK];
  __shared__ T tD[64][kRouteTok + VEC], tS[64][kRouteTok + VEC];
  const int t0 = blockIdx.x * kRouteTok, tid = threadIdx.x;
  const int tl = tid >> 3, sub = tid & 7, t = t0 + tl;
  const bool live = t < N;
  const T* Sb = S + (size_t)t0 * kx;
  const T* Gb = G + (size_t)t0 * kx;

  // logits, selections and counts of the tile -> LDS
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
  __syncthreads();
  // gates (every thread of the token, in slot order) and dg (thread j: slot j)
  {
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
          const T* sr = Sb + (size_t)tl * kx + e * r;
          const T* gr = Gb + (size_t)tl * kx + e * r;
          for (int i = 0; i < r; ++i) acc += to_f(sr[i]) * to_f(gr[i]);
        }
        es[tl][sub] = e;
        gs[tl][sub] = g16 ? rnd<f16>(gt) : rnd<T>(gt);
        gts[tl][sub] = gt;
        dgs[tl][sub] = acc;
      }
    }
  }
  __syncthreads();
  // softmax, lse and <P, f> over the experts, 8 threads per token
  {
    if (emask && live && sub == 0) {
      unsigned long long msk = 0;
      for (int j = 0; j < kBwdMaxK; ++j)
        if (es[tl][j] >= 0) msk |= 1ull << es[tl][j];
      emask[t] = msk;
    }
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
        cs.raw = *(const u32x4*)(Sb + (size_t)rl * kx + col0);
        cg.raw = *(const u32x4*)(Gb + (size_t)rl * kx + col0);
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
      if (sgd && tt < N) *(u32x4*)(sgd + (size_t)tt * kx + col0) = os.raw;
    }
    __syncthreads();
    for (int i = tid; rT && i < 64 * TPR; i += NT) {
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
  for (int i = tid; rT && i < ep * TPR; i += NT) {
    const int e = i / TPR, q = i - e * TPR;
    Chunk<T> c;
#pragma unroll
    for (int j = 0; j < VEC; ++j) c.e[j] = from_f<T>(e < 64 ? dls[q * VEC + j][e] : 0.f);
    *(u32x4*)(rT + (size_t)(kx + e) * np + t0 + q * VEC) = c.raw;
  }
}

// The same routing gradient with S = x·A_allᵀ and G = dO·B_rowsᵀ computed
// in the kernel (16-bit elements, Kx = 128, C <= 768, C % 32 == 0),
// 16 tokens and 512 threads per workgroup:
//  1. every load is issued up front.  Waves 0-1 (8 threads per token) load
//     their token's logits, selection and the counts of their experts;
//     waves 2-7 load the tile's x and dO rows; then every wave loads its
//     weight fragments (A_all / B_rows in fragment order, 1 KB each), which
//     stay in flight while the rest lands in LDS.
//  2. waves 0-1 compute the gates g̃ (slot order, as the forward), their
//     dtype cast g as a dense per-expert table, and the softmax / aux / z
//     part of dℓ from their own token's values (no workgroup barrier).
//  3. after one barrier each wave computes S or G 16x16 blocks with
//     v_mfma_f32_16x16x32 (block b: S columns b·16.. for b < Kx/16, else
//     G), rounds them to the element type as the GEMM epilogue does, and
//     gates them: DSd = g·G, SGd = g·S (g = 0 off the selected experts),
//     stored transposed from the accumulators (4 tokens of a column per
//     lane); raw S, G and DSd go to LDS.  Before the products, while the
//     fragments land, every thread writes one 8x8 block of xᵀ or dOᵀ
//     (token-contiguous rows, the operands of the token-contracted
//     products) from the rows in LDS, when asked.
//  4. waves 0-1: dg_j = Σ_i S·G over slot j's expert columns and the slot
//     terms of dℓ; waves 2-7: DSd row-major.
//  5. dℓ row-major and transposed (rows Kx.. of DSdᵀ's array).
// Tiles are ordered so that each XCD holds a contiguous token range: the
// 32-byte pieces the tile writes into the transposed rows merge in one L2.
constexpr int kFusedThreads = 512;
constexpr int kFusedMaxKx = 128, kFusedMaxC = 768;

template <typename T>
__global__ __launch_bounds__(kFusedThreads) void bwd_route_fused_kernel(
    const float* __restrict__ logits, const int* __restrict__ inds, const int* __restrict__ cnt,
    const float* __restrict__ dloss, const T* __restrict__ x, const T* __restrict__ dO,
    const T* __restrict__ a_frag, const T* __restrict__ b_frag, int N, int E, int k, int r, int kx, int ep, int np,
    int C, T* __restrict__ dsd, T* __restrict__ dl, T* __restrict__ rT, T* __restrict__ sgdT, T* __restrict__ xt,
    T* __restrict__ dot, T* __restrict__ sgd, unsigned long long* __restrict__ emask) {
  constexpr int VEC = 8, NT = kFusedThreads, NW = NT / 64, TOK = kRouteTok;
  constexpr int NRT = TOK * 8, NR = NT - NRT;            // routing threads; row-staging threads
  constexpr int NQ = 2 * (kFusedMaxKx / 16) / NW;        // S and G 16-column blocks per wave
  constexpr int MAXKS = kFusedMaxC / 32;
  constexpr int LB = 2 * TOK * (kFusedMaxC / VEC) / NR;  // 16-byte row loads per staging thread
  static_assert(LB >= 5, "the routing waves' values ride in the row registers");
  using UM = Mma16<T>;
  typedef typename UM::frag ufrag;
  union Pack4 {
    T e[4];
    uint2 u;
  };
  __shared__ float lgs[TOK][65], dls[TOK][65], gE[TOK][64];
  __shared__ int ids[TOK][kBwdMaxK], cnts[2][64];
  extern __shared__ __attribute__((aligned(16))) unsigned char dyn[];
  const int XSS = C + 8, KXS = kx + 8;  // LDS row strides (16-byte aligned rows)
  T* xs = (T*)dyn;
  T* os = xs + TOK * XSS;
  T* sS = os + TOK * XSS;
  T* sG = sS + TOK * KXS;
  T* sD = sG + TOK * KXS;
  T* sSd = sD + TOK * KXS;  // SGd = g·S (row-major output only)
  const int tile = (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
  const int t0 = tile * TOK, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int nt = N - t0;  // live tokens of the tile (at most TOK used; <= 0 for padding tiles)
  const int nks = C / 32, nb = kx / 16;
  const int tl = tid >> 3, sub = tid & 7, t = t0 + tl;
  const bool rthread = tid < NRT;
  const bool live = rthread && t < N;
  const int cpr = C / VEC, per = TOK * cpr;

  // 1. loads (buffer loads: past-the-end reads give 0).  Routing threads:
  //    logits of experts sub + 8i (rv[0..1]), their counts (rv[2..3]) and
  //    slot sub's id (rv[4].x), all of token t.
  u32x4 rv[LB];
  if (rthread) {
    const __amdgpu_buffer_rsrc_t rl_ = buf_rsrc(logits, (unsigned)N * E * 4);
    const __amdgpu_buffer_rsrc_t rc_ = buf_rsrc(cnt, (unsigned)E * 4);
    const __amdgpu_buffer_rsrc_t ri_ = buf_rsrc(inds, (unsigned)N * k * 4);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = sub + 8 * i;
      rv[i >> 2][i & 3] = buf_load4(rl_, live && e < E ? ((unsigned)t * E + e) * 4u : kOOB);
      rv[2 + (i >> 2)][i & 3] = buf_load4(rc_, e < E ? (unsigned)e * 4u : kOOB);
    }
    rv[4][0] = buf_load4(ri_, live && sub < k ? ((unsigned)t * k + sub) * 4u : kOOB);
  } else {
    const __amdgpu_buffer_rsrc_t rx_ = buf_rsrc(x, (unsigned)N * C * sizeof(T));
    const __amdgpu_buffer_rsrc_t ro_ = buf_rsrc(dO, (unsigned)N * C * sizeof(T));
#pragma unroll
    for (int j = 0; j < LB; ++j) {
      const int i = (tid - NRT) + j * NR;
      const int which = i >= per ? 1 : 0, rem = i - which * per;
      const int rl = rem / cpr, c = (rem - rl * cpr) * VEC;
      const unsigned off = i < 2 * per && rl < nt ? ((unsigned)(t0 + rl) * C + c) * (unsigned)sizeof(T) : kOOB;
      rv[j] = buf_load16(which ? ro_ : rx_, off);
    }
  }
  // 2·nb = NQ·NW blocks: S blocks 0..nb-1, G blocks nb..2nb-1; block b = wave + q·NW
  ufrag bf[NQ][MAXKS];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int b = wave + q * NW;
    const bool isG = b >= nb;
    const T* src = (isG ? b_frag : a_frag) + ((size_t)(isG ? b - nb : b) * nks * 64 + lane) * 8;
#pragma unroll
    for (int j = 0; j < MAXKS; ++j) bf[q][j] = *(const ufrag*)(src + (size_t)min(j, nks - 1) * 512);
  }

  // 2. routing waves: gates and the softmax / aux / z part of dℓ.  The LDS
  //    values a thread reads were written by threads of its own wave.
  int ej[kBwdMaxK];
  float gtj[kBwdMaxK];
#pragma unroll
  for (int j = 0; j < kBwdMaxK; ++j) {
    ej[j] = -1;
    gtj[j] = 0.f;
  }
  if (rthread) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      lgs[tl][sub + 8 * i] = __uint_as_float(rv[i >> 2][i & 3]);
      cnts[wave][sub + 8 * i] = (int)rv[2 + (i >> 2)][i & 3];
    }
    ids[tl][sub] = live && sub < k ? (int)rv[4][0] : -1;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    if (live) {
      float m = 0.f, den = 0.f, ex[kBwdMaxK];
#pragma unroll
      for (int j = 0; j < kBwdMaxK; ++j) {
        ex[j] = 0.f;
        if (j < k) {
          const int raw = ids[tl][j];
          ej[j] = raw >= 0 && raw < E ? raw : -1;  // the forward writes only valid ids; others carry no gradient
          const float l = lgs[tl][ej[j] >= 0 ? ej[j] : 0];
          if (j == 0) m = l;
          ex[j] = expf(l - m);
          den += ex[j];
        }
      }
#pragma unroll
      for (int j = 0; j < kBwdMaxK; ++j)
        if (j < k) gtj[j] = ex[j] / den;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = sub + 8 * i;
      float g = 0.f;
#pragma unroll
      for (int j = 0; j < kBwdMaxK; ++j)
        if (ej[j] == e) g = rnd<T>(gtj[j]);
      gE[tl][e] = g;
    }
    if (emask && live && sub == 0) {
      unsigned long long msk = 0;
#pragma unroll
      for (int j = 0; j < kBwdMaxK; ++j)
        if (ej[j] >= 0) msk |= 1ull << ej[j];
      emask[t] = msk;
    }
    const float* lr = lgs[tl];
    const int* cw = cnts[wave];
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
      pf += p * ((float)cw[e] * inv_nk);
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
    for (int e = sub; e < 64; e += 8) {
      float v = 0.f;
      if (live && e < E) {
        const float P = expf(lr[e] - mx) / sp;
        v = caux * P * ((float)cw[e] * inv_nk - pf) + cz * P;
      }
      dls[tl][e] = v;
    }
  } else {
#pragma unroll
    for (int j = 0; j < LB; ++j) {
      const int i = (tid - NRT) + j * NR;
      if (i < 2 * per) {
        const int which = i >= per ? 1 : 0, rem = i - which * per;
        const int rl = rem / cpr, c = (rem - rl * cpr) * VEC;
        *(u32x4*)((which ? os : xs) + rl * XSS + c) = rv[j];
      }
    }
  }
  __syncthreads();

  // 3a. xᵀ / dOᵀ while the weight fragments land: one 8-token x 8-column
  //     block per thread (C <= 768), 16-byte LDS reads, transposed in
  //     registers, 16-byte stores
  {
    const int ncg = C / VEC, na = (xt ? 1 : 0) + (dot ? 1 : 0);
    if (tid < na * 2 * ncg) {
      const int cg = tid % ncg, rest = tid / ncg, h = rest & 1;
      const bool isO = (rest >> 1) == 1 || !xt;
      const T* src = (isO ? os : xs) + h * 8 * XSS + cg * VEC;
      u32x4 in[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) in[v] = *(const u32x4*)(src + v * XSS);
      T* dst = (isO ? dot : xt) + (size_t)(cg * VEC) * np + t0 + h * 8;
#pragma unroll
      for (int cc = 0; cc < 8; ++cc) {
        const int w = cc >> 1, sh = (cc & 1) * 16;
        u32x4 o;
#pragma unroll
        for (int u = 0; u < 4; ++u) o[u] = ((in[2 * u][w] >> sh) & 0xFFFFu) | (((in[2 * u + 1][w] >> sh) & 0xFFFFu) << 16);
        *(u32x4*)(dst + (size_t)cc * np) = o;
      }
    }
  }
  // 3b. S / G blocks on MFMA (A operand: the tile's rows from LDS), gated epilogue
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int b = wave + q * NW;
    const bool isG = b >= nb;
    const T* arow = (isG ? os : xs) + (lane & 15) * XSS + (lane >> 4) * UM::KV;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < MAXKS; ++j)
      if (j < nks) acc = UM::run(*(const ufrag*)(arow + j * UM::KS), bf[q][j], acc);
    const int col = (isG ? b - nb : b) * 16 + (lane & 15), e = col / r;
    T* raw = isG ? sG : sS;
    Pack4 pk;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int tk = (lane >> 4) * 4 + v;
      const T sv = from_f<T>(acc[v]);
      const float g = e < E ? gE[tk][e] : 0.f;
      raw[tk * KXS + col] = sv;
      pk.e[v] = from_f<T>(g * to_f(sv));
      if (isG) sD[tk * KXS + col] = pk.e[v];
      else sSd[tk * KXS + col] = pk.e[v];
    }
    T* dstT = isG ? rT : sgdT;
    if (dstT) *(uint2*)(dstT + (size_t)col * np + t0 + (lane >> 4) * 4) = pk.u;
  }
  __syncthreads();

  // 4. dg and the slot terms of dℓ (waves 0-1); DSd row-major (waves 2-7)
  if (rthread) {
    float dg = 0.f;
    int es = -1;
#pragma unroll
    for (int j = 0; j < kBwdMaxK; ++j)
      if (j == sub) es = ej[j];
    if (live && es >= 0) {
      const T* sr = sS + tl * KXS + es * r;
      const T* gr = sG + tl * KXS + es * r;
      for (int i = 0; i < r; ++i) dg += to_f(sr[i]) * to_f(gr[i]);
    }
    float dgj[kBwdMaxK], sdg = 0.f;
#pragma unroll
    for (int j = 0; j < kBwdMaxK; ++j) {
      dgj[j] = __shfl(dg, j, 8);
      sdg += gtj[j] * dgj[j];
    }
    if (live) {
      for (int e = sub; e < E; e += 8) {
        float v = dls[tl][e];
#pragma unroll
        for (int j = 0; j < kBwdMaxK; ++j)
          if (ej[j] == e) v += gtj[j] * (dgj[j] - sdg);
        dls[tl][e] = v;
      }
    }
  } else {
    const int vpr = kx / VEC, nrow = (sgd ? 2 : 1) * TOK * vpr;
    for (int i = tid - NRT; i < nrow; i += NR) {
      const int which = i >= TOK * vpr ? 1 : 0, rem = i - which * TOK * vpr;
      const int rl = rem / vpr, q = rem - rl * vpr;
      if (rl < nt)
        *(u32x4*)((which ? sgd : dsd) + (size_t)(t0 + rl) * kx + q * VEC) =
            *(const u32x4*)((which ? sSd : sD) + rl * KXS + q * VEC);
    }
  }
  __syncthreads();

  // 5. dℓ: row-major (tokens < N) and transposed (rows kx.. of rT)
  for (int i = tid; i < TOK * (ep / VEC); i += NT) {
    const int rl = i / (ep / VEC), q = i - rl * (ep / VEC);
    if (rl >= nt) continue;
    Chunk<T> c;
#pragma unroll
    for (int j = 0; j < VEC; ++j) c.e[j] = from_f<T>(q * VEC + j < 64 ? dls[rl][q * VEC + j] : 0.f);
    *(u32x4*)(dl + (size_t)(t0 + rl) * ep + q * VEC) = c.raw;
  }
  for (int i = tid; rT && i < ep * (TOK / VEC); i += NT) {
    const int e = i / (TOK / VEC), q = i - e * (TOK / VEC);
    Chunk<T> c;
#pragma unroll
    for (int j = 0; j < VEC; ++j) c.e[j] = from_f<T>(e < 64 ? dls[q * VEC + j][e] : 0.f);
    *(u32x4*)(rT + (size_t)(kx + e) * np + t0 + q * VEC) = c.raw;
  }
}

// Token-contracted products of the backward, per expert, for layers on the
// fused routing path.  With I_t the experts selected for token t:
//   dA_e[c][i] = Σ_{t: e ∈ I_t} x[t][c] · DSd[t][e·r+i]
//   dB_e[i][c] = Σ_{t: e ∈ I_t} SGd[t][e·r+i] · dO[t][c]
//   dW_gate[e][c] = Σ_t dℓ[t][e] · x[t][c]
// The dense products over Kx = E·r columns do E/k times the work of the
// first two.  Workgroup (e, token range, 64-column tile), for w < E·R·CT:
// the range's tokens routed to e (from the per-token expert masks), in token
// order, 128 at a time.  Every load of a chunk is issued together — the x
// and dO pieces of the tile as 8-token x 8-column blocks, expert e's DSd /
// SGd columns — and the next chunk's go out while the current one is on the
// MFMA; x and dO are transposed in registers and stored to LDS, and the
// contraction over tokens runs on v_mfma_f32_16x16x32 (K = tokens; DSd, SGd
// padded to 16-column blocks).  The workgroups past E·R·CT compute dW_gate
// the same way over every token of shorter ranges (dℓ columns as the second
// operand).  Each workgroup writes fp32 partials for its range, which
// bwd_finish_expert sums in range order, so the result is deterministic.
// About 52 KB of LDS: three workgroups share a CU.
constexpr int kXThreads = 256, kXChunk = 128, kXCW = 64, kXRow = kXChunk + 8;  // LDS row: 128 tokens + 16 B
constexpr int kXMaxTT = 2048;  // tokens per range at most (the token list lives in LDS)

template <typename T>
__global__ __launch_bounds__(kXThreads) void bwd_expert_kernel(
    const T* __restrict__ x, const T* __restrict__ dO, const T* __restrict__ dsd, const T* __restrict__ sgd,
    const T* __restrict__ dl, const unsigned long long* __restrict__ emask, int N, int C, int E, int r, int kx,
    int ep, int TT, int R, int TTW, int CT, int RPA, float* __restrict__ part_a, float* __restrict__ part_b,
    float* __restrict__ part_w) {
  using UM = Mma16<T>;
  typedef typename UM::frag ufrag;
  extern __shared__ __attribute__((aligned(16))) unsigned char dyn[];
  T* xT = (T*)dyn;            // [kXCW][kXRow]: x columns of the tile, tokens of the chunk
  T* oT = xT + kXCW * kXRow;  // dO columns
  T* aT = oT + kXCW * kXRow;  // [RPA][kXRow]: DSd columns of expert e, or dℓ columns
  T* bT = aT + RPA * kXRow;   // [RPA][kXRow]: SGd columns of expert e
  __shared__ int toks[kXMaxTT];
  __shared__ int wsum[kXThreads / 64];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int nA = E * R * CT;
  const bool kindA = (int)blockIdx.x < nA;
  int e = 0, rng, ct;
  if (kindA) {
    ct = blockIdx.x % CT;
    rng = (blockIdx.x / CT) % R;
    e = blockIdx.x / (CT * R);
  } else {
    ct = (blockIdx.x - nA) % CT;
    rng = (blockIdx.x - nA) / CT;
  }
  const int c0 = ct * kXCW;
  const int t0 = rng * (kindA ? TT : TTW);
  const int tend = min(N, t0 + (kindA ? TT : TTW));
  const int RP = kindA ? (r + 15) / 16 * 16 : (E + 15) / 16 * 16;  // rows of the second operand, 16-padded

  // token list: the range's tokens routed to e, in token order (kind A)
  int n;
  if (kindA) {
    // every mask word of the range first (loads in flight together)
    const __amdgpu_buffer_rsrc_t rm = buf_rsrc(emask, (unsigned)N * 8u);
    unsigned long long mk[kXMaxTT / kXThreads];
#pragma unroll
    for (int it = 0; it < kXMaxTT / kXThreads; ++it) {
      mk[it] = 0;
      if (t0 + it * kXThreads < tend) {  // (uniform: no load is issued past the range)
        const int t = t0 + it * kXThreads + tid;
        const unsigned off = t < tend ? (unsigned)t * 8u : kOOB;
        mk[it] = buf_load4(rm, off) | ((unsigned long long)buf_load4(rm, off + 4u) << 32);
      }
    }
    n = 0;
#pragma unroll
    for (int it = 0; it < kXMaxTT / kXThreads; ++it) {
      const int b0 = t0 + it * kXThreads;
      if (b0 >= tend) break;
      const int t = b0 + tid;
      const bool f = t < tend && ((mk[it] >> e) & 1ull);
      const unsigned long long bal = __ballot(f);
      const int pre = __popcll(bal & ((1ull << lane) - 1ull));
      if (lane == 0) wsum[wave] = __popcll(bal);
      __syncthreads();
      int base = n;
      for (int w = 0; w < wave; ++w) base += wsum[w];
      if (f) toks[base + pre] = t;
      int tot = 0;
      for (int w = 0; w < kXThreads / 64; ++w) tot += wsum[w];
      n += tot;
      __syncthreads();
    }
  } else {
    n = max(0, tend - t0);
  }

  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, (unsigned)N * C * sizeof(T));
  const __amdgpu_buffer_rsrc_t ro = buf_rsrc(dO, (unsigned)N * C * sizeof(T));
  const __amdgpu_buffer_rsrc_t rs = buf_rsrc(kindA ? ((tid >> 7) ? sgd : dsd) : dl,
                                             (unsigned)N * (kindA ? kx : ep) * sizeof(T));
  const bool vec2 = kindA ? r % 8 == 0 : true;  // second operand by 16-byte loads
  const int width = kindA ? r : E;
  // this thread's share of a chunk.  Kind A: one 8x8 block of x (tid < 128)
  // or dO (tid >= 128), and token p = tid & 127's DSd (tid < 128) or SGd
  // columns.  Kind W: one block of x (tid < 128); token tid - 128's dℓ columns.
  const int blk = tid & 127, to = blk >> 3, co = blk & 7;
  const bool arrO = kindA && tid >= 128;
  const bool doBlk = kindA || tid < 128;
  const int sp = kindA ? (tid & 127) : tid - 128;  // token of the second-operand loads (kind W: tid >= 128)
  const bool doSec = kindA || tid >= 128;
  u32x4 in[8];
  Chunk<T> sv[8];  // second-operand values (2-byte loads: sv[i / 8].e[i % 8])
  auto issue = [&](int q0) {
    const int nq = min(kXChunk, n - q0);
    const int c = c0 + co * 8;
    if (doBlk) {  // (uniform per wave)
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const int p = to * 8 + v;
        const int t = p < nq ? (kindA ? toks[q0 + p] : t0 + q0 + p) : -1;
        const unsigned off = t >= 0 && c < C ? ((unsigned)t * C + c) * (unsigned)sizeof(T) : kOOB;
        in[v] = buf_load16(arrO ? ro : rx, off);
      }
    }
    const bool ok = doSec && sp < nq;
    const int t = ok ? (kindA ? toks[q0 + sp] : t0 + q0 + sp) : 0;
    const unsigned base = ((unsigned)t * (kindA ? kx : ep) + (kindA ? e * r : 0)) * (unsigned)sizeof(T);
    if (vec2) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        sv[j].raw = zero4();
        if (j * 8 < width && doSec) sv[j].raw = buf_load16(rs, ok ? base + j * 16u : kOOB);  // (uniform)
      }
    } else {
#pragma unroll
      for (int i = 0; i < 32; ++i)
        sv[i >> 3].e[i & 7] =
            __builtin_bit_cast(T, buf_load2(rs, ok && i < width ? base + i * (unsigned)sizeof(T) : kOOB));
    }
  };
  auto stash = [&]() {
    if (doBlk) {
      T* dst = (arrO ? oT : xT) + (co * 8) * kXRow + to * 8;
#pragma unroll
      for (int cc = 0; cc < 8; ++cc) {
        const int w = cc >> 1, sh = (cc & 1) * 16;
        u32x4 o;
#pragma unroll
        for (int h = 0; h < 4; ++h)
          o[h] = ((in[2 * h][w] >> sh) & 0xFFFFu) | (((in[2 * h + 1][w] >> sh) & 0xFFFFu) << 16);
        *(u32x4*)(dst + cc * kXRow) = o;
      }
    }
    if (doSec) {
      T* dst = (kindA && tid >= 128 ? bT : aT) + sp;
#pragma unroll
      for (int i = 0; i < 64; ++i)
        if (i < RP) dst[i * kXRow] = i < width ? sv[i >> 3].e[i & 7] : from_f<T>(0.f);
    }
  };

  const int nblk = 4 * (RP / 16);  // 16x16 output blocks per product (<= 8 for kind A, <= 16 for kind W)
  f32x4 acc[2][4];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[a][q] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (n > 0) issue(0);
  for (int q0 = 0; q0 < n; q0 += kXChunk) {
    stash();
    __syncthreads();
    if (q0 + kXChunk < n) issue(q0 + kXChunk);  // the next chunk's loads, in flight during the products
    // block j = (second-operand block ib, column block cb) of wave j % 4.
    // Kind A (j < 8): dA as D[c][i] in acc[0], dB as D[i][c] in acc[1];
    // kind W (j < 16): D[c][e] in acc[j / 8][j / 4 % 2]
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int j = wave + q * 4;
      if (j < nblk && (q < 2 || !kindA)) {
        const int cb = j & 3, ib = j >> 2;
        f32x4& d0 = acc[q >> 1][q & 1];
#pragma unroll
        for (int ks = 0; ks < kXChunk / 32; ++ks) {
          const int ko = ks * 32 + (lane >> 4) * 8;
          const ufrag fx = *(const ufrag*)(xT + (cb * 16 + (lane & 15)) * kXRow + ko);
          const ufrag fa = *(const ufrag*)(aT + (ib * 16 + (lane & 15)) * kXRow + ko);
          d0 = UM::run(fx, fa, d0);
          if (kindA) {
            const ufrag fb = *(const ufrag*)(bT + (ib * 16 + (lane & 15)) * kXRow + ko);
            const ufrag fo = *(const ufrag*)(oT + (cb * 16 + (lane & 15)) * kXRow + ko);
            acc[1][2 + q] = UM::run(fb, fo, acc[1][2 + q]);
          }
        }
      }
    }
    __syncthreads();
  }

  // fp32 partials of this range; accumulator v of a lane is D[m][n] with
  // m = (lane >> 4)·4 + v, n = lane & 15
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int j = wave + q * 4;
    if (j >= nblk || (q >= 2 && kindA)) continue;
    const int cb = j & 3, ib = j >> 2;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = (lane >> 4) * 4 + v, nn = lane & 15;
      if (kindA) {
        const int c = c0 + cb * 16 + m, i = ib * 16 + nn;  // dA: D[c][i]
        if (c < C && i < r) part_a[(((size_t)e * R + rng) * C + c) * r + i] = acc[0][q][v];
        const int i2 = ib * 16 + m, c2 = c0 + cb * 16 + nn;  // dB: D[i][c]
        if (c2 < C && i2 < r) part_b[(((size_t)e * R + rng) * r + i2) * C + c2] = acc[1][2 + q][v];
      } else {
        const int c = c0 + cb * 16 + m, ee = ib * 16 + nn;  // dW: D[c][e]
        if (c < C && ee < E) part_w[((size_t)rng * E + ee) * C + c] = acc[q >> 1][q & 1][v];
      }
    }
  }
}

// dA, dB and dW_gate of the per-expert path: the range partials summed in
// range order, rounded to T once.  Null outputs are skipped.
template <typename T>
__global__ __launch_bounds__(256) void bwd_finish_expert_kernel(const float* __restrict__ part_a,
                                                                const float* __restrict__ part_b,
                                                                const float* __restrict__ part_w, int E, int C, int r,
                                                                int R, int RW, T* __restrict__ dA, T* __restrict__ dB,
                                                                T* __restrict__ dwg) {
  const size_t i = blockIdx.x * (size_t)256 + threadIdx.x;
  const size_t per = (size_t)C * r;  // elements of one expert's dA (and dB)
  const size_t na = dA ? E * per : 0, nb = dB ? E * per : 0, nw = dwg ? (size_t)E * C : 0;
  // partials q = 0..n-1 at src + q·stride, added in ascending q; loads go
  // out 8 at a time
  auto sum = [](const float* src, size_t stride, int n) {
    float a = src[0];
    for (int q0 = 1; q0 < n; q0 += 8) {
      float b[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) b[u] = src[(size_t)min(q0 + u, n - 1) * stride];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (q0 + u < n) a += b[u];
    }
    return a;
  };
  if (i < na + nb) {
    const bool isB = i >= na;
    const size_t j = isB ? i - na : i;
    const size_t e = j / per, rem = j - e * per;
    (isB ? dB : dA)[j] = from_f<T>(sum((isB ? part_b : part_a) + e * R * per + rem, per, R));
  } else if (i < na + nb + nw) {
    const size_t j = i - na - nb;
    dwg[j] = from_f<T>(sum(part_w + j, (size_t)E * C, RW));
  }
}

// The backward's last step: dA[e][c][i] = O[c][e·r+i] and dW_gate[e][c] =
// O[c][kx+e] for the merged product O = xᵀ·[DSd | dℓ] (C x (kx + ep)) and,
// when dB's product was split, dB = the sum of its partials.  A split
// product (ks > 1) is read from its fp32 partials, summed in ascending split
// order and rounded to T once, as the GEMM's split-K reduction does, so the
// results equal that reduction followed by the copy; ks <= 1: O is read as
// stored.  Null outputs are skipped.
template <typename T>
__global__ __launch_bounds__(256) void bwd_finish_kernel(const float* __restrict__ part_o, int ks_o,
                                                         const T* __restrict__ o, int E, int C, int r, int kx, int ep,
                                                         T* __restrict__ dA, T* __restrict__ dwg,
                                                         const float* __restrict__ part_b, int ks_b,
                                                         T* __restrict__ dB) {
  const size_t i = blockIdx.x * (size_t)256 + threadIdx.x;
  const size_t na = dA ? (size_t)E * C * r : 0;
  const size_t nw = dwg ? (size_t)E * C : 0;
  const size_t nbk = dB && ks_b > 1 ? (size_t)E * r * C : 0;
  const int ow = kx + ep;
  auto o_at = [&](size_t at) -> T {
    if (ks_o <= 1) return o[at];
    const size_t plane = (size_t)C * ow;
    float a = part_o[at];
    for (int q = 1; q < ks_o; ++q) a += part_o[q * plane + at];
    return from_f<T>(a);
  };
  if (i < na) {
    const int e = (int)(i / ((size_t)C * r));
    const int rem = (int)(i - (size_t)e * C * r);
    const int c = rem / r, j = rem - c * r;
    dA[i] = o_at((size_t)c * ow + e * r + j);
  } else if (i < na + nw) {
    const size_t w = i - na;
    const int e = (int)(w / C), c = (int)(w - (size_t)e * C);
    dwg[w] = o_at((size_t)c * ow + kx + e);
  } else if (i < na + nw + nbk) {
    const size_t j = i - na - nw, plane = (size_t)E * r * C;
    float a = part_b[j];
    for (int q = 1; q < ks_b; ++q) a += part_b[q * plane + j];
    dB[j] = from_f<T>(a);
  }
}

}  // namespace

hipError_t launch_transpose_pad(int dtype, const void* src, int R, int W, int lds, void* dst, int Rp, hipStream_t s,
                                int batch, long long sstride, long long dstride) {
  if (W % 64 || Rp % 64 || lds % 8 || batch < 1) return hipErrorInvalidValue;
  const dim3 grid(W / 64, Rp / 64, batch);
  RWKV_DISPATCH_DTYPE(dtype, T, {
    launch_kernel(transpose_pad_kernel<T>, grid, dim3(256), 0, s, (const T*)src, R, W, lds, (T*)dst, Rp,
                       sstride, dstride);
  });
  return mark(hipGetLastError(), "bwd_transpose", s);
}

hipError_t launch_bwd_prep(int dtype, const void* A, const void* B, const void* wg, int E, int C, int r, int kx,
                           int ep, bool frag, void* a_all, void* a_t, void* b_rows, void* wgt, const int* inds, int nk,
                           int* cnt, hipStream_t s) {
  if (frag && (kx % 16 || C % 32)) return hipErrorInvalidValue;
  const size_t total = 3 * (size_t)kx * C + (size_t)C * ep;
  const dim3 grid((unsigned)((total + 255) / 256 + (cnt ? 1 : 0)));
  RWKV_DISPATCH_DTYPE(dtype, T, {
    launch_kernel(bwd_prep_kernel<T>, grid, dim3(256), 0, s, (const T*)A, (const T*)B, (const T*)wg, E, C, r, kx,
                       ep, frag ? 1 : 0, (T*)a_all, (T*)a_t, (T*)b_rows, (T*)wgt, inds, nk, cnt);
  });
  return mark(hipGetLastError(), "bwd_prep", s);
}

hipError_t launch_ortho_mask(int dtype, void* gram, int er, int r, int kx, const float* d_ortho, hipStream_t s) {
  const dim3 grid((unsigned)(((size_t)kx * kx + 255) / 256));
  RWKV_DISPATCH_DTYPE(dtype, T, {
    launch_kernel(ortho_mask_kernel<T>, grid, dim3(256), 0, s, (T*)gram, er, r, kx, d_ortho);
  });
  return mark(hipGetLastError(), "ortho_mask", s);
}

hipError_t launch_bwd_route(int dtype, const float* logits, const int* inds, const void* S, const void* G,
                            const int* cnt, const float* dloss, int N, int E, int k, int r, int kx, int ep, int np,
                            void* dsd, void* dl, void* rT, void* sgdT, void* sgd, unsigned long long* emask,
                            hipStream_t s, bool g16) {
  if (k > kBwdMaxK || E > 64 || ep < 64 || ep % 64 || kx % 64 || np % kRouteTok) return hipErrorInvalidValue;
  const dim3 grid(np / kRouteTok);
  RWKV_DISPATCH_DTYPE(dtype, T, {
    launch_kernel(bwd_route_kernel<T>, grid, dim3(kRouteThreads), 0, s, logits, inds, (const T*)S, (const T*)G,
                       cnt, dloss, N, E, k, r, kx, ep, np, (T*)dsd, (T*)dl, (T*)rT, (T*)sgdT, (T*)sgd, emask,
                       g16 ? 1 : 0);
  });
  return mark(hipGetLastError(), "bwd_route", s);
}

hipError_t launch_bwd_route_fused(int dtype, const float* logits, const int* inds, const int* cnt, const float* dloss,
                                  int N, int E, int k, int r, int kx, int ep, int np, int C, const void* x,
                                  const void* dO, const void* a_frag, const void* b_frag, void* dsd, void* dl, void* rT,
                                  void* sgdT, void* xt, void* dot, void* sgd, unsigned long long* emask,
                                  hipStream_t s) {
  if (!bwd_route_fuses(dtype, kx, C) || k > kBwdMaxK || E > 64 || ep < 64 || ep % 64 || np % (8 * kRouteTok))
    return hipErrorInvalidValue;
  const dim3 grid(np / kRouteTok);  // a multiple of 8: one contiguous token range per XCD
  const size_t smem = (size_t)kRouteTok * (2 * (C + 8) + 4 * (kx + 8)) * 2;
  RWKV_DISPATCH_DTYPE(dtype, T, {
    if constexpr (sizeof(T) == 2) {
      auto launch = [&](auto kern) {
        if (smem > 65536) {
          const hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   (int)smem);
          if (e != hipSuccess) return e;
        }
        launch_kernel(kern, grid, dim3(kFusedThreads), smem, s, logits, inds, cnt, dloss, (const T*)x,
                           (const T*)dO, (const T*)a_frag, (const T*)b_frag, N, E, k, r, kx, ep, np, C, (T*)dsd,
                           (T*)dl, (T*)rT, (T*)sgdT, (T*)xt, (T*)dot, (T*)sgd, emask);
        return hipSuccess;
      };
      const hipError_t e = launch(bwd_route_fused_kernel<T>);
      if (e != hipSuccess) return e;
    }
  });
  return mark(hipGetLastError(), "bwd_route_fused", s);
}

BwdExpertPlan bwd_expert_plan(int N, int C, int E, int k) {
  BwdExpertPlan pl;
  pl.CT = (C + kXCW - 1) / kXCW;
  // the shortest ranges (multiples of 512 tokens) that keep the workgroups
  // within three per CU; the dW_gate ranges hold about as many tokens as a
  // range routes to one expert
  for (pl.TT = 512;; pl.TT += 512) {
    pl.R = (N + pl.TT - 1) / pl.TT;
    int ttw = (pl.TT * k + E - 1) / E;
    ttw = (ttw + 127) / 128 * 128;
    pl.TTW = std::min(std::max(ttw, 128), pl.TT);
    pl.RW = (N + pl.TTW - 1) / pl.TTW;
    if (pl.TT >= kXMaxTT || (long long)pl.CT * (E * pl.R + pl.RW) <= 3LL * num_cus()) break;
  }
  return pl;
}

hipError_t launch_bwd_expert(int dtype, const void* x, const void* dO, const void* dsd, const void* sgd, const void* dl,
                             const unsigned long long* emask, int N, int C, int E, int r, int kx, int ep,
                             const BwdExpertPlan& pl, float* part_a, float* part_b, float* part_w, hipStream_t s) {
  if (dtype == 0 || r > 32 || E > 64 || pl.TT > kXMaxTT || N <= 0) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(E * pl.R * pl.CT + pl.RW * pl.CT));
  const int rpa = std::max((r + 15) / 16 * 16, (E + 15) / 16 * 16);  // rows of each second-operand buffer
  const size_t smem = (size_t)(2 * kXCW + 2 * rpa) * kXRow * 2;
  RWKV_DISPATCH_DTYPE(dtype, T, {
    if constexpr (sizeof(T) == 2) {
      auto kern = bwd_expert_kernel<T>;
      if (smem > 65536) {
        const hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)smem);
        if (e != hipSuccess) return e;
      }
      launch_kernel(kern, grid, dim3(kXThreads), smem, s, (const T*)x, (const T*)dO, (const T*)dsd,
                         (const T*)sgd, (const T*)dl, emask, N, C, E, r, kx, ep, pl.TT, pl.R, pl.TTW, pl.CT, rpa,
                         part_a, part_b, part_w);
    }
  });
  return mark(hipGetLastError(), "bwd_expert", s);
}

hipError_t launch_bwd_finish_expert(int dtype, const float* part_a, const float* part_b, const float* part_w, int E,
                                    int C, int r, int R, int RW, void* dA, void* dB, void* dwg, hipStream_t s) {
  const size_t total = (dA ? (size_t)E * C * r : 0) + (dB ? (size_t)E * C * r : 0) + (dwg ? (size_t)E * C : 0);
  if (total == 0) return hipSuccess;
  const dim3 grid((unsigned)((total + 255) / 256));
  RWKV_DISPATCH_DTYPE(dtype, T, {
    launch_kernel(bwd_finish_expert_kernel<T>, grid, dim3(256), 0, s, part_a, part_b, part_w, E, C, r, R,
                       RW, (T*)dA, (T*)dB, (T*)dwg);
  });
  return mark(hipGetLastError(), "bwd_finish_expert", s);
}

bool bwd_route_fuses(int dtype, int kx, int C) {
  return dtype != 0 && kx == kFusedMaxKx && C <= kFusedMaxC && C % 32 == 0;
}

hipError_t launch_bwd_finish(int dtype, const float* part_o, int ks_o, const void* o, int E, int C, int r, int kx,
                             int ep, void* dA, void* dwg, const float* part_b, int ks_b, void* dB, hipStream_t s) {
  const size_t total = (dA ? (size_t)E * C * r : 0) + (dwg ? (size_t)E * C : 0) +
                       (dB && ks_b > 1 ? (size_t)E * r * C : 0);
  if (total == 0) return hipSuccess;
  const dim3 grid((unsigned)((total + 255) / 256));
  RWKV_DISPATCH_DTYPE(dtype, T, {
    launch_kernel(bwd_finish_kernel<T>, grid, dim3(256), 0, s, part_o, ks_o, (const T*)o, E, C, r, kx, ep,
                       (T*)dA, (T*)dwg, part_b, ks_b, (T*)dB);
  });
  return mark(hipGetLastError(), "bwd_finish", s);
}

}  // namespace rwkvmoe
