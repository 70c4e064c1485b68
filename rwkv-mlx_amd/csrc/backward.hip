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
//   dA_all_T = xᵀ · DSd           (C, Kx)  K = tokens
//   dB_rows  = SGdᵀ · dO          (E·r, C) = dB in its (E, r, C) layout
//   dW_gate  = dℓᵀ · x            (E, C)
//   dx       = DSd · A_allᵀᵀ + dℓ · W_gate   (one K-extended GEMM)
// Products whose K runs over tokens take operands transposed once
// (transpose_pad_kernel: token-contiguous rows, zero-padded to Np tokens).
#include "common.h"
#include "internal.h"

namespace rwkvmoe {
namespace {

// dst (W rows x Rp columns) = srcᵀ for src (R rows x W columns, row stride
// lds); columns R..Rp-1 of dst are zero.  64x64 tiles through LDS (float
// holds every element type exactly).
template <typename T>
__global__ __launch_bounds__(256) void transpose_pad_kernel(const T* __restrict__ src, int R, int W, int lds,
                                                            T* __restrict__ dst, int Rp) {
  __shared__ float tile[64][65];
  const int w0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += 4) {
    const int r = r0 + i, w = w0 + tx;
    tile[i][tx] = (r < R && w < W) ? to_f(src[(size_t)r * lds + w]) : 0.f;
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int w = w0 + i, r = r0 + tx;
    if (w < W && r < Rp) dst[(size_t)w * Rp + r] = from_f<T>(tile[tx][i]);
  }
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

constexpr int kRouteTok = 64;
constexpr int kBwdMaxK = 8;

// Per token (one thread each, 64 per workgroup), from the saved logits ℓ and
// selection: the gates g̃ = softmax(ℓ[I]) and their dtype cast g (the
// forward's values), dg_j = Σ_i S·G over the slot's expert columns, then
//   dℓ[I_j] += g̃_j (dg_j − Σ_i g̃_i dg_i)
//   dℓ      += d_aux·(E/N)·P ⊙ (f − <P, f>) + d_z·(2 lse / N)·P
// with P = softmax(ℓ), lse = log Σ exp ℓ, f = counts / (N k).  Then all
// threads write DSd / dℓ row-major (t < N) and DSdᵀ, SGdᵀ, dℓᵀ (zero for
// padding tokens N..Np-1).
template <typename T>
__global__ __launch_bounds__(256) void bwd_route_kernel(const float* __restrict__ logits, const int* __restrict__ inds,
                                                        const T* __restrict__ S, const T* __restrict__ G,
                                                        const int* __restrict__ cnt, const float* __restrict__ dloss,
                                                        int N, int E, int k, int r, int kx, int ep, int np,
                                                        T* __restrict__ dsd, T* __restrict__ dl, T* __restrict__ dsdT,
                                                        T* __restrict__ sgdT, T* __restrict__ dlT) {
  __shared__ float dls[kRouteTok][65];
  __shared__ float gs[kRouteTok][kBwdMaxK];
  __shared__ int es[kRouteTok][kBwdMaxK];
  const int t0 = blockIdx.x * kRouteTok, tid = threadIdx.x;
  if (tid < kRouteTok) {
    const int tl = tid, t = t0 + tl;
    for (int e = 0; e < 64; ++e) dls[tl][e] = 0.f;
    for (int j = 0; j < kBwdMaxK; ++j) {
      es[tl][j] = -1;
      gs[tl][j] = 0.f;
    }
    if (t < N) {
      const float* lr = logits + (size_t)t * E;
      int ej[kBwdMaxK];
      float gt[kBwdMaxK], dg[kBwdMaxK];
      // gates: the forward's softmax over the selected logits, top-1 first
      float m = 0.f, den = 0.f;
      bool ok[kBwdMaxK];
      for (int j = 0; j < k; ++j) {
        const int raw = inds[(size_t)t * k + j];
        ok[j] = raw >= 0 && raw < E;  // the forward writes only valid ids; others carry no gradient
        ej[j] = ok[j] ? raw : 0;
        const float l = lr[ej[j]];
        if (j == 0) m = l;
        gt[j] = expf(l - m);
        den += gt[j];
      }
      float sdg = 0.f;
      for (int j = 0; j < k; ++j) {
        gt[j] = gt[j] / den;
        const T* sr = S + (size_t)t * kx + ej[j] * r;
        const T* gr = G + (size_t)t * kx + ej[j] * r;
        float acc = 0.f;
        for (int i = 0; i < r; ++i) acc += to_f(sr[i]) * to_f(gr[i]);
        dg[j] = ok[j] ? acc : 0.f;
        sdg += gt[j] * dg[j];
        es[tl][j] = ok[j] ? ej[j] : -1;
        gs[tl][j] = rnd<T>(gt[j]);
      }
      float mx = lr[0];
      for (int e = 1; e < E; ++e) mx = fmaxf(mx, lr[e]);
      float sp = 0.f, se = 0.f;
      for (int e = 0; e < E; ++e) {
        sp += expf(lr[e] - mx);
        se += expf(lr[e]);
      }
      const float lse = logf(se);
      const float inv_nk = 1.f / ((float)N * (float)k);
      float pf = 0.f;
      for (int e = 0; e < E; ++e) pf += expf(lr[e] - mx) / sp * ((float)cnt[e] * inv_nk);
      const float daux = dloss ? dloss[0] : 0.f, dz = dloss ? dloss[1] : 0.f;
      const float caux = daux * (float)E / (float)N, cz = dz * 2.f * lse / (float)N;
      for (int e = 0; e < E; ++e) {
        const float P = expf(lr[e] - mx) / sp;
        dls[tl][e] = caux * P * ((float)cnt[e] * inv_nk - pf) + cz * P;
      }
      for (int j = 0; j < k; ++j)
        if (ok[j]) dls[tl][ej[j]] += gt[j] * (dg[j] - sdg);
    }
  }
  __syncthreads();
  // the gate of expert column `col` for token row tl (0 when not selected)
  auto gate_of = [&](int tl, int col) {
    const int e = col / r;
    float g = 0.f;
    for (int j = 0; j < kBwdMaxK; ++j)
      if (es[tl][j] == e && col < E * r) g = gs[tl][j];
    return g;
  };
  for (int idx = tid; idx < kRouteTok * kx; idx += blockDim.x) {
    const int tl = idx / kx, col = idx - tl * kx, t = t0 + tl;
    if (t >= N) continue;
    dsd[(size_t)t * kx + col] = from_f<T>(gate_of(tl, col) * to_f(G[(size_t)t * kx + col]));
  }
  for (int idx = tid; idx < kRouteTok * ep; idx += blockDim.x) {
    const int tl = idx / ep, e = idx - tl * ep, t = t0 + tl;
    if (t >= N) continue;
    dl[(size_t)t * ep + e] = from_f<T>(e < E ? dls[tl][e] : 0.f);
  }
  for (int idx = tid; idx < kx * kRouteTok; idx += blockDim.x) {
    const int col = idx / kRouteTok, tl = idx - col * kRouteTok, t = t0 + tl;
    if (t >= np) continue;
    float vd = 0.f, vs = 0.f;
    if (t < N) {
      const float g = gate_of(tl, col);
      vd = g * to_f(G[(size_t)t * kx + col]);
      vs = g * to_f(S[(size_t)t * kx + col]);
    }
    dsdT[(size_t)col * np + t] = from_f<T>(vd);
    sgdT[(size_t)col * np + t] = from_f<T>(vs);
  }
  for (int idx = tid; idx < ep * kRouteTok; idx += blockDim.x) {
    const int e = idx / kRouteTok, tl = idx - e * kRouteTok, t = t0 + tl;
    if (t >= np) continue;
    dlT[(size_t)e * np + t] = from_f<T>(t < N && e < E ? dls[tl][e] : 0.f);
  }
}

// dA[e][c][i] = dA_all_T[c][e·r+i]
template <typename T>
__global__ __launch_bounds__(256) void relayout_da_kernel(const T* __restrict__ dat, int E, int C, int r, int kx,
                                                          T* __restrict__ dA) {
  const size_t i = blockIdx.x * (size_t)256 + threadIdx.x;
  const size_t total = (size_t)E * C * r;
  if (i >= total) return;
  const int e = (int)(i / ((size_t)C * r));
  const int rem = (int)(i - (size_t)e * C * r);
  const int c = rem / r, j = rem - c * r;
  dA[i] = dat[(size_t)c * kx + e * r + j];
}

}  // namespace

hipError_t launch_transpose_pad(int dtype, const void* src, int R, int W, int lds, void* dst, int Rp, hipStream_t s) {
  const dim3 grid((W + 63) / 64, (Rp + 63) / 64);
  RWKV_DISPATCH_DTYPE(dtype, T, {
    hipLaunchKernelGGL(transpose_pad_kernel<T>, grid, dim3(256), 0, s, (const T*)src, R, W, lds, (T*)dst, Rp);
  });
  return mark(hipGetLastError(), "bwd_transpose", s);
}

hipError_t launch_bwd_count(const int* inds, int nk, int E, int* cnt, hipStream_t s) {
  hipLaunchKernelGGL(bwd_count_kernel, dim3(1), dim3(1024), 0, s, inds, nk, E, cnt);
  return mark(hipGetLastError(), "bwd_count", s);
}

hipError_t launch_bwd_route(int dtype, const float* logits, const int* inds, const void* S, const void* G,
                            const int* cnt, const float* dloss, int N, int E, int k, int r, int kx, int ep, int np,
                            void* dsd, void* dl, void* dsdT, void* sgdT, void* dlT, hipStream_t s) {
  if (k > kBwdMaxK || E > 64 || np % kRouteTok) return hipErrorInvalidValue;
  const dim3 grid(np / kRouteTok);
  RWKV_DISPATCH_DTYPE(dtype, T, {
    hipLaunchKernelGGL(bwd_route_kernel<T>, grid, dim3(256), 0, s, logits, inds, (const T*)S, (const T*)G, cnt, dloss,
                       N, E, k, r, kx, ep, np, (T*)dsd, (T*)dl, (T*)dsdT, (T*)sgdT, (T*)dlT);
  });
  return mark(hipGetLastError(), "bwd_route", s);
}

hipError_t launch_relayout_da(int dtype, const void* dat, int E, int C, int r, int kx, void* dA, hipStream_t s) {
  const size_t total = (size_t)E * C * r;
  const dim3 grid((unsigned)((total + 255) / 256));
  RWKV_DISPATCH_DTYPE(dtype, T, {
    hipLaunchKernelGGL(relayout_da_kernel<T>, grid, dim3(256), 0, s, (const T*)dat, E, C, r, kx, (T*)dA);
  });
  return mark(hipGetLastError(), "bwd_relayout_da", s);
}

}  // namespace rwkvmoe
