// Host-side launchers shared between the translation units of librwkvmoe.
// Each returns hipSuccess or the launch error; shapes are validated by the
// C-ABI layer (api.hip) before any of these is called.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>

#include <tuple>
#include <utility>

#include "dispatch.h"
#include "losses.h"

namespace rwkvmoe {

// Per-kernel timing probe of rwkvmoe_forward_timed, set for the calling host
// thread while that entry point runs.  Two forms:
//   * between (pairs == false): mark() records ev[n + 1] on the launch stream
//     right after kernel n and stores its name; ev[0] is recorded before the
//     first launch.  An interval then holds the kernel and the cost of the
//     event records around it.
//   * pairs: launch n records its own begin and end timestamps into ev[2n]
//     and ev[2n + 1] (hipExtLaunchKernel), the kernel's duration alone, and
//     mark() names every launch since the previous mark.
// Without a probe, mark() only passes the launch status on.
struct Probe {
  hipEvent_t* ev;
  const char** names;
  int cap;     // kernels that can be recorded
  int n;       // between: kernels marked so far; pairs: kernels launched so far
  bool pairs;
  int named;   // pairs: launches named so far
};
Probe*& probe_slot();
// Compute units of the current device (read once per process).
int num_cus();
hipError_t mark(hipError_t launched, const char* name, hipStream_t s);

// Every kernel of the library is launched through here (the arguments are
// converted to the kernel's parameter types, as by hipLaunchKernelGGL).  A
// pairs probe gets the launch's begin / end events.  The launch status is
// left for hipGetLastError, which the launchers read after every launch.
template <typename... Formals, typename... Actuals>
void launch_kernel(void (*kernel)(Formals...), dim3 grid, dim3 block, unsigned shm, hipStream_t s,
                         Actuals... actuals) {
  static_assert(sizeof...(Formals) == sizeof...(Actuals), "kernel argument count");
  std::tuple<Formals...> f{std::move(actuals)...};
  void* args[sizeof...(Formals) + 1];
  std::apply([&](auto&... a) {
    int i = 0;
    ((args[i++] = (void*)&a), ...);
  }, f);
  hipEvent_t start = nullptr, stop = nullptr;
  if (Probe* p = probe_slot(); p && p->pairs) {
    if (p->n < p->cap) {
      start = p->ev[2 * p->n];
      stop = p->ev[2 * p->n + 1];
    }
    p->n++;
  }
  (void)hipExtLaunchKernel((const void*)kernel, grid, block, args, shm, s, start, stop, 0);
}

// Router: tokens handled per workgroup for a given C, E and element type.
int router_tile_tokens(int N, int C, int E, int dtype);
// With u: the adapter product U = gate ⊙ (x · A_allᵀ), A_all (at) in MFMA
// fragment order (launch_lora_prep with frag).  gate32: W_gate is fp32 (x
// 16-bit).  fpk = 2 (dtype f16, with u): fp32 adapters as fp16 pairs
// (launch_lora_prep with mixed); U is then written as [U_hi | 2^-11·U_hi |
// U_lo], N x 3·128.
// tt: tokens per router workgroup, 1..16 (router_tile_tokens' choice, or 16;
// 16 with `u`).
// The decode front (launch_router with `front`, N <= 64, 16-bit, E <= 16,
// no `u`): F / 32 workgroups computing the key projection
// h = relu(xk · W_keyᵀ)² and kx / 32 computing u = x · A_allᵀ (not
// gate-masked) for all tokens, in the router's launch.  h and u are written
// in fragment order (frag_pos) for 16·ceil(N/16) rows (zero past N).
struct DecodeFront {
  const void* wk;  // (F, C): row-major, or fragment order with wk_packed
  bool wk_packed;
  void* h;         // (16·nb, F) fragment order
  int F;
  const void* at;  // (kx, C) A_all in fragment order
  void* u;         // (16·nb, kx) fragment order
  int kx;
  void* g;         // (16·nb, kx) the gate of each adapter column, fragment order (rows < N)
};
hipError_t launch_router(int dtype, bool gate32, int fpk, const void* x, const void* wg, const float* bias,
                         const void* xprev, const void* mu, const void* at, int N, int T_, int C, int E, int k, int r,
                         float* logits, int* inds, void* gates, void* gate_dense, void* xk, void* u, double* part_f64,
                         int* part_cnt, int* loss_claim, int tt, hipStream_t s, const DecodeFront* front = nullptr,
                         const void* ln_w = nullptr, const void* ln_b = nullptr, void* xn = nullptr,
                         bool u_raw = false);
// u_raw (with u, fpk 1): u receives round(x·A_all) without the gates — the
// SPARSE value product's adapter operand — instead of U = w ⊙ round(x·A_all).
// ln_w / ln_b (many-token kernel only): x is the residual stream and the
// router normalizes its tile (ln2, ln.h's arithmetic) before every use;
// xn, when given, receives LN(x) (N, C) for the kernels that read it later.
// Whether the decode front (router + key and adapter tiles) applies.
bool decode_front_ok(int N, int C, int F, int E, int dtype, bool gate32);
// Decode value launch (decode.hip): out = h·W_valueᵀ + (g ⊙ u)·B_allᵀ
// (+ residual) for N <= 64 tokens; h (16·nb, F), u and g (16·nb, kx) from
// the decode front in fragment order (frag_pos), W_value row-major or
// (wv_packed) in fragment order.  With `loss`, one more workgroup reduces the
// router's loss partials.
hipError_t launch_decode_value(int dtype, const void* h, const void* wv, bool wv_packed, const void* u,
                               const void* g, const void* bt, const void* resid, void* out, int N, int C, int F,
                               int kx, const LossJob* loss, hipStream_t s);
// A 16-bit (R x K) row-major matrix to fragment order (frag_pos).
hipError_t launch_frag_pack(int dtype, const void* src, void* dst, int R, int K, hipStream_t s);
// Dynamic LDS bytes of one router workgroup (must stay within 160 KB).
size_t router_smem_bytes(int dtype, int N, int C, int E, bool gate32 = false, bool ln = false);
// Whether the router pass also produces U (adapter width E*r <= 128 and
// 16-token workgroups); otherwise the key GEMM does, as extra column tiles.
bool router_fuses_adapters(int N, int C, int E, int r, int dtype);
hipError_t launch_router_finalize(const LossJob& jb, hipStream_t s);

// Dispatch.
int dispatch_blocks(int nk);
bool dispatch_job_plan(const int* inds, int nk, int E, int* perm, int* inv, int* offsets, const int* router_cnt,
                       int router_tt, int k, int* ticket, DispatchJob* job);
// router_cnt: the router pass's per-workgroup expert counts of these ids
// ([e][block], router_tt tokens a block, k slots a token), or nullptr.
hipError_t launch_dispatch(const int* inds, int nk, int E, int* block_counts, int* perm, int* inv, int* offsets,
                           hipStream_t s, const int* router_cnt = nullptr, int router_tt = 0, int k = 0);

// GEMMs and the token-shift mix.
hipError_t launch_shift_mix(int dtype, const void* x, const void* xprev, const void* mu, void* xk, int N, int T,
                            int C, hipStream_t s);
// With u != null the key GEMM also produces U (N, kx) = gate ⊙ (x · A_allᵀ).
// With loss != null, the first of its workgroups to finish also reduces the
// router's loss partials.
// `part`: fp32 scratch for products whose K is split over work items (decode
// batches, small layers), gemm_partial_bytes of it.
hipError_t launch_cmix_key(int dtype, const void* xk, const void* wk, void* h, int N, int C, int F, const void* x,
                           const void* at, const void* gdense, int E, int r, int kx, void* u, const LossJob* loss,
                           float* part, hipStream_t s, const DispatchJob* disp = nullptr);
// The dispatch scatter over the router's per-workgroup expert counts as a
// job for another launch (launch_cmix_key's `disp`): false when the shape
// needs the standalone launches (launch_dispatch).  ticket: one int, zeroed
// by the router pass before the job's launch.
// `mixed` (dtype f16, fp32 adapters): u is [U_hi | 2^-11·U_hi | U_lo] (N x
// 3·kx) and bt [B_hi | B_lo' | B_hi] (C x 3·kx); the base product is rounded
// to fp16 before the K-extension adds the delta, and out (and the residual
// add) are fp32.  Unsplit tiles only (value_plan_mixed_ok).
hipError_t launch_cmix_value(int dtype, const void* h, const void* wv, int F, const void* u, const void* bt, int kx,
                             const void* resid, void* out, int N, int C, float* part, hipStream_t s,
                             bool mixed = false);
// SPARSE value product with the combine in its epilogue (EPI_COMBINE):
// out = round(h·W_valueᵀ + δ) (+ residual), δ from the adapter rows in
// assignment order (launch_combine with inv NULL), so the base never goes
// to memory and no combine launch follows.  16-bit layers with 16-bit rows,
// k <= kCombineMaxK, and a value plan with a VGPR-staged tile
// (value_combine_fusable); else hipErrorInvalidValue.
bool value_combine_fusable(int dtype, int N, int C, int F, int k);
hipError_t launch_cmix_value_combine(int dtype, const void* h, const void* wv, int F, const void* rows,
                                     const int* inds, const void* gates, const void* resid, void* out, int N, int C,
                                     int k, hipStream_t s);
// The SPARSE value product with the adapters in the same launch
// (EPI_SPARSE): out = round(h·W_valueᵀ + δ) (+ resid) with δ the combine of
// a_s = round(u_e·B_e) over the token's routed experts in ascending id, where
// u (N x kx, row stride kx) is the router's unscaled adapter product
// round(x·A_all) and bt is B_all (C x kx).  16-bit layers, kx = 128 holding
// every expert's r columns (r a multiple of 8), k <= kCombineMaxK, and a
// value plan with the 128x96 VGPR-staged tile (value_sparse_fusable); else
// hipErrorInvalidValue.
bool value_sparse_fusable(int dtype, int N, int C, int F, int E, int r, int k, int kx);
hipError_t launch_cmix_value_sparse(int dtype, const void* h, const void* wv, int F, const void* u, const void* bt,
                                    int kx, const int* inds, const void* gates, int E, int r, const void* resid,
                                    void* out, int N, int C, int k, hipStream_t s);
// Whether the 16-bit value product (m x n, K = k_total) plans an unsplit
// tile, which its mixed form needs.
bool value_plan_mixed_ok(int m, int n, int k_total);
// Bytes of split-K partials the (m x n, K = k_total) product needs (0: not split).
size_t gemm_partial_bytes(int dtype, int m, int n, int n_key, int k_total, bool keyad);
// out (m x n, row stride ldo) = a1 · b1ᵀ (+ a2 · b2ᵀ when k2 > 0): rows of
// every operand are K-contiguous; n and the K lengths as for the value GEMM.
// `hint` picks the tiling for the shapes of the backward (measured):
//   GEMM_HINT_AUTO      the forward's automatic plan;
//   GEMM_HINT_NO_SPLIT  short K: unsplit 128x64 tiles;
//   GEMM_HINT_SPLIT64   long K over a small output: 64x64 tiles, K split 8 ways.
enum { GEMM_HINT_AUTO = 0, GEMM_HINT_NO_SPLIT = 1, GEMM_HINT_SPLIT64 = 2 };
// With `deferred` not null, a product whose plan splits K leaves its fp32
// partials part[s][m][n] unreduced and sets *deferred to the split count (1:
// the product was not split and `out` holds it).
hipError_t launch_gemm_nt(int dtype, const void* a1, int lda1, const void* b1, int ldb1, int k1, const void* a2,
                          int lda2, const void* b2, int ldb2, int k2, int m, int n, void* out, int ldo, float* part,
                          const char* name, hipStream_t s, int hint = GEMM_HINT_AUTO, int* deferred = nullptr);
// Grouped product over expert-contiguous row segments: rows
// [offsets[e], offsets[e+1]) of a (m = offsets[n_groups] rows at most) times
// (b + e·bstride)ᵀ, each (n x k) with row stride ldb; relu² epilogue when
// relu2 (the key projection), plain store otherwise.
// `loss`: the router's loss reduction, run by the first workgroup to finish
// (nullptr: none).
hipError_t launch_grouped_gemm(int dtype, bool relu2, const void* a, int lda, const void* b, int ldb,
                               long long bstride, int k, int m, int n, const int* offsets, int n_groups, void* out,
                               int ldo, const char* name, hipStream_t s, const LossJob* loss = nullptr);
// Grouped-K product: out + g·ostride (m x n, row stride ldo) = a · bᵀ over
// the operand columns [koff[g], koff[g+1]) for g < n_groups (koff in device
// memory, each range a non-empty multiple of 128 elements); a is m rows of
// stride lda, b n rows of stride ldb.  n % 64 == 0.
hipError_t launch_gemm_grouped_k(int dtype, const void* a, int lda, const void* b, int ldb, const int* koff,
                                 int n_groups, int m, int n, void* out, int ldo, long long ostride, const char* name,
                                 hipStream_t s);
// Split-K partial bytes launch_gemm_nt needs for the product and hint.
size_t gemm_nt_partial_bytes(int dtype, int m, int n, int k_total, int hint = GEMM_HINT_AUTO);

// Full-expert layer (experts.hip): xk rows in perm order with each row's
// expert mix x_k[e] (mu is (E, C)).
hipError_t launch_experts_mix(int dtype, const void* x, const void* xprev, const void* mu, const int* perm,
                              const int* inds, int N, int T_, int C, int E, int k, void* xk, hipStream_t s);

// Full-expert backward (experts_bwd.hip); rows j in perm order (nk = N·k).
// dO rows gathered (dog, nk x C) and each row's gate gr (fp32, the forward's
// rounding) recomputed from logits and inds.
hipError_t launch_exb_gather(int dtype, const void* dO, const int* perm, const float* logits, const int* inds,
                             int nk, int C, int E, int k, void* dog, float* gr, hipStream_t s);
// From p (nk x F, the key product before relu²) and u = dO·W_val (nk x F):
// dw[j] = <relu(p)², u> (fp32) and dp = g·u·2·relu(p), written over u's rows
// when dp == U (each element is read before it is written).
hipError_t launch_exb_hidden(int dtype, const void* P, const void* U, const float* gr, int nk, int F, void* dp,
                             float* dw, hipStream_t s);
// The packed token ranges of the weight-gradient products (koff, E + 1
// ints): expert e's rows take columns [koff[e], koff[e+1]), its count
// rounded up to 128 (128 when it has none); exb_seg_cols(nk, E) bounds
// koff[E] (a multiple of 128).
hipError_t launch_exb_koff(const int* off, int E, int* koff, hipStream_t s);
int exb_seg_cols(int nk, int E);
// dst (W x ld) with range e (columns [koff[e], koff[e+1])) the transpose of
// src rows [off[e], off[e+1]) (nk x W), zero past the count.  mode 0 copies,
// 1 writes round(relu(v)²), 2 writes round(v · gr[row]).  W % 64, ld % 128.
hipError_t launch_exb_seg_transpose(int dtype, int mode, const void* src, int W, const int* off, const int* koff,
                                    int E, int ld, const float* gr, void* dst, hipStream_t s);
// Router cotangents dl (N x E, fp32) from the slot cotangents dw (perm
// order) and the loss cotangents (dloss: [d_aux, d_z] or null).
hipError_t launch_exb_route(const float* logits, const int* inds, const int* inv, const float* dw, const int* off,
                            const float* dloss, int N, int E, int k, float* dl, hipStream_t s);
// The standalone router's dl (N x E, fp32): the gates' cotangents d_gates
// (N x k, dtype, assignment order t·k + s; may be null) through the
// selected-logit softmax, plus the loss cotangents; counts from off.
hipError_t launch_router_route(int dtype, const float* logits, const int* inds, const int* inv, const void* d_gates,
                               const int* off, const float* dloss, int N, int E, int k, float* dl, hipStream_t s);
// dx (N x C) and, when dxprev is not null, d x_prev (B x C) from dk (nk x C,
// perm order), x_k (mu, E x C), dl and W_gate; dx may be null; with dk null
// only the logit term dl · W_gate (the standalone router).
hipError_t launch_exb_dx(int dtype, const void* dk, const int* inv, const int* inds, const void* mu, const float* dl,
                         const void* wg, int N, int T_, int C, int E, int k, void* dx, void* dxprev, hipStream_t s);
// Column sums in fixed row chunks, then their ordered sum into out (E x C):
// mode 0: d x_k[e] = Σ_{rows of e} a ⊙ round(shift(x) − x); mode 1:
// d W_gate[e] = Σ_t dl[t][e] · x[t].  part: E · exb_col_chunks(N, C, E) · C
// floats.
int exb_col_chunks(int N, int C, int E);
hipError_t launch_exb_colsum(int dtype, int mode, const void* a, const void* x, const void* xprev, const int* off,
                             const int* perm, const float* dl, int N, int T_, int C, int E, int k, float* part,
                             void* out, hipStream_t s);

// Backward helpers (backward.hip).
// dst (W x Rp) = transpose of src (R x W, row stride lds), columns R..Rp-1
// zero; a batch of such matrices at element strides sstride / dstride.
hipError_t launch_transpose_pad(int dtype, const void* src, int R, int W, int lds, void* dst, int Rp, hipStream_t s,
                                int batch = 1, long long sstride = 0, long long dstride = 0);
// A_all (kx, C), A_T (C, kx), B_rows (kx, C), W_gateᵀ (C, ep), zero-padded;
// with `frag`, A_all and B_rows in the fused routing kernel's fragment order.
// With cnt not null, one more workgroup (the first) counts the nk selections
// in inds per expert into cnt (E ints).
hipError_t launch_bwd_prep(int dtype, const void* A, const void* B, const void* wg, int E, int C, int r, int kx,
                           int ep, bool frag, void* a_all, void* a_t, void* b_rows, void* wgt, const int* inds, int nk,
                           int* cnt, hipStream_t s);
// Gram (kx x kx) -> 2·d_ortho·Gram off the diagonal r x r blocks, in place.
hipError_t launch_ortho_mask(int dtype, void* gram, int er, int r, int kx, const float* d_ortho, hipStream_t s);
// Routing gradient: DSd (N x kx) and dℓ (N x ep) row-major, [DSd | dℓ]ᵀ into
// rT ((kx + ep) x np) and SGdᵀ (kx x np), from S and G in memory; SGd
// row-major and the per-token expert masks when sgd / emask are given.
// rT and sgdT may be null (both or neither).
// g16 (fp32 dtype): the gates are rounded to fp16, as an fp16 layer with fp32
// adapters computed them.
hipError_t launch_bwd_route(int dtype, const float* logits, const int* inds, const void* S, const void* G,
                            const int* cnt, const float* dloss, int N, int E, int k, int r, int kx, int ep, int np,
                            void* dsd, void* dl, void* rT, void* sgdT, void* sgd, unsigned long long* emask,
                            hipStream_t s, bool g16 = false);
// The same with S and G computed inside from x, dO and the fragment-ordered
// A_all / B_rows (bwd_route_fuses: 16-bit, kx 128, C <= 768).  Outputs
// left null are skipped: rT and sgdT; xᵀ and dOᵀ (C x np, zero past N); SGd
// row-major (N x kx); the per-token expert masks (bit e: e selected).
hipError_t launch_bwd_route_fused(int dtype, const float* logits, const int* inds, const int* cnt, const float* dloss,
                                  int N, int E, int k, int r, int kx, int ep, int np, int C, const void* x,
                                  const void* dO, const void* a_frag, const void* b_frag, void* dsd, void* dl, void* rT,
                                  void* sgdT, void* xt, void* dot, void* sgd, unsigned long long* emask,
                                  hipStream_t s);
bool bwd_route_fuses(int dtype, int kx, int C);
// Per-expert token contractions (layers on the fused routing path): token
// ranges of TT tokens (R of them) for dA / dB, of TTW (RW) for dW_gate,
// 128-column tiles (CT).
struct BwdExpertPlan {
  int TT, R, TTW, RW, CT;
};
BwdExpertPlan bwd_expert_plan(int N, int C, int E, int k);
// fp32 partials: part_a (E, R, C, r), part_b (E, R, r, C), part_w (RW, E, C),
// from DSd / SGd (N x kx), dℓ (N x ep) and the per-token expert masks.
hipError_t launch_bwd_expert(int dtype, const void* x, const void* dO, const void* dsd, const void* sgd, const void* dl,
                             const unsigned long long* emask, int N, int C, int E, int r, int kx, int ep,
                             const BwdExpertPlan& pl, float* part_a, float* part_b, float* part_w, hipStream_t s);
// dA (E, C, r), dB (E, r, C), dW_gate (E, C) from those partials; null outputs skipped.
hipError_t launch_bwd_finish_expert(int dtype, const float* part_a, const float* part_b, const float* part_w, int E,
                                    int C, int r, int R, int RW, void* dA, void* dB, void* dwg, hipStream_t s);
// dA and dW_gate out of the merged product O = xᵀ·[DSd | dℓ] (C x (kx + ep)),
// read from its ks_o fp32 split partials (ks_o > 1) or from o; and dB from
// the ks_b partials of its product when ks_b > 1.  Null outputs are skipped.
hipError_t launch_bwd_finish(int dtype, const float* part_o, int ks_o, const void* o, int E, int C, int r, int kx,
                             int ep, void* dA, void* dwg, const float* part_b, int ks_b, void* dB, hipStream_t s);

// LoRA helpers, grouped LoRA, combine, orthogonality loss.
int lora_kx(int E, int r);
// A_all and B_all in one launch.
// A_all (kx x C; with `frag`, in MFMA fragment order, frag_pos — the form
// the router's adapter product reads) and B_all (C x kx).
// `mixed` (dtype f16, A and B fp32): the fp16 pair form of lora_prep_kernel
// (A_all 2·kx rows, B_all 3·kx columns).
hipError_t launch_lora_prep(int dtype, const void* A, const void* B, int E, int C, int r, int kx, void* at, void* bt,
                            hipStream_t s, bool frag = false, bool mixed = false);
// The row of perm position j is stored at ag row perm[j] (assignment order,
// the order of inds and gates).  `mixed` (dtype f16, fp32 adapters): at /
// bt are launch_lora_prep's mixed (row-major) operands and the adapter rows
// ag are fp32.  `valu`: the products on the vector ALUs
// (lora_grouped_valu_kernel; not mixed).
hipError_t launch_lora_grouped(int dtype, const void* x, const void* at, const void* bt, const int* perm,
                               const int* offsets, int N, int C, int E, int k, int r, int kx, void* ag, hipStream_t s,
                               bool mixed = false, bool valu = false);
// ag's rows: at inv[t·k + s] (perm order), or with inv NULL at t·k + s
// (assignment order).  `mixed` (dtype f16 or bf16): ag, δ and out are fp32;
// base, gates and the residual in dtype.
hipError_t launch_combine(int dtype, const void* base, const void* ag, const int* inds, const void* gates,
                          const int* inv, const void* resid, void* out, int N, int C, int k, hipStream_t s,
                          bool mixed = false);
hipError_t launch_ortho(int dtype, const void* A, int E, int C, int r, float* part, float* out, hipStream_t s);
// y = fp32(x) for n (a multiple of 8) elements of a 16-bit dtype
hipError_t launch_widen(int dtype, const void* x, float* y, size_t n, hipStream_t s);
// y = LN(x) per row of C (ln2 of the Block, norm.hip): fp64 statistics, one
// rounding to dtype by way of fp32.
hipError_t launch_layer_norm(int dtype, const void* x, const void* w, const void* b, void* y, int N, int C,
                             hipStream_t s);
// The VJP of ln2 (norm.hip): dx = LN's VJP of dy [+ dres] (dx may be NULL,
// and may alias dy or dres), dw = Σ dy·x̂ and db = Σ dy over rows (either
// may be NULL; with one of them, `part` holds layer_norm_bwd_part_bytes).
size_t layer_norm_bwd_part_bytes(int N, int C);
hipError_t launch_layer_norm_bwd(int dtype, const void* x, const void* w, const void* dy, const void* dres, void* dx,
                                 void* dw, void* db, float* part, int N, int C, hipStream_t s);

}  // namespace rwkvmoe
