/*
 * rwkvmoe.h — C ABI of librwkvmoe.so: the LoRA-MoE ChannelMix forward of
 * RWKV-v7 on AMD Instinct MI355X (gfx950).
 *
 * The reference path is `LoRAMoE_CMix.__call__` (rwkv_mlx/moe.py:129-147),
 * which composes
 *   - the frozen base ChannelMix `RWKV_CMix_x070.__call__` (rwkv_mlx/model.py:259-263)
 *     with its token shift `_time_shift` (rwkv_mlx/model.py:67-75),
 *   - the top-k `Router.__call__` (rwkv_mlx/moe.py:51-86),
 *   - E low-rank adapters (x @ A_e) @ B_e mixed by gate weight (rwkv_mlx/moe.py:138-147),
 *   - and, called by the Block after every forward, `orthogonal_loss`
 *     (rwkv_mlx/moe.py:149-163, rwkv_mlx/model.py:323).
 * The reference has no FFI of its own (it is an MLX nn.Module); these entry
 * points are what a ctypes binding of that module's forward binds.  The
 * Python mirror of the module lives in rwkv_mlx_amd/moe.py.
 *
 * Conventions
 *   - Every pointer is a device pointer unless stated, 16-byte aligned.
 *   - Tensors are dense row-major in the reference's layouts:
 *       x (B,T,C)  x_k (C)  w_key (F,C)  w_value (C,F)  w_gate (E,C)
 *       lora_A (E,C,r)  lora_B (E,r,C)  out (B,T,C)
 *     They share one element type (`dtype`), except that with a 16-bit
 *     dtype the flags RWKVMOE_GATE_F32 / RWKVMOE_ADAPTERS_F32 declare w_gate
 *     / lora_A and lora_B fp32, the layer the reference fine-tunes (an fp16
 *     base from convert.py with the fp32 router and adapters of
 *     moe.py:47, 124-125); MLX type promotion then fixes each op's dtype
 *     (see the flags).  The router's dot products follow an order-fixed
 *     definition (see rwkvmoe_router_topk).
 *   - Return codes: 0 success; < 0 argument error, detected on the host
 *     before any HIP call; > 0 a hipError_t passed through.
 *   - All work is enqueued on `stream` (a hipStream_t; NULL = default
 *     stream).  The library never allocates device memory, never frees,
 *     never synchronises the host and keeps no pointer after it returns.
 *     Scratch memory is the caller's `ws` of `rwkvmoe_workspace_bytes` bytes.
 *   - The library is stateless apart from a once-initialised device property
 *     cache; distinct host threads may call it on distinct streams.
 */
#ifndef RWKVMOE_H
#define RWKVMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types of x, the weights and out */
enum rwkvmoe_dtype { RWKVMOE_F32 = 0, RWKVMOE_F16 = 1, RWKVMOE_BF16 = 2 };

/* how the expert adapters are evaluated (identical semantics):
 *   FUSED  — the reference's dense masked loop (rwkv_mlx/moe.py:139-145)
 *            recast as two MFMA GEMM segments: U = gate ⊙ (x · A_all) is
 *            produced next to the router, and the value projection runs over
 *            K = F + E·r with operands [h | U] and [W_value | B_all]; out is
 *            written once.
 *   SPARSE — dispatch (histogram, scan, stable scatter into expert-major
 *            order), grouped per-expert LoRA on the routed rows only, and a
 *            token-owned gate-weighted combine into base (+ residual). */
enum rwkvmoe_mode { RWKVMOE_MODE_FUSED = 0, RWKVMOE_MODE_SPARSE = 1 };

/* flags */
#define RWKVMOE_HAS_PREV     1 /* x_prev (B,C) is the token before x[:,0] (RNN-mode state, model.py:498-506) */
#define RWKVMOE_HAS_BIAS     2 /* logit_bias (E) fp32 is added to the router logits */
#define RWKVMOE_ADD_RESIDUAL 4 /* out = residual + ffn_out (Block's x = x + ffn_out, model.py:321-322) */
/* Parameter element types that differ from `dtype` (no-ops when dtype is
 * RWKVMOE_F32).  MLX promotion decides every op (moe.py:56, 86, 138-147;
 * model.py:259-263):
 *   GATE_F32      w_gate is fp32: logits = fp32(x)·W_gate as stored, with
 *                 the fp32 definition of the chunked dot products; gates
 *                 are still cast to dtype (moe.py:86).
 *   ADAPTERS_F32  lora_A and lora_B are fp32: the base runs in dtype and
 *                 is rounded to it, while (x·A_e)·B_e, the gate-weighted
 *                 delta and out = base + delta (+ residual) are fp32, so
 *                 `out` (and adapter_rows) are fp32 tensors; gates stay in
 *                 dtype.  fp16 layers run it in either mode (fp16 pairs of
 *                 the fp32 operands); bf16 layers in SPARSE mode whatever
 *                 `mode` says (the grouped LoRA in fp32 on an fp32 copy of
 *                 x), since no pair of bf16 values holds fp32's 24 bits. */
#define RWKVMOE_GATE_F32     8
#define RWKVMOE_ADAPTERS_F32 16
/* rwkvmoe_backward only, with dtype RWKVMOE_F32: the forward whose VJP this
 * is kept its gates in fp16 (the fine-tune layer, an fp16 x and base with
 * fp32 gate and adapters: RWKVMOE_ADAPTERS_F32, moe.py:86), so the backward
 * rounds the gates to fp16 where that forward did.  The caller passes x
 * converted to fp32 (exact) and the fp32 parameters and d_out; every other
 * entry point rejects it (RWKVMOE_ERR_FLAGS). */
#define RWKVMOE_GATES_F16    32
/* SPARSE mode: the grouped LoRA products (x·A_e)·B_e on the vector ALUs
 * (v_dot2 into fp32) instead of MFMA blocks, the same rounding points; for
 * A/B measurements of that choice.  Ignored in FUSED mode; not with
 * RWKVMOE_ADAPTERS_F32 (RWKVMOE_ERR_FLAGS). */
#define RWKVMOE_LORA_VALU    64
/* x is the Block's residual stream before ln2 (model.py:321): the layer runs
 * on y = LN(x), per token (x - mean) / sqrt(var + 1e-5) · ln_weight +
 * ln_bias (nn.LayerNorm(C), model.py:283; _layer_norm_1d, model.py:434-438):
 * mean and 1 / sqrt(var + 1e-5) over the row in fp64 (an order-fixed sum),
 * then ((x - mean)·rstd)·ln_weight + ln_bias in fp32, rounded to dtype.
 * ln_weight and ln_bias (C) are in dtype.  x_prev
 * (RWKVMOE_HAS_PREV) is the previous token's y — the RNN state of
 * model.py:413-416.  When x_ln is given it receives y (the next RNN state).
 * With RWKVMOE_ADD_RESIDUAL and residual = x, out is the Block's
 * x + ffn(ln2(x)) (model.py:321-322).  rwkvmoe_forward, rwkvmoe_decode,
 * rwkvmoe_forward_noalloc and rwkvmoe_experts_forward take it; every other
 * entry point rejects it (RWKVMOE_ERR_FLAGS). */
#define RWKVMOE_LN_IN        128

typedef struct rwkvmoe_desc {
  int32_t batch;     /* B */
  int32_t seq_len;   /* T (1 for a decode step) */
  int32_t d_model;   /* C, multiple of 64 */
  int32_t d_ffn;     /* F, multiple of 64 */
  int32_t n_experts; /* E, 1..64 */
  int32_t top_k;     /* k, 1..min(E,8) */
  int32_t lora_rank; /* r, 1..32 */
  int32_t dtype;     /* enum rwkvmoe_dtype */
  int32_t mode;      /* enum rwkvmoe_mode */
  int32_t flags;     /* RWKVMOE_* flags */
} rwkvmoe_desc;

typedef struct rwkvmoe_tensors {
  /* sizeof(rwkvmoe_tensors) as the caller compiled it: every entry point
   * taking this struct rejects any other value (RWKVMOE_ERR_VERSION), so a
   * caller built against another layout of the struct is refused instead of
   * having pointers read past its end */
  uint64_t struct_size;
  /* inputs */
  const void* x;           /* (B,T,C) */
  const void* x_prev;      /* (B,C) when RWKVMOE_HAS_PREV, else NULL */
  const void* x_k;         /* (C)    base.x_k (reference shape (1,1,C)) */
  const void* w_key;       /* (F,C)  base.key.weight */
  const void* w_value;     /* (C,F)  base.value.weight */
  const void* w_gate;      /* (E,C)  router.gate.weight (fp32 with RWKVMOE_GATE_F32) */
  const void* lora_A;      /* (E,C,r) (fp32 with RWKVMOE_ADAPTERS_F32) */
  const void* lora_B;      /* (E,r,C) (fp32 with RWKVMOE_ADAPTERS_F32) */
  const float* logit_bias; /* (E) fp32 when RWKVMOE_HAS_BIAS, else NULL */
  const void* residual;    /* (B,T,C) when RWKVMOE_ADD_RESIDUAL, else NULL */
  /* outputs */
  void* out;               /* (B,T,C), dtype; fp32 with RWKVMOE_ADAPTERS_F32 */
  float* losses;           /* [2] fp32: aux_loss, z_loss (moe.py:84, :62) */
  /* optional outputs / stage operands (NULL: held in the workspace) */
  float* logits;           /* (N,E) fp32 router logits (bias included) */
  int32_t* inds;           /* (N,k) selected experts, descending logit, ties to the lower id */
  void* gates;             /* (N,k) softmax over the selected logits, in dtype */
  void* gate_dense;        /* (N,E) the gates scattered to expert columns, 0 elsewhere */
  int32_t* perm;           /* (N*k) assignment ids t*k+slot in stable expert-major order */
  int32_t* inv_perm;       /* (N*k) position of assignment t*k+slot in perm */
  int32_t* offsets;        /* (E+1) exclusive prefix of per-expert counts */
  void* hidden;            /* (N,F) relu(shift-mixed x · W_keyᵀ)² */
  void* base_out;          /* (N,C) hidden · W_valueᵀ, dtype */
  void* adapter_rows;      /* (N*k,C) (x·A_e)·B_e per assignment t*k+slot (SPARSE); fp32 with RWKVMOE_ADAPTERS_F32 */
  float* ortho_loss;       /* [1] fp32 Σ_{i<j} ||A_iᵀ A_j||_F² (moe.py:149-163), or NULL */
  /* optional input */
  const void* prepared;    /* lora_A / lora_B laid out by rwkvmoe_prepare_adapters for a desc
                              of the same d_model, n_experts, lora_rank, dtype and flags; the
                              forward then reads them from here and launches no layout pass.
                              NULL: the forward lays them out in its workspace. */
  const void* prepared_base; /* w_key / w_value laid out by rwkvmoe_prepare_base for a desc of the
                              same d_model, d_ffn and dtype; read by the decode launches (a FUSED
                              forward of at most 64 tokens), ignored otherwise.  NULL: the decode
                              launches read w_key / w_value as stored. */
  /* with RWKVMOE_LN_IN (NULL otherwise) */
  const void* ln_weight;   /* (C) ln2.weight, dtype */
  const void* ln_bias;     /* (C) ln2.bias, dtype */
  void* x_ln;              /* (B,T,C) optional output: LN(x), dtype */
} rwkvmoe_tensors;

/* Operands of the backward (rwkvmoe_backward).  All device pointers; element
 * type = desc->dtype unless noted.  Any gradient output may be NULL (not
 * computed). */
typedef struct rwkvmoe_grads {
  /* forward inputs */
  const void* x;           /* (B,T,C) */
  const void* w_gate;      /* (E,C)  router.gate.weight */
  const void* lora_A;      /* (E,C,r) */
  const void* lora_B;      /* (E,r,C) */
  /* saved by the forward (rwkvmoe_tensors.logits / .inds of the same call) */
  const float* logits;     /* (N,E) fp32 router logits (bias included) */
  const int32_t* inds;     /* (N,k) selected experts */
  /* cotangents */
  const void* d_out;       /* (B,T,C) d loss / d out */
  const float* d_losses;   /* [2] fp32: d loss / d aux_loss, d loss / d z_loss; NULL: both 0 */
  /* gradients (written, not accumulated) */
  void* d_x;               /* (B,T,C) */
  void* d_lora_A;          /* (E,C,r) */
  void* d_lora_B;          /* (E,r,C) */
  void* d_w_gate;          /* (E,C) */
  /* rwkvmoe_ortho_backward only */
  const float* d_ortho;    /* [1] fp32 d loss / d ortho_loss; NULL: 1 */
} rwkvmoe_grads;

/* Operands of rwkvmoe_experts_backward (the full-expert layer).  All device
 * pointers; element type = desc->dtype unless noted.  Any gradient output
 * may be NULL (not computed). */
typedef struct rwkvmoe_experts_grads {
  /* forward inputs */
  const void* x;           /* (B,T,C) */
  const void* x_prev;      /* (B,C) when RWKVMOE_HAS_PREV, else NULL */
  const void* x_k;         /* (E,C)   (reference shape (E,1,1,C)) */
  const void* w_key;       /* (E,F,C) expert_key */
  const void* w_value;     /* (E,C,F) expert_val */
  const void* w_gate;      /* (E,C)   router.gate.weight */
  /* saved by the forward (rwkvmoe_tensors.logits / .inds of the same call) */
  const float* logits;     /* (N,E) fp32 router logits (bias included) */
  const int32_t* inds;     /* (N,k) selected experts */
  /* cotangents */
  const void* d_out;       /* (B,T,C) d loss / d out */
  const float* d_losses;   /* [2] fp32: d loss / d aux_loss, d loss / d z_loss; NULL: both 0 */
  /* gradients (written, not accumulated) */
  void* d_x;               /* (B,T,C) */
  void* d_x_prev;          /* (B,C), RWKVMOE_HAS_PREV only */
  void* d_x_k;             /* (E,C) */
  void* d_w_key;           /* (E,F,C) */
  void* d_w_value;         /* (E,C,F) */
  void* d_w_gate;          /* (E,C) */
} rwkvmoe_experts_grads;

/* Operands of rwkvmoe_router_backward (the standalone Router's VJP).  All
 * device pointers; element type = desc->dtype unless noted. */
typedef struct rwkvmoe_router_grads {
  /* forward inputs */
  const void* x;           /* (B,T,C) */
  const void* w_gate;      /* (E,C)  router.gate.weight */
  /* saved by the forward (rwkvmoe_tensors.logits / .inds of the same call) */
  const float* logits;     /* (N,E) fp32 router logits (bias included) */
  const int32_t* inds;     /* (N,k) selected experts */
  /* cotangents */
  const void* d_gates;     /* (N,k) d loss / d gates (the forward's `gates`); NULL: 0 */
  const float* d_losses;   /* [2] fp32: d loss / d aux_loss, d loss / d z_loss; NULL: both 0 */
  /* gradients (written, not accumulated) */
  void* d_x;               /* (B,T,C) */
  void* d_w_gate;          /* (E,C) */
} rwkvmoe_router_grads;

/* Operands of rwkvmoe_layer_norm_backward (the VJP of the Block's ln2).
 * All device pointers; element type = desc->dtype. */
typedef struct rwkvmoe_ln_grads {
  /* forward inputs */
  const void* x;           /* (B,T,C) ln2's input (the Block's residual stream) */
  const void* ln_weight;   /* (C) ln2.weight */
  /* cotangents */
  const void* d_y;         /* (B,T,C) d loss / d LN(x): a layer VJP's d_x taken at x = LN(x) */
  const void* d_res;       /* (B,T,C) added to d_x (the cotangent of the residual branch); NULL: none */
  /* gradients (written, not accumulated; any may be NULL) */
  void* d_x;               /* (B,T,C); may alias d_y or d_res */
  void* d_ln_weight;       /* (C) */
  void* d_ln_bias;         /* (C) */
} rwkvmoe_ln_grads;

/* status codes (< 0: argument errors found on the host before any HIP call) */
#define RWKVMOE_OK              0
#define RWKVMOE_ERR_NULL_DESC  -1 /* desc or tensors pointer is NULL */
#define RWKVMOE_ERR_SHAPE      -2 /* a dimension is out of range or not a multiple of 64 */
#define RWKVMOE_ERR_DTYPE      -3 /* dtype is not an rwkvmoe_dtype */
#define RWKVMOE_ERR_NULL_PTR   -4 /* a tensor the entry point requires is NULL */
#define RWKVMOE_ERR_ALIGN      -5 /* a tensor pointer is not suitably aligned */
#define RWKVMOE_ERR_WORKSPACE  -6 /* ws is NULL or ws_bytes < rwkvmoe_workspace_bytes */
#define RWKVMOE_ERR_TOPK       -7 /* top_k outside 1..min(n_experts, 8) */
#define RWKVMOE_ERR_FLAGS      -8 /* unknown flag, or a flag without its tensor */
#define RWKVMOE_ERR_MODE       -9 /* mode is not an rwkvmoe_mode, or decode without T == 1 and x_prev */
#define RWKVMOE_ERR_EVENTS    -10 /* rwkvmoe_forward_timed: missing or too few events */
#define RWKVMOE_ERR_SCRATCH   -11 /* rwkvmoe_forward_noalloc: the layer needs more scratch than the library holds */
#define RWKVMOE_ERR_VERSION   -12 /* rwkvmoe_tensors.struct_size is not this library's sizeof(rwkvmoe_tensors) */

/* bytes of device scratch rwkvmoe_forward_noalloc holds per GPU (64 MiB) */
#define RWKVMOE_NOALLOC_SCRATCH_BYTES 67108864

/* most kernels one forward launches (rwkvmoe_forward_timed) */
#define RWKVMOE_MAX_KERNELS 16
/* events that select rwkvmoe_forward_timed's per-launch (start, stop) form */
#define RWKVMOE_TIMED_PAIR_EVENTS 32

/* Human-readable text for a status code returned by any entry point. */
const char* rwkvmoe_status_string(int status);

/* Library version as MAJOR*10000 + MINOR*100 + PATCH (200: rwkvmoe_tensors
 * leads with struct_size; 100 had no such field). */
int rwkvmoe_version(void);

/* Scratch bytes of rwkvmoe_router_backward for `desc` (host only). */
int rwkvmoe_router_backward_workspace_bytes(const rwkvmoe_desc* desc, size_t* bytes);

/* VJP of the standalone Router (rwkv_mlx/moe.py:35-86, an nn.Module MLX
 * differentiates): given the cotangents of its outputs (gates, aux_loss,
 * z_loss; the indices are integers), d_x = dℓ·W_gate and
 * d_w_gate = dℓᵀ·x with dℓ (N,E) the logits' cotangent — the softmax
 * Jacobian over the selected logits applied to d_gates, plus the aux term
 * d_aux·(E/N)·P⊙(f − <P,f>) and the z term d_z·(2·lse/N)·P (P = softmax(ℓ),
 * f_e the selection counts over N·k, as moe.py:76-84 defines aux).  The
 * selection and counts are piecewise constant (no gradient); the gates'
 * cast to dtype passes its cotangent through.  Reductions run in a fixed
 * order (two calls are bit-identical).  Only RWKVMOE_HAS_BIAS is accepted
 * among the flags (the saved logits include the bias; it gets no
 * gradient); d_ffn and lora_rank are not used. */
int rwkvmoe_router_backward(const rwkvmoe_desc* desc, const rwkvmoe_router_grads* g, void* ws, size_t ws_bytes,
                            void* stream);

/* Scratch bytes of rwkvmoe_layer_norm_backward for `desc` (host only). */
int rwkvmoe_layer_norm_backward_workspace_bytes(const rwkvmoe_desc* desc, size_t* bytes);

/* VJP of the Block's ln2 in front of the ChannelMix (rwkv_mlx/model.py:321,
 * x + ffn(ln2(x)) with nn.LayerNorm(C), model.py:283, which MLX autodiff
 * differentiates in a training step).  With x̂ = (x - mean)·rstd (the
 * statistics of the RWKVMOE_LN_IN forward, eps 1e-5) and g = d_y·ln_weight:
 *   d_x = rstd·(g - mean(g) - x̂·mean(g·x̂)) + d_res,
 *   d_ln_weight = Σ_rows d_y·x̂,   d_ln_bias = Σ_rows d_y,
 * row sums in fp64, the rest in fp32, outputs rounded to dtype.  Column
 * sums run in a fixed order (two calls are bit-identical).  A training
 * step of the Block form runs the layer's forward with RWKVMOE_LN_IN and
 * x_ln, the layer's VJP (rwkvmoe_backward / rwkvmoe_experts_backward) with
 * x = x_ln, then this call with d_y = that VJP's d_x.  desc: any desc the
 * forward accepts (dtype, batch, seq_len and d_model are used).  Requires
 * x, ln_weight, d_y. */
int rwkvmoe_layer_norm_backward(const rwkvmoe_desc* desc, const rwkvmoe_ln_grads* g, void* ws, size_t ws_bytes,
                                void* stream);

/* Bytes of scratch `ws` that rwkvmoe_forward (and each stage entry point)
 * needs for `desc`.  Host-only; returns < 0 on an invalid desc.
 * Replaces nothing in the reference (MLX allocates lazily inside mx.eval). */
int rwkvmoe_workspace_bytes(const rwkvmoe_desc* desc, size_t* bytes);

/* Bytes of the buffer rwkvmoe_prepare_adapters fills for `desc` (only its
 * d_model, n_experts, lora_rank, dtype and flags matter).  Host-only. */
int rwkvmoe_prepared_bytes(const rwkvmoe_desc* desc, size_t* bytes);

/* Lays out lora_A (E,C,r) and lora_B (E,r,C) (moe.py:124-125) the way the
 * forward's kernels read them (A_all in MFMA fragment order and row-major,
 * B_all with the reduction index innermost; fp16 pairs with
 * RWKVMOE_ADAPTERS_F32) into `prepared` (256-byte aligned, at least
 * rwkvmoe_prepared_bytes).  For callers whose adapters stay constant over
 * many forwards (inference): pass the buffer as rwkvmoe_tensors.prepared and
 * each forward skips its layout pass.  After the adapters change the buffer
 * must be prepared again.  No counterpart in the reference (MLX reads the
 * parameters as stored). */
int rwkvmoe_prepare_adapters(const rwkvmoe_desc* desc, const void* lora_A, const void* lora_B, void* prepared,
                             size_t prepared_bytes, void* stream);

/* Bytes of the buffer rwkvmoe_prepare_base fills for `desc` (only its
 * d_model, d_ffn and dtype matter; fp16 / bf16 layers).  Host-only. */
int rwkvmoe_prepared_base_bytes(const rwkvmoe_desc* desc, size_t* bytes);

/* Lays out the frozen base ChannelMix weights w_key (F,C) and w_value (C,F)
 * (model.py:256-257) in MFMA fragment order, the layout the decode launches
 * read with one contiguous kilobyte per wave load, into `prepared_base`
 * (256-byte aligned, at least rwkvmoe_prepared_base_bytes).  For decode loops
 * (the base is frozen: moe.py:131 stops its gradient): pass the buffer as
 * rwkvmoe_tensors.prepared_base.  After the base weights change the buffer
 * must be prepared again.  No counterpart in the reference. */
int rwkvmoe_prepare_base(const rwkvmoe_desc* desc, const void* w_key, const void* w_value, void* prepared_base,
                         size_t prepared_bytes, void* stream);

/* Host-only query: *reads = 1 when rwkvmoe_forward (rwkvmoe_decode,
 * rwkvmoe_forward_noalloc) for `desc` reads rwkvmoe_tensors.prepared_base —
 * the two-launch decode path of a FUSED forward of at most 64 tokens
 * (16-bit, at most 16 experts, no fp32 adapters, no bf16 layer with an fp32
 * gate) when the caller requests no `hidden` output — else 0, so a caller
 * lays the base out only when a forward will read it.  No counterpart in
 * the reference. */
int rwkvmoe_reads_prepared_base(const rwkvmoe_desc* desc, int* reads);

/* Whole forward: (out, aux_loss, z_loss) = LoRAMoE_CMix(x) — moe.py:129-147,
 * plus ortho_loss when t->ortho_loss != NULL (model.py:323, moe.py:149-163).
 * Required: x, x_k, w_key, w_value, w_gate, lora_A, lora_B, out, losses. */
int rwkvmoe_forward(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t,
                    void* ws, size_t ws_bytes, void* stream);

/* rwkvmoe_forward without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Scratch is a device array of RWKVMOE_NOALLOC_SCRATCH_BYTES that the library
 * holds on each GPU it runs on until the process ends; layers whose
 * rwkvmoe_workspace_bytes exceeds it get RWKVMOE_ERR_SCRATCH (the headline
 * D=768 layer at 4096 tokens needs 32 MiB FUSED, 49 MiB SPARSE).  Calls no
 * allocating routine.  All calls on one GPU share its scratch: calls that
 * overlap on one GPU (other streams or host threads) race.  Same tensors,
 * outputs and argument checks as rwkvmoe_forward.  The scratch's device
 * address is looked up on a device's first call: make that call outside a
 * HIP graph capture (a first call under capture returns
 * hipErrorStreamCaptureUnsupported); later calls may be captured and
 * replayed. */
int rwkvmoe_forward_noalloc(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t, void* stream);

/* RNN-mode decode step for a batch of independent sequences: T must be 1 and
 * RWKVMOE_HAS_PREV set; the new shift state is x itself (model.py:498-506,
 * which the reference cannot run on MoE blocks).  Same tensors as forward.
 * A FUSED forward or decode of at most 64 tokens (fp16, or bf16 without
 * RWKVMOE_GATE_F32; n_experts <= 16; no RWKVMOE_ADAPTERS_F32; t->hidden
 * NULL) runs as two launches: the router with the key projection and the
 * adapter down-projection, then the value projection with the gated adapter
 * K-extension and the loss reduction. */
int rwkvmoe_decode(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t,
                   void* ws, size_t ws_bytes, void* stream);

/* rwkvmoe_forward with per-kernel timing.  No counterpart in the reference
 * (MLX offers no per-kernel timing); it serves throughput measurement.
 * Launches exactly what rwkvmoe_forward launches.  `events` holds n_events
 * hipEvent_t handles created by the caller:
 *   - n_events >= RWKVMOE_TIMED_PAIR_EVENTS: launch i records its own begin
 *     and end timestamps into events[2i] and events[2i + 1] (the kernel's
 *     duration alone, as a kernel trace reports it); names[i] names launch i
 *     (several launches of one step share a name) and *n_kernels counts the
 *     launches;
 *   - else n_events >= RWKVMOE_MAX_KERNELS + 1: events[0] is recorded on
 *     `stream` before the first kernel and events[i + 1] right after step i
 *     (an interval then includes the event records), names[i] names step i
 *     and *n_kernels counts the steps.
 * names has RWKVMOE_MAX_KERNELS entries of static strings. */
int rwkvmoe_forward_timed(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t,
                          void* ws, size_t ws_bytes, void* stream,
                          void* const* events, int n_events,
                          const char** names, int* n_kernels);

/* ---- stage entry points (parity tests and per-kernel profiling) ---------- */

/* Router (moe.py:51-86): logits = fp32(Σ_q acc_q) with the 64-wide chunk
 * sums acc_q (ascending c, one fused multiply-add per term: in fp32 when x
 * and W_gate are 16-bit, whose products are exact in fp32; in fp64 when
 * either is fp32) added in fp64 in ascending q (+ logit_bias); top-k in descending logit with ties to the lower expert id
 * (moe.py:66-68); gates = softmax over the selected logits cast to dtype
 * (moe.py:69-70, 86); losses[0] = aux (moe.py:76-84), losses[1] = z
 * (moe.py:61-62).  Writes logits, inds, gates, gate_dense, losses (those
 * given). */
int rwkvmoe_router_topk(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t,
                        void* ws, size_t ws_bytes, void* stream);

/* Dispatch (replaces the mask loop of moe.py:139-145): per-expert histogram
 * of inds, exclusive scan into offsets, stable scatter of assignment ids into
 * perm (expert-major, ascending t*k+slot within an expert) and inv_perm.
 * Requires inds, perm, inv_perm, offsets. */
int rwkvmoe_dispatch(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t,
                     void* ws, size_t ws_bytes, void* stream);

/* Base key projection (model.py:260-262): hidden = relu(xk·W_keyᵀ)² with
 * xk = x + (shift(x) − x)·x_k, shift per sequence (model.py:67-75).
 * Requires x, x_k, w_key, hidden (x_prev with RWKVMOE_HAS_PREV). */
int rwkvmoe_cmix_key(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t,
                     void* ws, size_t ws_bytes, void* stream);

/* Base value projection (model.py:263): base_out = hidden·W_valueᵀ.
 * Requires hidden, w_value, base_out. */
int rwkvmoe_cmix_value(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t,
                       void* ws, size_t ws_bytes, void* stream);

/* Grouped LoRA over routed rows (moe.py:140-142 without the masking), in
 * expert-major row blocks of perm: for perm position j of expert e,
 * adapter_rows[a] = (x[a/k]·A_e)·B_e with a = perm[j] (the assignment
 * t*k+slot: rows in the order of inds and gates).  Requires x, lora_A,
 * lora_B, perm, offsets, adapter_rows. */
int rwkvmoe_lora_grouped(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t,
                         void* ws, size_t ws_bytes, void* stream);

/* Combine (moe.py:138, 144-147): out[t] = base_out[t] + Σ_e w_e[t]·a_e[t]
 * with experts taken in ascending id, (+ residual); a_e[t] is
 * adapter_rows[t*k+slot] for e = inds[t,slot].  Requires base_out,
 * adapter_rows, inds, gates, out (inv_perm is not read). */
int rwkvmoe_combine(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t,
                    void* ws, size_t ws_bytes, void* stream);

/* ---- full-expert layer ----------------------------------------------------- */

/* Bytes of scratch `ws` that rwkvmoe_experts_forward needs for `desc`
 * (lora_rank and mode are ignored).  Host-only. */
int rwkvmoe_experts_workspace_bytes(const rwkvmoe_desc* desc, size_t* bytes);

/* (out, aux_loss, z_loss) = MoE_CMix(x) — moe.py:170-242: E full ChannelMix
 * experts, top-k routed.  The tensors take the full-expert shapes:
 * x_k (E,C) (reference (E,1,1,C)), w_key (E,F,C) expert_key, w_value (E,C,F)
 * expert_val; lora_A / lora_B are not read.  Only routed rows are computed
 * (the reference evaluates every expert on every token and masks); experts
 * are added in ascending id as moe.py:231-232 does.  Requires x, x_k,
 * w_key, w_value, w_gate, out, losses; optional outputs as for the forward
 * (logits, inds, gates, perm, inv_perm, offsets). */
int rwkvmoe_experts_forward(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t,
                            void* ws, size_t ws_bytes, void* stream);

/* Bytes of scratch `ws` that rwkvmoe_experts_backward needs for `desc`
 * (lora_rank and mode are ignored).  Host-only. */
int rwkvmoe_experts_backward_workspace_bytes(const rwkvmoe_desc* desc, size_t* bytes);

/* VJP of (out, aux_loss, z_loss) = MoE_CMix(x) (moe.py:218-234) with respect
 * to x, the carried shift state x_prev (RWKVMOE_HAS_PREV), x_k, expert_key,
 * expert_val and router.gate.weight: the gradients MLX autodiff gives a
 * training step through the full-expert layer (every parameter trainable;
 * the top-k selection and the aux-loss counts are piecewise constant).
 * logits and inds are the ones rwkvmoe_experts_forward wrote for the same x
 * and parameters.  Only routed rows are evaluated.  Sums over tokens take a
 * fixed order: results do not depend on timing.  Requires x, x_k, w_key,
 * w_value, w_gate, logits, inds, d_out (and x_prev with RWKVMOE_HAS_PREV);
 * d_x_prev without RWKVMOE_HAS_PREV is RWKVMOE_ERR_FLAGS.  The fp32 gate of
 * RWKVMOE_GATE_F32 is not supported (RWKVMOE_ERR_DTYPE). */
int rwkvmoe_experts_backward(const rwkvmoe_desc* desc, const rwkvmoe_experts_grads* g,
                             void* ws, size_t ws_bytes, void* stream);

/* ---- backward ------------------------------------------------------------ */

/* Bytes of scratch `ws` that rwkvmoe_backward needs for `desc` (mode and
 * flags other than the dtype and shape are ignored).  Host-only. */
int rwkvmoe_backward_workspace_bytes(const rwkvmoe_desc* desc, size_t* bytes);

/* VJP of (out, aux_loss, z_loss) = LoRAMoE_CMix(x) with respect to x,
 * lora_A, lora_B and router.gate.weight: the gradients MLX autodiff gives
 * the reference's training step (finetune_moe.py:215-232 over
 * moe.py:129-147).  The base output is under stop_gradient (moe.py:131) and
 * contributes nothing; the top-k selection and the aux-loss counts are
 * piecewise constant (moe.py:66-68, 80-83).  logits and inds are the ones
 * the forward wrote for the same x and parameters (logit_bias, if any, is
 * inside the logits).  Requires x, w_gate, lora_A, lora_B, logits, inds,
 * d_out. */
int rwkvmoe_backward(const rwkvmoe_desc* desc, const rwkvmoe_grads* g,
                     void* ws, size_t ws_bytes, void* stream);

/* Gradient of the orthogonality loss (moe.py:149-163), which the reference's
 * Block adds to the training loss on every forward (model.py:323):
 * d_lora_A = d_ortho · 2 Σ_{j≠i} A_j (A_jᵀ A_i) for each expert i (written,
 * not accumulated).  Requires lora_A, d_lora_A; workspace as
 * rwkvmoe_backward_workspace_bytes. */
int rwkvmoe_ortho_backward(const rwkvmoe_desc* desc, const rwkvmoe_grads* g,
                           void* ws, size_t ws_bytes, void* stream);

/* Orthogonality loss (moe.py:149-163): ortho_loss[0] = Σ_{i<j} ||A_iᵀA_j||_F²
 * in fp32.  Requires lora_A, ortho_loss. */
int rwkvmoe_ortho_loss(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t,
                       void* ws, size_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RWKVMOE_H */
