// C ABI of librwkvmoe: argument validation, workspace layout and the launch
// sequence of the LoRA-MoE ChannelMix forward (rwkv_mlx/moe.py:129-147).
// Every argument error is detected here, on the host, before any HIP call.
#include <algorithm>
#include <stdint.h>
#include <string.h>

#include "../../include/rwkvmoe.h"
#include "internal.h"

namespace rwkvmoe {

Probe*& probe_slot() {
  static thread_local Probe* p = nullptr;
  return p;
}

hipError_t mark(hipError_t launched, const char* name, hipStream_t s) {
  Probe* p = probe_slot();
  if (launched != hipSuccess || !p) return launched;
  if (p->pairs) {  // the launches recorded their own events: name them
    for (int i = p->named; i < p->n && i < p->cap; ++i) p->names[i] = name;
    p->named = p->n;
    return hipSuccess;
  }
  hipError_t e = hipSuccess;
  if (p->n < p->cap) {
    p->names[p->n] = name;
    e = hipEventRecord(p->ev[p->n + 1], s);
  }
  p->n++;
  return e;
}

}  // namespace rwkvmoe

using namespace rwkvmoe;

namespace {

constexpr int kMaxE = 64, kMaxK = 8, kMaxR = 32;

size_t elem_size(int dtype) { return dtype == RWKVMOE_F32 ? 4 : 2; }

struct Dims {
  int B, T, N, C, F, E, k, r, kx, dtype, mode, flags;
  size_t s;
  // mixed dtypes (16-bit layers only): W_gate fp32; lora_A / lora_B fp32,
  // which makes the delta, out and the adapter rows fp32 (sa, so: their
  // element sizes)
  bool gate32, ad32;
  // fp32 adapters beside a bf16 base: the delta runs as fp32 adapter rows
  // (SPARSE, the grouped LoRA in fp32 on fp32 copies of x; no 16-bit pair
  // form holds fp32's 24 bits with bf16's 8-bit significand)
  bool a32rows;
  size_t sa, so;
  bool ln;  // RWKVMOE_LN_IN: the layer reads LN(x)
  // the forward's algorithm: the SPARSE one (dispatch, grouped LoRA,
  // combine) when asked for, or for fp32 adapters whose fused form does not
  // apply (the router cannot fuse the adapter product, or the value product
  // would split K)
  bool sparse;
  // SPARSE through the router's unscaled adapter product u and the value
  // product's rank slices (launch_cmix_value_sparse) applies to the shape:
  // the workspace holds u.  The forward takes it (no dispatch, grouped LoRA
  // or adapter rows) unless the caller asks for the adapter rows or for the
  // grouped products on the vector ALUs (RWKVMOE_LORA_VALU)
  bool sfuse;
  // FUSED with at most 64 tokens (decode steps): two launches, the decode
  // front (router + key and adapter tiles) and the decode value product
  bool dec;
  int rtt;  // tokens per router workgroup
};

int check_desc(const rwkvmoe_desc* d, Dims* o, bool backward = false) {
  if (!d) return RWKVMOE_ERR_NULL_DESC;
  if (d->dtype < RWKVMOE_F32 || d->dtype > RWKVMOE_BF16) return RWKVMOE_ERR_DTYPE;
  if (d->mode != RWKVMOE_MODE_FUSED && d->mode != RWKVMOE_MODE_SPARSE) return RWKVMOE_ERR_MODE;
  if (d->flags & ~(RWKVMOE_HAS_PREV | RWKVMOE_HAS_BIAS | RWKVMOE_ADD_RESIDUAL | RWKVMOE_GATE_F32 |
                   RWKVMOE_ADAPTERS_F32 | RWKVMOE_GATES_F16 | RWKVMOE_LORA_VALU | RWKVMOE_LN_IN))
    return RWKVMOE_ERR_FLAGS;
  // ln2 in front of the layer: forward passes only (the VJPs take LN(x))
  if ((d->flags & RWKVMOE_LN_IN) && backward) return RWKVMOE_ERR_FLAGS;
  if ((d->flags & RWKVMOE_LORA_VALU) && (d->flags & RWKVMOE_ADAPTERS_F32)) return RWKVMOE_ERR_FLAGS;
  // fp16 gates in an fp32 backward: the fine-tune layer's VJP only
  if ((d->flags & RWKVMOE_GATES_F16) && (!backward || d->dtype != RWKVMOE_F32)) return RWKVMOE_ERR_FLAGS;
  if (d->batch < 1 || d->seq_len < 1) return RWKVMOE_ERR_SHAPE;
  if (d->d_model < 64 || d->d_model > 8192 || d->d_model % 64) return RWKVMOE_ERR_SHAPE;
  if (d->d_ffn < 64 || d->d_ffn > 65536 || d->d_ffn % 64) return RWKVMOE_ERR_SHAPE;
  if (d->n_experts < 1 || d->n_experts > kMaxE) return RWKVMOE_ERR_SHAPE;
  if (d->lora_rank < 1 || d->lora_rank > kMaxR) return RWKVMOE_ERR_SHAPE;
  if (d->top_k < 1 || d->top_k > kMaxK || d->top_k > d->n_experts) return RWKVMOE_ERR_TOPK;
  const long long N = (long long)d->batch * d->seq_len;
  // every index product the kernels form must stay below 2^31
  const long long wide = d->d_ffn > d->d_model * d->top_k ? d->d_ffn : (long long)d->d_model * d->top_k;
  if (N * wide >= (1ll << 31) || N * 64 >= (1ll << 31)) return RWKVMOE_ERR_SHAPE;
  o->B = d->batch; o->T = d->seq_len; o->N = (int)N;
  o->C = d->d_model; o->F = d->d_ffn; o->E = d->n_experts; o->k = d->top_k; o->r = d->lora_rank;
  o->kx = lora_kx(o->E, o->r);
  o->dtype = d->dtype; o->mode = d->mode; o->flags = d->flags;
  o->s = elem_size(d->dtype);
  o->gate32 = d->dtype != RWKVMOE_F32 && (d->flags & RWKVMOE_GATE_F32);
  o->ad32 = d->dtype != RWKVMOE_F32 && (d->flags & RWKVMOE_ADAPTERS_F32);
  o->a32rows = o->ad32 && d->dtype == RWKVMOE_BF16;
  o->sa = o->ad32 ? 4 : o->s;
  o->ln = (d->flags & RWKVMOE_LN_IN) != 0;
  o->so = o->sa;
  o->sparse = d->mode == RWKVMOE_MODE_SPARSE || o->a32rows ||
              (o->ad32 && !(router_fuses_adapters(o->N, o->C, o->E, o->r, o->dtype) &&
                            value_plan_mixed_ok(o->N, o->C, o->F + 3 * o->kx)));
  o->dec = !o->sparse && !o->ad32 && decode_front_ok(o->N, o->C, o->F, o->E, o->dtype, o->gate32);
  o->sfuse = o->sparse && d->mode == RWKVMOE_MODE_SPARSE && !o->ad32 &&
             router_fuses_adapters(o->N, o->C, o->E, o->r, o->dtype) &&
             value_sparse_fusable(o->dtype, o->N, o->C, o->F, o->E, o->r, o->k, o->kx);
  o->rtt = router_tile_tokens(o->N, o->C, o->E, o->dtype);
  if (router_smem_bytes(o->dtype, o->N, o->C, o->E, o->gate32, o->ln) > 163840) return RWKVMOE_ERR_SHAPE;  // one router workgroup's LDS
  return RWKVMOE_OK;
}

// Workspace layout; each region 256-byte aligned.
struct Layout {
  size_t part_f64, part_cnt, loss_claim, inds, gates, gdense, xk, hidden, at, bt, u, dcounts, perm, inv, offsets, base, ag,
      ortho, splitk, dh, du, dg, xn, x32;
  size_t total;
};

Layout layout(const Dims& d) {
  Layout L;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += (bytes + 255) / 256 * 256;
    return at;
  };
  const int nbr = (d.N + d.rtt - 1) / d.rtt;
  const size_t nk = (size_t)d.N * d.k;
  L.part_f64 = take((size_t)nbr * (d.E + 1) * sizeof(double));
  L.part_cnt = take((size_t)nbr * d.E * sizeof(int));
  L.loss_claim = take(2 * sizeof(int));  // the loss claim and the dispatch ticket
  L.inds = take(nk * sizeof(int));
  L.gates = take(nk * d.s);
  L.gdense = take((size_t)d.N * d.E * d.s);
  L.xk = take((size_t)d.N * d.C * d.s);
  L.hidden = take((size_t)d.N * d.F * d.s);
  // fp32 adapters: A_all as fp16 pairs (2·kx rows), B_all as [hi | lo' | hi]
  // (3·kx columns), U as [U_hi | 2^-11·U_hi | U_lo] (3·kx columns)
  const size_t pa = d.ad32 ? 2 : 1, pb = d.ad32 ? 3 : 1;
  L.at = take(pa * d.kx * d.C * d.s);
  L.bt = take(pb * d.C * d.kx * d.s);
  L.u = take(!d.sparse || d.sfuse ? pb * d.N * d.kx * d.s : 0);
  L.dcounts = take((size_t)dispatch_blocks((int)nk) * d.E * sizeof(int));
  L.perm = take(nk * sizeof(int));
  L.inv = take(nk * sizeof(int));
  L.offsets = take((d.E + 1) * sizeof(int));
  const bool sp = d.sparse;
  L.base = take(sp ? (size_t)d.N * d.C * d.s : 0);
  L.ag = take(sp ? nk * d.C * d.so : 0);
  L.ortho = take((size_t)(d.E * (d.E - 1) / 2 + 1) * sizeof(float));
  // split-K partials of the key product (with or without adapter columns)
  // and of the value product (K = F, or F + Kx in FUSED mode); one region
  // serves both, as they run one after the other
  const bool fused = !d.sparse;
  size_t sk = gemm_partial_bytes(d.dtype, d.N, d.F, d.F, d.C, false);
  if (fused && !router_fuses_adapters(d.N, d.C, d.E, d.r, d.dtype))
    sk = std::max(sk, gemm_partial_bytes(d.dtype, d.N, d.F + d.kx, d.F, d.C, true));
  sk = std::max(sk, gemm_partial_bytes(d.dtype, d.N, d.C, d.C, d.F + (fused ? d.kx : 0), false));
  sk = std::max(sk, gemm_partial_bytes(d.dtype, d.N, d.C, d.C, d.F, false));
  L.splitk = take(sk);
  // decode: h and u in fragment order, 16·ceil(N/16) rows
  const size_t rows16 = (size_t)(d.N + 15) / 16 * 16;
  L.dh = take(d.dec ? rows16 * d.F * d.s : 0);
  L.du = take(d.dec ? rows16 * d.kx * d.s : 0);
  L.dg = take(d.dec ? rows16 * d.kx * d.s : 0);
  L.xn = take(d.ln ? (size_t)d.N * d.C * d.s : 0);  // LN(x) when the caller gives no x_ln
  L.x32 = take(d.a32rows ? (size_t)d.N * d.C * sizeof(float) : 0);  // fp32 copy of the rows (a32rows)
  L.total = off;
  return L;
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

int check_ws(const Dims& d, void* ws, size_t ws_bytes, Layout* L) {
  *L = layout(d);
  if (!ws || ws_bytes < L->total || !aligned(ws, 256)) return RWKVMOE_ERR_WORKSPACE;
  return RWKVMOE_OK;
}

// Pointer checks: 16-byte alignment for tensors read or written with
// 16-byte vector accesses, element alignment for the rest.
int need(const void* p) { return p ? RWKVMOE_OK : RWKVMOE_ERR_NULL_PTR; }
int vec_ok(const void* p) { return (!p || aligned(p, 16)) ? RWKVMOE_OK : RWKVMOE_ERR_ALIGN; }
int elem_ok(const void* p, size_t a) { return (!p || aligned(p, a)) ? RWKVMOE_OK : RWKVMOE_ERR_ALIGN; }

#define TRY(expr)                       \
  do {                                  \
    const int _st = (expr);             \
    if (_st != RWKVMOE_OK) return _st;  \
  } while (0)

#define HIPTRY(expr)                          \
  do {                                        \
    const hipError_t _e = (expr);             \
    if (_e != hipSuccess) return (int)_e;     \
  } while (0)

int check_common_ptrs(const Dims& d, const rwkvmoe_tensors* t) {
  TRY(vec_ok(t->x)); TRY(vec_ok(t->x_prev)); TRY(vec_ok(t->x_k)); TRY(vec_ok(t->w_key)); TRY(vec_ok(t->w_value));
  TRY(vec_ok(t->w_gate)); TRY(elem_ok(t->lora_A, d.sa)); TRY(elem_ok(t->lora_B, d.sa)); TRY(elem_ok(t->logit_bias, 4));
  TRY(vec_ok(t->residual)); TRY(vec_ok(t->out)); TRY(elem_ok(t->losses, 4)); TRY(elem_ok(t->logits, 4));
  TRY(elem_ok(t->inds, 4)); TRY(elem_ok(t->gates, d.s)); TRY(elem_ok(t->gate_dense, d.s));
  TRY(elem_ok(t->perm, 4)); TRY(elem_ok(t->inv_perm, 4)); TRY(elem_ok(t->offsets, 4)); TRY(vec_ok(t->prepared));
  TRY(vec_ok(t->prepared_base));
  TRY(vec_ok(t->hidden)); TRY(vec_ok(t->base_out)); TRY(vec_ok(t->adapter_rows)); TRY(elem_ok(t->ortho_loss, 4));
  TRY(vec_ok(t->ln_weight)); TRY(vec_ok(t->ln_bias)); TRY(vec_ok(t->x_ln));
  return RWKVMOE_OK;
}

// A flag that an entry point acts on needs its tensor.
int check_flag_tensors(const Dims& d, const rwkvmoe_tensors* t, bool prev, bool bias, bool resid) {
  if (prev && (d.flags & RWKVMOE_HAS_PREV) && !t->x_prev) return RWKVMOE_ERR_FLAGS;
  if (bias && (d.flags & RWKVMOE_HAS_BIAS) && !t->logit_bias) return RWKVMOE_ERR_FLAGS;
  if (resid && (d.flags & RWKVMOE_ADD_RESIDUAL) && !t->residual) return RWKVMOE_ERR_FLAGS;
  if (d.ln && (!t->ln_weight || !t->ln_bias)) return RWKVMOE_ERR_FLAGS;
  return RWKVMOE_OK;
}

template <typename P>
P* pick(P* given, void* ws, size_t off) {
  return given ? given : (P*)((char*)ws + off);
}

// Layouts in a prepared-adapter buffer: A_all in fragment order (16-bit
// layers), A_all row-major, B_all; each as launch_lora_prep writes it.
struct PrepLayout {
  size_t frag, row, b, total;
};

// Layout of a prepared-base buffer (rwkvmoe_prepare_base): W_key (F x C) and
// W_value (C x F) in fragment order, for the decode launches.
struct BaseLayout {
  size_t wk, wv, total;
};

BaseLayout base_layout(const Dims& d) {
  BaseLayout B;
  const size_t one = ((size_t)d.F * d.C * d.s + 255) / 256 * 256;
  B.wk = 0;
  B.wv = one;
  B.total = 2 * one;
  return B;
}

PrepLayout prep_layout(const Dims& d) {
  PrepLayout P;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += (bytes + 255) / 256 * 256;
    return at;
  };
  const size_t pa = d.ad32 ? 2 : 1, pb = d.ad32 ? 3 : 1;
  P.frag = take(d.dtype != RWKVMOE_F32 ? pa * d.kx * d.C * d.s : 0);
  P.row = take(pa * d.kx * d.C * d.s);
  P.b = take(pb * d.C * d.kx * d.s);
  P.total = off;
  return P;
}

struct Ctx {
  Dims d;
  Layout L;
  PrepLayout P;
  const rwkvmoe_tensors* t;
  void* ws;
  hipStream_t s;
  const void* xprev() const { return (d.flags & RWKVMOE_HAS_PREV) ? t->x_prev : nullptr; }
  const float* bias() const { return (d.flags & RWKVMOE_HAS_BIAS) ? t->logit_bias : nullptr; }
  const void* resid() const { return (d.flags & RWKVMOE_ADD_RESIDUAL) ? t->residual : nullptr; }
  // the rows the layer reads: x, or LN(x) (written first by the forward)
  const void* xin() const { return d.ln ? pick(t->x_ln, ws, L.xn) : t->x; }
  int* inds() const { return pick(t->inds, ws, L.inds); }
  void* gates() const { return pick(t->gates, ws, L.gates); }
  void* hidden() const { return pick(t->hidden, ws, L.hidden); }
  int* perm() const { return pick(t->perm, ws, L.perm); }
  int* inv() const { return pick(t->inv_perm, ws, L.inv); }
  int* offsets() const { return pick(t->offsets, ws, L.offsets); }
  void* base() const { return pick(t->base_out, ws, L.base); }
  void* ag() const { return pick(t->adapter_rows, ws, L.ag); }
  void* gdense() const { return pick(t->gate_dense, ws, L.gdense); }
  void* xk() const { return (char*)ws + L.xk; }
  // adapter operands: from the caller's prepared buffer (rwkvmoe_prepare_adapters)
  // or from the workspace, where this call's prep launch writes the layout it
  // needs (fragment order for the router's adapter product, else row-major)
  const void* at_frag() const { return t->prepared ? (const char*)t->prepared + P.frag : (const char*)ws + L.at; }
  const void* at_row() const { return t->prepared ? (const char*)t->prepared + P.row : (const char*)ws + L.at; }
  const void* bt() const { return t->prepared ? (const char*)t->prepared + P.b : (const char*)ws + L.bt; }
  void* u() const { return (char*)ws + L.u; }
  float* part() const { return (float*)((char*)ws + L.splitk); }
};

// `ln_ok`: the entry point takes RWKVMOE_LN_IN (the forwards).
int setup(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t, void* ws, size_t ws_bytes, void* stream, Ctx* c,
          bool ln_ok = false) {
  TRY(check_desc(desc, &c->d));
  if (c->d.ln && !ln_ok) return RWKVMOE_ERR_FLAGS;
  if (!t) return RWKVMOE_ERR_NULL_DESC;
  if (t->struct_size != sizeof(rwkvmoe_tensors)) return RWKVMOE_ERR_VERSION;
  TRY(check_common_ptrs(c->d, t));
  TRY(check_ws(c->d, ws, ws_bytes, &c->L));
  c->P = prep_layout(c->d);
  c->t = t;
  c->ws = ws;
  c->s = (hipStream_t)stream;
  return RWKVMOE_OK;
}

// The reduction of the router's loss partials into c.t->losses.
LossJob loss_job(const Ctx& c) {
  const Dims& d = c.d;
  const int tt = d.rtt;
  LossJob j;
  j.part = (const double*)((char*)c.ws + c.L.part_f64);
  j.cnt = (const int*)((char*)c.ws + c.L.part_cnt);
  j.nb = (d.N + tt - 1) / tt;
  j.N = d.N;
  j.E = d.E;
  j.k = d.k;
  j.losses = c.t->losses;
  j.claim = (int*)((char*)c.ws + c.L.loss_claim);
  return j;
}

// Router; with `with_xk` the same pass writes the token-shift mix xk, with
// `with_u` also the gate-masked adapter down-projection U (needs A_all).
// `finalize`: reduce the losses with a launch of their own (otherwise the
// caller hands loss_job() to the key GEMM).  With ln2 (RWKVMOE_LN_IN) the
// router normalizes its tile itself and writes LN(x) where the caller asked
// for it or a later kernel reads it (`need_xn`).
int run_router(const Ctx& c, bool with_xk, bool with_u, bool finalize, bool need_xn = false, bool u_raw = false) {
  const Dims& d = c.d;
  const LossJob j = loss_job(c);
  const bool ln = d.ln;
  void* xn = ln && (need_xn || c.t->x_ln) ? (void*)c.xin() : nullptr;
  HIPTRY(launch_router(d.dtype, d.gate32, with_u && d.ad32 ? 2 : 1, ln ? c.t->x : c.xin(), c.t->w_gate, c.bias(),
                       c.xprev(), c.t->x_k, with_u ? c.at_frag() : nullptr, d.N, d.T, d.C, d.E, d.k, d.r,
                       c.t->logits, c.inds(), c.gates(), c.gdense(),
                       with_xk ? c.xk() : nullptr, with_u ? c.u() : nullptr, (double*)j.part, (int*)j.cnt, j.claim,
                       d.rtt, c.s, nullptr, ln ? c.t->ln_weight : nullptr, ln ? c.t->ln_bias : nullptr, xn,
                       u_raw));
  if (finalize && c.t->losses) HIPTRY(launch_router_finalize(j, c.s));
  return RWKVMOE_OK;
}

// `routed`: the ids were written by run_router in this call, whose
// per-workgroup expert counts then serve as the dispatch histograms.
int run_dispatch(const Ctx& c, bool routed) {
  const Dims& d = c.d;
  const int* rcnt = routed ? (const int*)((char*)c.ws + c.L.part_cnt) : nullptr;
  HIPTRY(launch_dispatch(c.inds(), d.N * d.k, d.E, (int*)((char*)c.ws + c.L.dcounts), c.perm(), c.inv(), c.offsets(),
                         c.s, rcnt, d.rtt, d.k));
  return RWKVMOE_OK;
}

// A_all and B_all; `frag`: A_all in fragment order (read only by the router's
// adapter product then)
int run_prep(const Ctx& c, bool frag = false) {
  if (c.t->prepared) return RWKVMOE_OK;  // the caller's prepared layouts
  const Dims& d = c.d;
  // (a32rows: A_all and B_all in fp32, the operands of the fp32 grouped LoRA)
  HIPTRY(launch_lora_prep(d.a32rows ? RWKVMOE_F32 : d.dtype, c.t->lora_A, c.t->lora_B, d.E, d.C, d.r, d.kx,
                          (char*)c.ws + c.L.at, (char*)c.ws + c.L.bt, c.s, frag && !d.a32rows,
                          d.ad32 && !d.a32rows));
  return RWKVMOE_OK;
}

// The grouped LoRA's adapter rows (assignment order) for rows x; a32rows: in
// fp32, on an fp32 copy of x (exact) in the workspace
int run_lora(const Ctx& c, const void* x, const int* perm, const int* offsets, void* ag) {
  const Dims& d = c.d;
  if (d.a32rows) {
    float* x32 = (float*)((char*)c.ws + c.L.x32);
    HIPTRY(launch_widen(d.dtype, x, x32, (size_t)d.N * d.C, c.s));
    HIPTRY(launch_lora_grouped(RWKVMOE_F32, x32, c.at_row(), c.bt(), perm, offsets, d.N, d.C, d.E, d.k, d.r, d.kx, ag,
                               c.s));
    return RWKVMOE_OK;
  }
  HIPTRY(launch_lora_grouped(d.dtype, x, c.at_row(), c.bt(), perm, offsets, d.N, d.C, d.E, d.k, d.r, d.kx, ag, c.s,
                             d.ad32, (d.flags & RWKVMOE_LORA_VALU) != 0));
  return RWKVMOE_OK;
}

// Key projection; `mixed`: xk already in the workspace (written by the router
// pass).  `adapters`: also U = gate ⊙ (x · A_allᵀ) for the FUSED value GEMM.
// `losses`: also the router's loss reduction (see run_router).
int run_key(const Ctx& c, bool mixed, bool adapters, bool losses, const DispatchJob* disp = nullptr) {
  const Dims& d = c.d;
  if (!mixed) HIPTRY(launch_shift_mix(d.dtype, c.xin(), c.xprev(), c.t->x_k, c.xk(), d.N, d.T, d.C, c.s));
  const LossJob j = loss_job(c);
  HIPTRY(launch_cmix_key(d.dtype, c.xk(), c.t->w_key, c.hidden(), d.N, d.C, d.F, c.xin(), c.at_row(), c.gdense(), d.E,
                         d.r, d.kx, adapters ? c.u() : nullptr, losses && j.losses ? &j : nullptr, c.part(), c.s,
                         disp));
  return RWKVMOE_OK;
}

int run_ortho(const Ctx& c) {
  const Dims& d = c.d;
  // in lora_A's dtype (moe.py:149-163 on the stored A)
  HIPTRY(launch_ortho(d.ad32 ? RWKVMOE_F32 : d.dtype, c.t->lora_A, d.E, d.C, d.r, (float*)((char*)c.ws + c.L.ortho),
                      c.t->ortho_loss, c.s));
  return RWKVMOE_OK;
}

// `check_only`: every argument check of the forward (the workspace aside),
// then return without a HIP call.
int forward_impl(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t, void* ws, size_t ws_bytes, void* stream,
                 bool decode, bool check_only = false) {
  Ctx c;
  if (check_only) {
    ws = (void*)(uintptr_t)256;  // stands in for a workspace of any size; never dereferenced
    ws_bytes = SIZE_MAX;
  }
  TRY(setup(desc, t, ws, ws_bytes, stream, &c, true));
  const Dims& d = c.d;
  if (decode && (d.T != 1 || !(d.flags & RWKVMOE_HAS_PREV))) return RWKVMOE_ERR_MODE;
  TRY(need(t->x)); TRY(need(t->x_k)); TRY(need(t->w_key)); TRY(need(t->w_value)); TRY(need(t->w_gate));
  TRY(need(t->lora_A)); TRY(need(t->lora_B)); TRY(need(t->out)); TRY(need(t->losses));
  TRY(check_flag_tensors(d, t, true, true, true));
  if (check_only) return RWKVMOE_OK;

  if (Probe* p = probe_slot(); p && !p->pairs) HIPTRY(hipEventRecord(p->ev[0], c.s));
  if (d.dec && !t->hidden) {  // (h as an output is row-major: the many-token kernels write it)
    // (the decode front cannot normalize: its key tiles read x beside the
    // router; LN(x) is written first)
    if (d.ln)
      HIPTRY(launch_layer_norm(d.dtype, t->x, t->ln_weight, t->ln_bias, (void*)c.xin(), d.N, d.C, c.s));
    // decode: the router with the key and adapter tiles in one launch, the
    // value product (gates applied to the adapter columns) and the loss
    // reduction in the other
    TRY(run_prep(c, true));
    const LossJob j = loss_job(c);
    const BaseLayout B = base_layout(d);
    const char* pb = (const char*)t->prepared_base;
    void* dh = (char*)c.ws + c.L.dh;
    void* du = (char*)c.ws + c.L.du;
    void* dg = (char*)c.ws + c.L.dg;
    DecodeFront fr{pb ? pb + B.wk : t->w_key, pb != nullptr, dh, d.F, c.at_frag(), du, d.kx, dg};
    HIPTRY(launch_router(d.dtype, d.gate32, 1, c.xin(), t->w_gate, c.bias(), c.xprev(), t->x_k, nullptr, d.N, d.T,
                         d.C, d.E, d.k, d.r, t->logits, c.inds(), c.gates(), c.gdense(), nullptr, nullptr, (double*)j.part,
                         (int*)j.cnt, j.claim, d.rtt, c.s, &fr));
    HIPTRY(launch_decode_value(d.dtype, dh, pb ? pb + B.wv : t->w_value, pb != nullptr, du, dg, c.bt(), c.resid(),
                               t->out, d.N, d.C, d.F, d.kx, j.losses ? &j : nullptr, c.s));
    if (t->perm || t->inv_perm || t->offsets) TRY(run_dispatch(c, true));
    if (t->ortho_loss) TRY(run_ortho(c));
    return RWKVMOE_OK;
  }
  const bool fused = !d.sparse;
  // SPARSE on chip (d.sfuse), unless the caller asks for the adapter rows or
  // for the grouped products on the vector ALUs
  const bool sfuse = d.sfuse && !t->adapter_rows && !(d.flags & RWKVMOE_LORA_VALU);
  // (fp32 adapters run fused only with the router's adapter product: d.sparse)
  const bool u_in_router = (fused && router_fuses_adapters(d.N, d.C, d.E, d.r, d.dtype)) || sfuse;
  TRY(run_prep(c, u_in_router));
  // LN(x) is read after the router by the key GEMM's adapter columns and the
  // grouped LoRA
  TRY(run_router(c, true, u_in_router, false, !u_in_router, sfuse));
  if (fused) {
    TRY(run_key(c, true, !u_in_router, true));
    HIPTRY(launch_cmix_value(d.dtype, c.hidden(), t->w_value, d.F, c.u(), c.bt(), d.kx, c.resid(), t->out, d.N, d.C,
                             c.part(), c.s, d.ad32));
    if (t->perm || t->inv_perm || t->offsets) TRY(run_dispatch(c, true));
  } else if (sfuse) {
    // u = round(x·A_all) from the router; the value product's rank slices
    // turn it into the combined adapter delta on chip
    TRY(run_key(c, true, false, true));
    HIPTRY(launch_cmix_value_sparse(d.dtype, c.hidden(), t->w_value, d.F, c.u(), c.bt(), d.kx, c.inds(), c.gates(),
                                    d.E, d.r, c.resid(), t->out, d.N, d.C, d.k, c.s));
    if (t->perm || t->inv_perm || t->offsets) TRY(run_dispatch(c, true));
  } else {
    // the dispatch scatter runs inside the key GEMM's launch where the
    // router's per-workgroup counts serve as its histograms (the key product
    // does not read it, the grouped LoRA after it does); else on its own
    const LossJob lj = loss_job(c);
    DispatchJob job;
    const bool in_key = dispatch_job_plan(c.inds(), d.N * d.k, d.E, c.perm(), c.inv(), c.offsets(),
                                          (const int*)((char*)c.ws + c.L.part_cnt), d.rtt, d.k, lj.claim + 1, &job);
    if (!in_key) TRY(run_dispatch(c, true));
    TRY(run_key(c, true, false, true, in_key ? &job : nullptr));
    TRY(run_lora(c, c.xin(), c.perm(), c.offsets(), c.ag()));
    if (!d.ad32 && value_combine_fusable(d.dtype, d.N, d.C, d.F, d.k)) {
      // the combine in the value product's epilogue: the base stays on chip
      HIPTRY(launch_cmix_value_combine(d.dtype, c.hidden(), t->w_value, d.F, c.ag(), c.inds(), c.gates(), c.resid(),
                                       t->out, d.N, d.C, d.k, c.s));
    } else {
      HIPTRY(launch_cmix_value(d.dtype, c.hidden(), t->w_value, d.F, nullptr, nullptr, 0, nullptr, c.base(), d.N,
                               d.C, c.part(), c.s));
      HIPTRY(launch_combine(d.dtype, c.base(), c.ag(), c.inds(), c.gates(), nullptr, c.resid(), t->out, d.N, d.C,
                            d.k, c.s, d.ad32));  // (the rows in assignment order)
    }
  }
  if (t->ortho_loss) TRY(run_ortho(c));
  return RWKVMOE_OK;
}

// ---- backward -----------------------------------------------------------------
// Workspace of rwkvmoe_backward; np / ep: tokens / experts padded to 128 (the
// K lengths of the token-contracted products and of dx's router segment).
struct BwdLayout {
  size_t at, a_t, b_rows, wgt, xt, dot, S, G, cnt, dsd, dl, rT, sgdT, o, gram, splitk, splitk_b, total;
  // per-expert products (16-bit layers): SGd row-major, per-token expert
  // masks, fp32 range partials of dA, dB and dW_gate
  size_t sgd, emask, pa, pb, pw;
  bool fx;  // the fused routing kernel computes S and G
  bool px;  // per-expert token contractions (else the dense products)
  BwdExpertPlan xp;
  int np, ep;
};

int round_up(int v, int m) { return (v + m - 1) / m * m; }

BwdLayout bwd_layout(const Dims& d) {
  BwdLayout L;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += (bytes + 255) / 256 * 256;
    return at;
  };
  L.np = round_up(d.N, 128);
  L.ep = round_up(d.E, 128);
  const size_t s = d.s, np = L.np, ep = L.ep, kx = d.kx, C = d.C, N = d.N;
  L.fx = bwd_route_fuses(d.dtype, d.kx, d.C);
  L.px = d.dtype != 0;
  const size_t sg = L.fx ? 0 : 1;     // S and G in memory
  const size_t dense = L.px ? 0 : 1;  // the dense token-contracted products
  const size_t px = L.px ? 1 : 0;
  L.at = take(kx * C * s);
  L.a_t = take(C * kx * s);
  L.b_rows = take(kx * C * s);
  L.wgt = take(C * ep * s);
  L.xt = take(dense * C * np * s);
  L.dot = take(dense * C * np * s);
  L.S = take(sg * N * kx * s);
  L.G = take(sg * N * kx * s);
  L.cnt = take(64 * sizeof(int));
  L.dsd = take(N * kx * s);
  L.dl = take(N * ep * s);
  L.rT = take(dense * (kx + ep) * np * s);
  L.sgdT = take(dense * kx * np * s);
  L.o = take(C * (kx + ep) * s);
  L.xp = bwd_expert_plan(d.N, d.C, d.E, d.k);
  L.sgd = take(px * N * kx * s);
  L.emask = take(px * N * sizeof(unsigned long long));
  L.pa = take(px * (size_t)d.E * L.xp.R * C * d.r * sizeof(float));
  L.pb = take(px * (size_t)d.E * L.xp.R * C * d.r * sizeof(float));
  L.pw = take(px * (size_t)L.xp.RW * d.E * C * sizeof(float));
  L.gram = take(kx * kx * s);
  size_t sk = gemm_nt_partial_bytes(d.dtype, d.N, d.kx, d.C, GEMM_HINT_NO_SPLIT);
  sk = std::max(sk, gemm_nt_partial_bytes(d.dtype, d.C, d.kx + L.ep, L.np));
  sk = std::max(sk, gemm_nt_partial_bytes(d.dtype, d.N, d.C, d.kx + L.ep));
  sk = std::max(sk, gemm_nt_partial_bytes(d.dtype, d.kx, d.kx, d.C));   // ortho: Gram
  sk = std::max(sk, gemm_nt_partial_bytes(d.dtype, d.C, d.kx, d.kx));   // ortho: A_T · Gm
  L.splitk = take(sk);
  // dB's partials live beside O's until bwd_finish reduces both
  L.splitk_b = take(dense * gemm_nt_partial_bytes(d.dtype, d.E * d.r, d.C, L.np, GEMM_HINT_SPLIT64));
  L.total = off;
  return L;
}

int check_bwd_desc(const rwkvmoe_desc* desc, Dims* d) {
  TRY(check_desc(desc, d, true));
  if (d->gate32 || d->ad32) return RWKVMOE_ERR_DTYPE;  // mixed layers: see backward_impl
  const long long np = round_up(d->N, 128);
  const long long w = std::max(std::max(d->kx, d->C), round_up(d->E, 128));
  if (np * w >= (1ll << 31)) return RWKVMOE_ERR_SHAPE;
  return RWKVMOE_OK;
}

int backward_impl(const rwkvmoe_desc* desc, const rwkvmoe_grads* g, void* ws, size_t ws_bytes, void* stream) {
  Dims d;
  TRY(check_bwd_desc(desc, &d));
  if (!g) return RWKVMOE_ERR_NULL_DESC;
  TRY(need(g->x)); TRY(need(g->w_gate)); TRY(need(g->lora_A)); TRY(need(g->lora_B)); TRY(need(g->logits));
  TRY(need(g->inds)); TRY(need(g->d_out));
  TRY(vec_ok(g->x)); TRY(vec_ok(g->w_gate)); TRY(elem_ok(g->lora_A, d.s)); TRY(elem_ok(g->lora_B, d.s));
  TRY(elem_ok(g->logits, 4)); TRY(elem_ok(g->inds, 4)); TRY(vec_ok(g->d_out)); TRY(elem_ok(g->d_losses, 4));
  TRY(vec_ok(g->d_x)); TRY(elem_ok(g->d_lora_A, d.s)); TRY(vec_ok(g->d_lora_B)); TRY(vec_ok(g->d_w_gate));
  const BwdLayout L = bwd_layout(d);
  if (!ws || ws_bytes < L.total || !aligned(ws, 256)) return RWKVMOE_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  char* w = (char*)ws;
  const int dt = d.dtype, N = d.N, C = d.C, E = d.E, kx = d.kx, np = L.np, ep = L.ep;
  float* part = (float*)(w + L.splitk);
  const bool fused = L.fx;
  const bool need_xt = g->d_lora_A || g->d_w_gate, need_dot = g->d_lora_B;
  // A_all (kx, C), A_T (C, kx), B_rows (kx, C), W_gateᵀ (C, ep); A_all and
  // B_rows in fragment order for the fused routing kernel; and the
  // per-expert selection counts
  int* cnt = (int*)(w + L.cnt);
  HIPTRY(launch_bwd_prep(dt, g->lora_A, g->lora_B, g->w_gate, E, C, d.r, kx, ep, fused, w + L.at, w + L.a_t,
                         w + L.b_rows, w + L.wgt, g->inds, N * d.k, cnt, s));
  unsigned long long* emask = L.px ? (unsigned long long*)(w + L.emask) : nullptr;
  void* sgd = L.px ? w + L.sgd : nullptr;
  void* rT = L.px ? nullptr : w + L.rT;
  void* sgdT = L.px ? nullptr : w + L.sgdT;
  if (fused) {
    // S = x · A_allᵀ and G = dO · B_rowsᵀ inside the routing-gradient kernel,
    // which writes DSd, SGd and dℓ row-major and the per-token expert masks
    HIPTRY(launch_bwd_route_fused(dt, g->logits, g->inds, cnt, g->d_losses, N, E, d.k, d.r, kx, ep, np, C, g->x,
                                  g->d_out, w + L.at, w + L.b_rows, w + L.dsd, w + L.dl, rT, sgdT, nullptr, nullptr,
                                  sgd, emask, s));
  } else {
    HIPTRY(launch_gemm_nt(dt, g->x, C, w + L.at, C, C, nullptr, 0, nullptr, 0, 0, N, kx, w + L.S, kx, part, "bwd_s",
                          s, GEMM_HINT_NO_SPLIT));
    HIPTRY(launch_gemm_nt(dt, g->d_out, C, w + L.b_rows, C, C, nullptr, 0, nullptr, 0, 0, N, kx, w + L.G, kx, part,
                          "bwd_g", s, GEMM_HINT_NO_SPLIT));
    HIPTRY(launch_bwd_route(dt, g->logits, g->inds, w + L.S, w + L.G, cnt, g->d_losses, N, E, d.k, d.r, kx, ep, np,
                            w + L.dsd, w + L.dl, rT, sgdT, sgd, emask, s, (d.flags & RWKVMOE_GATES_F16) != 0));
  }
  if (L.px) {
    // dA, dB and dW_gate as per-expert token contractions
    if (need_xt || need_dot) {
      float* pa = (float*)(w + L.pa);
      float* pb = (float*)(w + L.pb);
      float* pw = (float*)(w + L.pw);
      HIPTRY(launch_bwd_expert(dt, g->x, g->d_out, w + L.dsd, sgd, w + L.dl, emask, N, C, E, d.r, kx, ep, L.xp, pa,
                               pb, pw, s));
      HIPTRY(launch_bwd_finish_expert(dt, pa, pb, pw, E, C, d.r, L.xp.R, L.xp.RW, g->d_lora_A, g->d_lora_B,
                                      g->d_w_gate, s));
    }
  } else {
    if (need_xt) HIPTRY(launch_transpose_pad(dt, g->x, N, C, C, w + L.xt, np, s));
    if (need_dot) HIPTRY(launch_transpose_pad(dt, g->d_out, N, C, C, w + L.dot, np, s));
    // dA_all_T and dW_gateᵀ in one product, O = xᵀ · [DSd | dℓ], and dB =
    // SGdᵀ · dO; split products leave their partials to bwd_finish, which
    // reduces both and scatters O into dA and dW_gate in one launch
    int ks_o = 1, ks_b = 1;
    float* part_b = (float*)(w + L.splitk_b);
    if (need_xt)
      HIPTRY(launch_gemm_nt(dt, w + L.xt, np, w + L.rT, np, np, nullptr, 0, nullptr, 0, 0, C, kx + ep, w + L.o,
                            kx + ep, part, "bwd_da_dwg", s, GEMM_HINT_AUTO, &ks_o));
    if (need_dot)
      HIPTRY(launch_gemm_nt(dt, w + L.sgdT, np, w + L.dot, np, np, nullptr, 0, nullptr, 0, 0, E * d.r, C,
                            g->d_lora_B, C, part_b, "bwd_db", s, GEMM_HINT_SPLIT64, &ks_b));
    HIPTRY(launch_bwd_finish(dt, part, ks_o, w + L.o, E, C, d.r, kx, ep, need_xt ? g->d_lora_A : nullptr,
                             need_xt ? g->d_w_gate : nullptr, part_b, ks_b, need_dot ? g->d_lora_B : nullptr, s));
    // (dx's own split partials, if any, reuse O's region after bwd_finish)
  }
  if (g->d_x) {
    HIPTRY(launch_gemm_nt(dt, w + L.dsd, kx, w + L.a_t, kx, kx, w + L.dl, ep, w + L.wgt, ep, ep, N, C, g->d_x, C, part,
                          "bwd_dx", s));
  }
  return RWKVMOE_OK;
}

// ---- the standalone router's VJP (moe.py:35-86) --------------------------------
struct RouterBwdLayout {
  size_t dcounts, perm, inv, offsets, dl, cpart, total;
};

RouterBwdLayout router_bwd_layout(const Dims& d) {
  RouterBwdLayout L;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += (bytes + 255) / 256 * 256;
    return at;
  };
  const size_t nk = (size_t)d.N * d.k;
  L.dcounts = take((size_t)dispatch_blocks((int)nk) * d.E * sizeof(int));
  L.perm = take(nk * sizeof(int));
  L.inv = take(nk * sizeof(int));
  L.offsets = take((d.E + 1) * sizeof(int));
  L.dl = take((size_t)d.N * d.E * sizeof(float));
  L.cpart = take((size_t)d.E * exb_col_chunks(d.N, d.C, d.E) * d.C * sizeof(float));
  L.total = off;
  return L;
}

int check_router_bwd_desc(const rwkvmoe_desc* desc, Dims* d) {
  TRY(check_desc(desc, d, true));
  if (d->flags & ~RWKVMOE_HAS_BIAS) return RWKVMOE_ERR_FLAGS;
  return RWKVMOE_OK;
}

int router_backward_impl(const rwkvmoe_desc* desc, const rwkvmoe_router_grads* g, void* ws, size_t ws_bytes,
                         void* stream) {
  Dims d;
  TRY(check_router_bwd_desc(desc, &d));
  if (!g) return RWKVMOE_ERR_NULL_DESC;
  TRY(need(g->x)); TRY(need(g->w_gate)); TRY(need(g->logits)); TRY(need(g->inds));
  TRY(vec_ok(g->x)); TRY(vec_ok(g->w_gate)); TRY(elem_ok(g->logits, 4)); TRY(elem_ok(g->inds, 4));
  TRY(elem_ok(g->d_gates, d.s)); TRY(elem_ok(g->d_losses, 4)); TRY(vec_ok(g->d_x)); TRY(vec_ok(g->d_w_gate));
  const RouterBwdLayout L = router_bwd_layout(d);
  if (!ws || ws_bytes < L.total || !aligned(ws, 256)) return RWKVMOE_ERR_WORKSPACE;
  if (!g->d_x && !g->d_w_gate) return RWKVMOE_OK;
  hipStream_t s = (hipStream_t)stream;
  char* w = (char*)ws;
  const int nk = d.N * d.k;
  int* inv = (int*)(w + L.inv);
  int* off = (int*)(w + L.offsets);
  float* dl = (float*)(w + L.dl);
  // the selection counts (f_e) and each assignment's validity, from a dispatch of the ids
  HIPTRY(launch_dispatch(g->inds, nk, d.E, (int*)(w + L.dcounts), (int*)(w + L.perm), inv, off, s));
  HIPTRY(launch_router_route(d.dtype, g->logits, g->inds, inv, g->d_gates, off, g->d_losses, d.N, d.E, d.k, dl, s));
  if (g->d_x)
    HIPTRY(launch_exb_dx(d.dtype, nullptr, inv, g->inds, nullptr, dl, g->w_gate, d.N, d.T, d.C, d.E, d.k, g->d_x,
                         nullptr, s));
  if (g->d_w_gate)
    HIPTRY(launch_exb_colsum(d.dtype, 1, nullptr, g->x, nullptr, off, nullptr, dl, d.N, d.T, d.C, d.E, d.k,
                             (float*)(w + L.cpart), g->d_w_gate, s));
  return RWKVMOE_OK;
}

// ---- full-expert layer (MoE_CMix, moe.py:170-242) ------------------------------
struct ExpLayout {
  size_t part_f64, part_cnt, loss_claim, inds, gates, dcounts, perm, inv, offsets, xkg, h, og, xn, total;
};

ExpLayout experts_layout(const Dims& d) {
  ExpLayout L;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += (bytes + 255) / 256 * 256;
    return at;
  };
  const int tt = router_tile_tokens(d.N, d.C, d.E, d.dtype);
  const int nbr = (d.N + tt - 1) / tt;
  const size_t nk = (size_t)d.N * d.k;
  L.part_f64 = take((size_t)nbr * (d.E + 1) * sizeof(double));
  L.part_cnt = take((size_t)nbr * d.E * sizeof(int));
  L.loss_claim = take(2 * sizeof(int));  // the loss claim and the dispatch ticket
  L.inds = take(nk * sizeof(int));
  L.gates = take(nk * d.s);
  L.dcounts = take((size_t)dispatch_blocks((int)nk) * d.E * sizeof(int));
  L.perm = take(nk * sizeof(int));
  L.inv = take(nk * sizeof(int));
  L.offsets = take((d.E + 1) * sizeof(int));
  L.xkg = take(nk * d.C * d.s);
  L.h = take(nk * d.F * d.s);
  L.og = take(nk * d.C * d.s);
  L.xn = take(d.ln ? (size_t)d.N * d.C * d.s : 0);  // LN(x) when the caller gives no x_ln
  L.total = off;
  return L;
}

int check_experts_desc(const rwkvmoe_desc* desc, Dims* d) {
  TRY(check_desc(desc, d));
  if (d->flags & RWKVMOE_ADAPTERS_F32) return RWKVMOE_ERR_FLAGS;  // the full-expert layer has no adapters
  const long long rows = (long long)d->N * d->k;
  if (rows * std::max(d->F, d->C) >= (1ll << 31)) return RWKVMOE_ERR_SHAPE;
  return RWKVMOE_OK;
}

int experts_forward_impl(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t, void* ws, size_t ws_bytes,
                         void* stream) {
  Dims d;
  TRY(check_experts_desc(desc, &d));
  if (!t) return RWKVMOE_ERR_NULL_DESC;
  if (t->struct_size != sizeof(rwkvmoe_tensors)) return RWKVMOE_ERR_VERSION;
  TRY(check_common_ptrs(d, t));
  TRY(need(t->x)); TRY(need(t->x_k)); TRY(need(t->w_key)); TRY(need(t->w_value)); TRY(need(t->w_gate));
  TRY(need(t->out)); TRY(need(t->losses));
  TRY(check_flag_tensors(d, t, true, true, true));
  const ExpLayout L = experts_layout(d);
  if (!ws || ws_bytes < L.total || !aligned(ws, 256)) return RWKVMOE_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  char* w = (char*)ws;
  const int nk = d.N * d.k;
  const void* xprev = (d.flags & RWKVMOE_HAS_PREV) ? t->x_prev : nullptr;
  const float* bias = (d.flags & RWKVMOE_HAS_BIAS) ? t->logit_bias : nullptr;
  const void* resid = (d.flags & RWKVMOE_ADD_RESIDUAL) ? t->residual : nullptr;
  const void* xin = d.ln ? pick(t->x_ln, ws, L.xn) : t->x;
  int* inds = pick(t->inds, ws, L.inds);
  void* gates = pick(t->gates, ws, L.gates);
  int* perm = pick(t->perm, ws, L.perm);
  int* inv = pick(t->inv_perm, ws, L.inv);
  int* offsets = pick(t->offsets, ws, L.offsets);
  LossJob j;
  const int tt = router_tile_tokens(d.N, d.C, d.E, d.dtype);
  j.part = (const double*)(w + L.part_f64);
  j.cnt = (const int*)(w + L.part_cnt);
  j.nb = (d.N + tt - 1) / tt;
  j.N = d.N;
  j.E = d.E;
  j.k = d.k;
  j.losses = t->losses;
  j.claim = (int*)(w + L.loss_claim);
  if (Probe* p = probe_slot(); p && !p->pairs) HIPTRY(hipEventRecord(p->ev[0], s));
  // with ln2 the router normalizes its tile and writes LN(x) for the mix
  HIPTRY(launch_router(d.dtype, d.gate32, 1, t->x, t->w_gate, bias, nullptr, nullptr, nullptr, d.N, d.T, d.C, d.E,
                       d.k, 1, t->logits, inds, gates, nullptr, nullptr, nullptr, (double*)j.part, (int*)j.cnt,
                       j.claim, tt, s, nullptr, d.ln ? t->ln_weight : nullptr, d.ln ? t->ln_bias : nullptr,
                       d.ln ? (void*)xin : nullptr));
  HIPTRY(launch_dispatch(inds, nk, d.E, (int*)(w + L.dcounts), perm, inv, offsets, s, j.cnt, tt, d.k));
  HIPTRY(launch_experts_mix(d.dtype, xin, xprev, t->x_k, perm, inds, d.N, d.T, d.C, d.E, d.k, w + L.xkg, s));
  // the key product's first workgroup to finish reduces the router's losses
  HIPTRY(launch_grouped_gemm(d.dtype, true, w + L.xkg, d.C, t->w_key, d.C, (long long)d.F * d.C, d.C, nk, d.F,
                             offsets, d.E, w + L.h, d.F, "experts_key", s, &j));
  HIPTRY(launch_grouped_gemm(d.dtype, false, w + L.h, d.F, t->w_value, d.F, (long long)d.C * d.F, d.F, nk, d.C,
                             offsets, d.E, w + L.og, d.C, "experts_value", s));
  HIPTRY(launch_combine(d.dtype, nullptr, w + L.og, inds, gates, inv, resid, t->out, d.N, d.C, d.k, s));
  return RWKVMOE_OK;
}

// Workspace of rwkvmoe_experts_backward.  np: tokens padded to 128, the
// length of each expert's segment in the token-major (transposed) operands of
// the weight-gradient products.
struct ExpBwdLayout {
  size_t dcounts, perm, inv, offsets, koff, xkg, P, dog, gr, U, dw, wT, dk, dl, cpart, tA, tB, total;
  int ncol;  // bound on the packed token columns of the transposed operands
};

ExpBwdLayout exp_bwd_layout(const Dims& d) {
  ExpBwdLayout L;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += (bytes + 255) / 256 * 256;
    return at;
  };
  const size_t nk = (size_t)d.N * d.k, s = d.s, C = d.C, F = d.F, E = d.E;
  L.ncol = exb_seg_cols((int)nk, d.E);
  L.dcounts = take((size_t)dispatch_blocks((int)nk) * E * sizeof(int));
  L.perm = take(nk * sizeof(int));
  L.inv = take(nk * sizeof(int));
  L.offsets = take((E + 1) * sizeof(int));
  L.koff = take((E + 1) * sizeof(int));
  L.xkg = take(nk * C * s);
  L.P = take(nk * F * s);
  L.dog = take(nk * C * s);
  L.gr = take(nk * sizeof(float));
  L.U = take(nk * F * s);  // u, then dp in place
  L.dw = take(nk * sizeof(float));
  L.wT = take(E * F * C * s);  // W_val,eᵀ, then W_key,eᵀ
  L.dk = take(nk * C * s);
  L.dl = take((size_t)d.N * E * sizeof(float));
  L.cpart = take(E * (size_t)exb_col_chunks(d.N, d.C, d.E) * C * sizeof(float));
  L.tA = take(std::max(F, C) * (size_t)L.ncol * s);  // dpᵀ, then (g·dO)ᵀ
  L.tB = take(std::max(F, C) * (size_t)L.ncol * s);  // xkᵀ, then hᵀ
  L.total = off;
  return L;
}

int check_exp_bwd_desc(const rwkvmoe_desc* desc, Dims* d) {
  TRY(check_experts_desc(desc, d));
  if (d->ln) return RWKVMOE_ERR_FLAGS;      // the VJP takes LN(x)
  if (d->gate32) return RWKVMOE_ERR_DTYPE;  // as rwkvmoe_backward: one element type
  const long long cols = exb_seg_cols(d->N * d->k, d->E);
  if (cols * std::max(d->F, d->C) >= (1ll << 31)) return RWKVMOE_ERR_SHAPE;
  return RWKVMOE_OK;
}

int experts_backward_impl(const rwkvmoe_desc* desc, const rwkvmoe_experts_grads* g, void* ws, size_t ws_bytes,
                          void* stream) {
  Dims d;
  TRY(check_exp_bwd_desc(desc, &d));
  if (!g) return RWKVMOE_ERR_NULL_DESC;
  const bool has_prev = d.flags & RWKVMOE_HAS_PREV;
  TRY(need(g->x)); TRY(need(g->x_k)); TRY(need(g->w_key)); TRY(need(g->w_value)); TRY(need(g->w_gate));
  TRY(need(g->logits)); TRY(need(g->inds)); TRY(need(g->d_out));
  if (has_prev) TRY(need(g->x_prev));
  if (g->d_x_prev && !has_prev) return RWKVMOE_ERR_FLAGS;
  TRY(vec_ok(g->x)); TRY(vec_ok(g->x_prev)); TRY(vec_ok(g->x_k)); TRY(vec_ok(g->w_key)); TRY(vec_ok(g->w_value));
  TRY(vec_ok(g->w_gate)); TRY(elem_ok(g->logits, 4)); TRY(elem_ok(g->inds, 4)); TRY(vec_ok(g->d_out));
  TRY(elem_ok(g->d_losses, 4)); TRY(vec_ok(g->d_x)); TRY(vec_ok(g->d_x_prev)); TRY(vec_ok(g->d_x_k));
  TRY(vec_ok(g->d_w_key)); TRY(vec_ok(g->d_w_value)); TRY(vec_ok(g->d_w_gate));
  const ExpBwdLayout L = exp_bwd_layout(d);
  if (!ws || ws_bytes < L.total || !aligned(ws, 256)) return RWKVMOE_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  char* w = (char*)ws;
  const int dt = d.dtype, N = d.N, C = d.C, F = d.F, E = d.E, k = d.k, nk = N * k;
  const void* xprev = has_prev ? g->x_prev : nullptr;
  int* perm = (int*)(w + L.perm);
  int* inv = (int*)(w + L.inv);
  int* off = (int*)(w + L.offsets);
  float* gr = (float*)(w + L.gr);
  float* dw = (float*)(w + L.dw);
  float* dl = (float*)(w + L.dl);
  // the forward's expert-major rows: xk_j and p_j = xk_j · W_key,eᵀ (before relu²)
  HIPTRY(launch_dispatch(g->inds, nk, E, (int*)(w + L.dcounts), perm, inv, off, s));
  HIPTRY(launch_experts_mix(dt, g->x, xprev, g->x_k, perm, g->inds, N, d.T, C, E, k, w + L.xkg, s));
  HIPTRY(launch_grouped_gemm(dt, false, w + L.xkg, C, g->w_key, C, (long long)F * C, C, nk, F, off, E, w + L.P, F,
                             "experts_bwd_key", s));
  // u_j = dO[t] · W_val,e, then dw_j = <h_j, u_j> and dp_j = g_j · u_j ⊙ 2·relu(p_j)
  HIPTRY(launch_exb_gather(dt, g->d_out, perm, g->logits, g->inds, nk, C, E, k, w + L.dog, gr, s));
  HIPTRY(launch_transpose_pad(dt, g->w_value, C, F, F, w + L.wT, C, s, E, (long long)C * F, (long long)F * C));
  HIPTRY(launch_grouped_gemm(dt, false, w + L.dog, C, w + L.wT, C, (long long)F * C, C, nk, F, off, E, w + L.U, F,
                             "experts_bwd_u", s));
  HIPTRY(launch_exb_hidden(dt, w + L.P, w + L.U, gr, nk, F, w + L.U, dw, s));
  // dk_j = dp_j · W_key,e
  const bool need_dk = g->d_x || g->d_x_prev || g->d_x_k;
  if (need_dk) {
    HIPTRY(launch_transpose_pad(dt, g->w_key, F, C, C, w + L.wT, F, s, E, (long long)F * C, (long long)C * F));
    HIPTRY(launch_grouped_gemm(dt, false, w + L.U, F, w + L.wT, F, (long long)C * F, F, nk, C, off, E, w + L.dk, C,
                               "experts_bwd_dk", s));
  }
  // router cotangents
  if (g->d_x || g->d_x_prev || g->d_w_gate)
    HIPTRY(launch_exb_route(g->logits, g->inds, inv, dw, off, g->d_losses, N, E, k, dl, s));
  if (g->d_x || g->d_x_prev)
    HIPTRY(launch_exb_dx(dt, w + L.dk, inv, g->inds, g->x_k, dl, g->w_gate, N, d.T, C, E, k, g->d_x, g->d_x_prev, s));
  if (g->d_x_k)
    HIPTRY(launch_exb_colsum(dt, 0, w + L.dk, g->x, xprev, off, perm, nullptr, N, d.T, C, E, k,
                             (float*)(w + L.cpart), g->d_x_k, s));
  if (g->d_w_gate)
    HIPTRY(launch_exb_colsum(dt, 1, nullptr, g->x, nullptr, off, perm, dl, N, d.T, C, E, k, (float*)(w + L.cpart),
                             g->d_w_gate, s));
  // weight gradients: one grouped-K product each, expert e contracting over
  // its own packed token range (zero past its count)
  if (g->d_w_key || g->d_w_value) {
    int* koff = (int*)(w + L.koff);
    const int ld = L.ncol;
    HIPTRY(launch_exb_koff(off, E, koff, s));
    if (g->d_w_key) {
      HIPTRY(launch_exb_seg_transpose(dt, 0, w + L.U, F, off, koff, E, ld, nullptr, w + L.tA, s));    // dpᵀ
      HIPTRY(launch_exb_seg_transpose(dt, 0, w + L.xkg, C, off, koff, E, ld, nullptr, w + L.tB, s));  // xkᵀ
      HIPTRY(launch_gemm_grouped_k(dt, w + L.tA, ld, w + L.tB, ld, koff, E, F, C, g->d_w_key, C, (long long)F * C,
                                   "experts_bwd_dwk", s));
    }
    if (g->d_w_value) {
      HIPTRY(launch_exb_seg_transpose(dt, 2, w + L.dog, C, off, koff, E, ld, gr, w + L.tA, s));     // (g·dO)ᵀ
      HIPTRY(launch_exb_seg_transpose(dt, 1, w + L.P, F, off, koff, E, ld, nullptr, w + L.tB, s));  // hᵀ
      HIPTRY(launch_gemm_grouped_k(dt, w + L.tA, ld, w + L.tB, ld, koff, E, C, F, g->d_w_value, F, (long long)C * F,
                                   "experts_bwd_dwv", s));
    }
  }
  return RWKVMOE_OK;
}

int ortho_backward_impl(const rwkvmoe_desc* desc, const rwkvmoe_grads* g, void* ws, size_t ws_bytes, void* stream) {
  Dims d;
  TRY(check_bwd_desc(desc, &d));
  if (!g) return RWKVMOE_ERR_NULL_DESC;
  TRY(need(g->lora_A)); TRY(need(g->d_lora_A));
  TRY(elem_ok(g->lora_A, d.s)); TRY(elem_ok(g->d_lora_A, d.s)); TRY(elem_ok(g->d_ortho, 4));
  const BwdLayout L = bwd_layout(d);
  if (!ws || ws_bytes < L.total || !aligned(ws, 256)) return RWKVMOE_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  char* w = (char*)ws;
  const int dt = d.dtype, C = d.C, E = d.E, kx = d.kx;
  float* part = (float*)(w + L.splitk);
  // A_all and A_T only
  HIPTRY(launch_bwd_prep(dt, g->lora_A, nullptr, nullptr, E, C, d.r, kx, L.ep, false, w + L.at, w + L.a_t, nullptr,
                         nullptr, nullptr, 0, nullptr, s));
  HIPTRY(launch_gemm_nt(dt, w + L.at, C, w + L.at, C, C, nullptr, 0, nullptr, 0, 0, kx, kx, w + L.gram, kx, part,
                        "ortho_gram", s));
  HIPTRY(launch_ortho_mask(dt, w + L.gram, E * d.r, d.r, kx, g->d_ortho, s));
  HIPTRY(launch_gemm_nt(dt, w + L.a_t, kx, w + L.gram, kx, kx, nullptr, 0, nullptr, 0, 0, C, kx, w + L.o, kx, part,
                        "ortho_da", s));
  HIPTRY(launch_bwd_finish(dt, nullptr, 1, w + L.o, E, C, d.r, kx, 0, g->d_lora_A, nullptr, nullptr, 1, nullptr, s));
  return RWKVMOE_OK;
}

}  // namespace

namespace rwkvmoe {
// Argument checks of rwkvmoe_forward without its workspace (host only).
int forward_check(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t) {
  return forward_impl(desc, t, nullptr, 0, nullptr, false, true);
}
}  // namespace rwkvmoe

extern "C" {

const char* rwkvmoe_status_string(int status) {
  switch (status) {
    case RWKVMOE_OK: return "success";
    case RWKVMOE_ERR_NULL_DESC: return "desc or tensors pointer is NULL";
    case RWKVMOE_ERR_SHAPE: return "a dimension is out of range or not a multiple of 64";
    case RWKVMOE_ERR_DTYPE: return "dtype is not one of RWKVMOE_F32/F16/BF16";
    case RWKVMOE_ERR_NULL_PTR: return "a tensor required by this entry point is NULL";
    case RWKVMOE_ERR_ALIGN: return "a tensor pointer is not suitably aligned";
    case RWKVMOE_ERR_WORKSPACE: return "workspace is NULL, not 256-byte aligned or smaller than rwkvmoe_workspace_bytes";
    case RWKVMOE_ERR_TOPK: return "top_k must be in 1..min(n_experts, 8)";
    case RWKVMOE_ERR_FLAGS: return "unknown flag, or a flag set without its tensor";
    case RWKVMOE_ERR_MODE: return "unknown mode, or decode without seq_len == 1 and x_prev";
    case RWKVMOE_ERR_EVENTS: return "events, names or n_kernels is NULL, or fewer than RWKVMOE_MAX_KERNELS + 1 events";
    case RWKVMOE_ERR_SCRATCH:
      return "the layer's workspace exceeds the RWKVMOE_NOALLOC_SCRATCH_BYTES the no-allocation forward holds";
    case RWKVMOE_ERR_VERSION:
      return "rwkvmoe_tensors.struct_size is not this library's sizeof(rwkvmoe_tensors): the caller was built "
             "against another version of rwkvmoe.h";
    default: break;
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown status";
}

int rwkvmoe_version(void) { return 200; }

int rwkvmoe_workspace_bytes(const rwkvmoe_desc* desc, size_t* bytes) {
  Dims d;
  TRY(check_desc(desc, &d));
  if (!bytes) return RWKVMOE_ERR_NULL_PTR;
  *bytes = layout(d).total;
  return RWKVMOE_OK;
}

int rwkvmoe_prepared_bytes(const rwkvmoe_desc* desc, size_t* bytes) {
  Dims d;
  TRY(check_desc(desc, &d));
  if (!bytes) return RWKVMOE_ERR_NULL_PTR;
  *bytes = prep_layout(d).total;
  return RWKVMOE_OK;
}

int rwkvmoe_prepare_adapters(const rwkvmoe_desc* desc, const void* lora_A, const void* lora_B, void* prepared,
                             size_t prepared_bytes, void* stream) {
  Dims d;
  TRY(check_desc(desc, &d));
  TRY(need(lora_A)); TRY(need(lora_B)); TRY(need(prepared));
  TRY(elem_ok(lora_A, d.sa)); TRY(elem_ok(lora_B, d.sa));
  const PrepLayout P = prep_layout(d);
  if (prepared_bytes < P.total || !aligned(prepared, 256)) return RWKVMOE_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  char* w = (char*)prepared;
  // fragment order (the router's adapter product) and row-major A_all, B_all;
  // a32rows: row-major fp32 (the fp32 grouped LoRA's operands) only
  if (d.a32rows) {
    HIPTRY(launch_lora_prep(RWKVMOE_F32, lora_A, lora_B, d.E, d.C, d.r, d.kx, w + P.row, w + P.b, s, false, false));
    return RWKVMOE_OK;
  }
  if (d.dtype != RWKVMOE_F32)
    HIPTRY(launch_lora_prep(d.dtype, lora_A, lora_B, d.E, d.C, d.r, d.kx, w + P.frag, w + P.b, s, true, d.ad32));
  HIPTRY(launch_lora_prep(d.dtype, lora_A, lora_B, d.E, d.C, d.r, d.kx, w + P.row, w + P.b, s, false, d.ad32));
  return RWKVMOE_OK;
}

int rwkvmoe_prepared_base_bytes(const rwkvmoe_desc* desc, size_t* bytes) {
  Dims d;
  TRY(check_desc(desc, &d));
  if (!bytes) return RWKVMOE_ERR_NULL_PTR;
  if (d.dtype == RWKVMOE_F32) return RWKVMOE_ERR_DTYPE;
  *bytes = base_layout(d).total;
  return RWKVMOE_OK;
}

int rwkvmoe_prepare_base(const rwkvmoe_desc* desc, const void* w_key, const void* w_value, void* prepared_base,
                         size_t prepared_bytes, void* stream) {
  Dims d;
  TRY(check_desc(desc, &d));
  if (d.dtype == RWKVMOE_F32) return RWKVMOE_ERR_DTYPE;
  TRY(need(w_key)); TRY(need(w_value)); TRY(need(prepared_base));
  TRY(vec_ok(w_key)); TRY(vec_ok(w_value));
  const BaseLayout B = base_layout(d);
  if (prepared_bytes < B.total || !aligned(prepared_base, 256)) return RWKVMOE_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  char* w = (char*)prepared_base;
  HIPTRY(launch_frag_pack(d.dtype, w_key, w + B.wk, d.F, d.C, s));
  HIPTRY(launch_frag_pack(d.dtype, w_value, w + B.wv, d.C, d.F, s));
  return RWKVMOE_OK;
}

int rwkvmoe_reads_prepared_base(const rwkvmoe_desc* desc, int* reads) {
  Dims d;
  TRY(check_desc(desc, &d));
  if (!reads) return RWKVMOE_ERR_NULL_PTR;
  *reads = d.dec ? 1 : 0;
  return RWKVMOE_OK;
}

int rwkvmoe_backward_workspace_bytes(const rwkvmoe_desc* desc, size_t* bytes) {
  Dims d;
  TRY(check_bwd_desc(desc, &d));
  if (!bytes) return RWKVMOE_ERR_NULL_PTR;
  *bytes = bwd_layout(d).total;
  return RWKVMOE_OK;
}

int rwkvmoe_layer_norm_backward_workspace_bytes(const rwkvmoe_desc* desc, size_t* bytes) {
  Dims d;
  TRY(check_desc(desc, &d));
  if (!bytes) return RWKVMOE_ERR_NULL_PTR;
  *bytes = layer_norm_bwd_part_bytes(d.N, d.C);
  return RWKVMOE_OK;
}

int rwkvmoe_layer_norm_backward(const rwkvmoe_desc* desc, const rwkvmoe_ln_grads* g, void* ws, size_t ws_bytes,
                                void* stream) {
  Dims d;
  TRY(check_desc(desc, &d));
  if (!g) return RWKVMOE_ERR_NULL_DESC;
  TRY(need(g->x)); TRY(need(g->ln_weight)); TRY(need(g->d_y));
  TRY(vec_ok(g->x)); TRY(vec_ok(g->ln_weight)); TRY(vec_ok(g->d_y)); TRY(vec_ok(g->d_res)); TRY(vec_ok(g->d_x));
  TRY(elem_ok(g->d_ln_weight, d.s)); TRY(elem_ok(g->d_ln_bias, d.s));
  const bool cols = g->d_ln_weight || g->d_ln_bias;
  if (cols && (!ws || ws_bytes < layer_norm_bwd_part_bytes(d.N, d.C) || !aligned(ws, 256)))
    return RWKVMOE_ERR_WORKSPACE;
  if (!g->d_x && !cols) return RWKVMOE_OK;
  HIPTRY(launch_layer_norm_bwd(d.dtype, g->x, g->ln_weight, g->d_y, g->d_res, g->d_x, g->d_ln_weight, g->d_ln_bias,
                               (float*)ws, d.N, d.C, (hipStream_t)stream));
  return RWKVMOE_OK;
}

int rwkvmoe_router_backward_workspace_bytes(const rwkvmoe_desc* desc, size_t* bytes) {
  Dims d;
  TRY(check_router_bwd_desc(desc, &d));
  if (!bytes) return RWKVMOE_ERR_NULL_PTR;
  *bytes = router_bwd_layout(d).total;
  return RWKVMOE_OK;
}

int rwkvmoe_router_backward(const rwkvmoe_desc* desc, const rwkvmoe_router_grads* g, void* ws, size_t ws_bytes,
                            void* stream) {
  return router_backward_impl(desc, g, ws, ws_bytes, stream);
}

int rwkvmoe_backward(const rwkvmoe_desc* desc, const rwkvmoe_grads* g, void* ws, size_t ws_bytes, void* stream) {
  return backward_impl(desc, g, ws, ws_bytes, stream);
}

int rwkvmoe_experts_backward_workspace_bytes(const rwkvmoe_desc* desc, size_t* bytes) {
  Dims d;
  TRY(check_exp_bwd_desc(desc, &d));
  if (!bytes) return RWKVMOE_ERR_NULL_PTR;
  *bytes = exp_bwd_layout(d).total;
  return RWKVMOE_OK;
}

int rwkvmoe_experts_backward(const rwkvmoe_desc* desc, const rwkvmoe_experts_grads* g, void* ws, size_t ws_bytes,
                             void* stream) {
  return experts_backward_impl(desc, g, ws, ws_bytes, stream);
}

int rwkvmoe_ortho_backward(const rwkvmoe_desc* desc, const rwkvmoe_grads* g, void* ws, size_t ws_bytes,
                           void* stream) {
  return ortho_backward_impl(desc, g, ws, ws_bytes, stream);
}

int rwkvmoe_experts_workspace_bytes(const rwkvmoe_desc* desc, size_t* bytes) {
  Dims d;
  TRY(check_experts_desc(desc, &d));
  if (!bytes) return RWKVMOE_ERR_NULL_PTR;
  *bytes = experts_layout(d).total;
  return RWKVMOE_OK;
}

int rwkvmoe_experts_forward(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t, void* ws, size_t ws_bytes,
                            void* stream) {
  return experts_forward_impl(desc, t, ws, ws_bytes, stream);
}

int rwkvmoe_forward(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t, void* ws, size_t ws_bytes, void* stream) {
  return forward_impl(desc, t, ws, ws_bytes, stream, false);
}

int rwkvmoe_decode(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t, void* ws, size_t ws_bytes, void* stream) {
  return forward_impl(desc, t, ws, ws_bytes, stream, true);
}

int rwkvmoe_forward_timed(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t, void* ws, size_t ws_bytes,
                          void* stream, void* const* events, int n_events, const char** names, int* n_kernels) {
  if (!events || !names || !n_kernels || n_events < RWKVMOE_MAX_KERNELS + 1) return RWKVMOE_ERR_EVENTS;
  const bool pairs = n_events >= RWKVMOE_TIMED_PAIR_EVENTS;
  for (int i = 0; i < (pairs ? RWKVMOE_TIMED_PAIR_EVENTS : RWKVMOE_MAX_KERNELS + 1); ++i)
    if (!events[i]) return RWKVMOE_ERR_EVENTS;
  Probe p{(hipEvent_t*)events, names, RWKVMOE_MAX_KERNELS, 0, pairs, 0};
  *n_kernels = 0;
  probe_slot() = &p;
  const int st = forward_impl(desc, t, ws, ws_bytes, stream, false);
  probe_slot() = nullptr;
  *n_kernels = p.n < p.cap ? p.n : p.cap;
  return st;
}

int rwkvmoe_router_topk(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t, void* ws, size_t ws_bytes,
                        void* stream) {
  Ctx c;
  TRY(setup(desc, t, ws, ws_bytes, stream, &c));
  TRY(need(t->x)); TRY(need(t->w_gate));
  TRY(check_flag_tensors(c.d, t, false, true, false));
  return run_router(c, false, false, true);
}

int rwkvmoe_dispatch(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t, void* ws, size_t ws_bytes, void* stream) {
  Ctx c;
  TRY(setup(desc, t, ws, ws_bytes, stream, &c));
  TRY(need(t->inds)); TRY(need(t->perm)); TRY(need(t->inv_perm)); TRY(need(t->offsets));
  return run_dispatch(c, false);
}

int rwkvmoe_cmix_key(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t, void* ws, size_t ws_bytes, void* stream) {
  Ctx c;
  TRY(setup(desc, t, ws, ws_bytes, stream, &c));
  TRY(need(t->x)); TRY(need(t->x_k)); TRY(need(t->w_key)); TRY(need(t->hidden));
  TRY(check_flag_tensors(c.d, t, true, false, false));
  return run_key(c, false, false, false);
}

int rwkvmoe_cmix_value(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t, void* ws, size_t ws_bytes,
                       void* stream) {
  Ctx c;
  TRY(setup(desc, t, ws, ws_bytes, stream, &c));
  TRY(need(t->hidden)); TRY(need(t->w_value)); TRY(need(t->base_out));
  const Dims& d = c.d;
  HIPTRY(launch_cmix_value(d.dtype, t->hidden, t->w_value, d.F, nullptr, nullptr, 0, nullptr, t->base_out, d.N, d.C,
                           c.part(), c.s));
  return RWKVMOE_OK;
}

int rwkvmoe_lora_grouped(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t, void* ws, size_t ws_bytes,
                         void* stream) {
  Ctx c;
  TRY(setup(desc, t, ws, ws_bytes, stream, &c));
  TRY(need(t->x)); TRY(need(t->lora_A)); TRY(need(t->lora_B)); TRY(need(t->perm)); TRY(need(t->offsets));
  TRY(need(t->adapter_rows));
  TRY(run_prep(c));
  TRY(run_lora(c, t->x, t->perm, t->offsets, t->adapter_rows));
  return RWKVMOE_OK;
}

int rwkvmoe_combine(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t, void* ws, size_t ws_bytes, void* stream) {
  Ctx c;
  TRY(setup(desc, t, ws, ws_bytes, stream, &c));
  TRY(need(t->base_out)); TRY(need(t->adapter_rows)); TRY(need(t->inds)); TRY(need(t->gates)); TRY(need(t->out));
  TRY(check_flag_tensors(c.d, t, false, false, true));
  const Dims& d = c.d;
  HIPTRY(launch_combine(d.dtype, t->base_out, t->adapter_rows, t->inds, t->gates, nullptr, c.resid(), t->out, d.N,
                        d.C, d.k, c.s, d.ad32));
  return RWKVMOE_OK;
}

int rwkvmoe_ortho_loss(const rwkvmoe_desc* desc, const rwkvmoe_tensors* t, void* ws, size_t ws_bytes,
                       void* stream) {
  Ctx c;
  TRY(setup(desc, t, ws, ws_bytes, stream, &c));
  TRY(need(t->lora_A)); TRY(need(t->ortho_loss));
  return run_ortho(c);
}

}  // extern "C"
