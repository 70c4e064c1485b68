"""LoRA-MoE ChannelMix on MI355X: PyTorch mirrors of the reference's
``Router`` (rwkv_mlx/moe.py:35-86) and ``LoRAMoE_CMix`` (rwkv_mlx/moe.py:93-163)
whose forward runs librwkvmoe's hand-written gfx950 kernels through the C ABI.

Drop-in contract (same as the reference):
  * ``LoRAMoE_CMix(base, n_experts, lora_rank, top_k=2)``; ``base`` exposes
    ``x_k (1,1,C)``, ``key.weight (F,C)``, ``value.weight (C,F)``.
  * ``forward(x)`` with x (B,T,C) returns ``(out (B,T,C), aux_loss, z_loss)``.
  * parameters ``lora_A (E,C,r)``, ``lora_B (E,r,C)``, ``router.gate.weight
    (E,C)``, ``base.*`` — the reference's state-dict keys.
  * ``orthogonal_loss()`` returns Σ_{i<j} ||A_iᵀ A_j||_F².

Differences, all deliberate:
  * ``Router.forward`` returns expert indices as int32 (MLX returns uint32;
    the values are identical) in descending-logit order with ties to the
    lower id, which for top_k <= 2 is exactly MLX's argpartition order.
  * Router logits follow an order-fixed chunked definition (64-wide chunks
    accumulated with one fused multiply-add per term, in fp32 when x and the
    gate are 16-bit and in fp64 when either is fp32; chunks summed in fp64;
    one rounding to fp32); moe.py:56 sums in fp32 in an order MLX does not
    specify.
  * Optional extensions the reference lacks: ``x_prev`` (carried token-shift
    state, for RNN-mode decode), ``residual`` (fused Block residual add),
    ``ln`` (the Block's ln2 applied to x inside the layer's launches),
    ``Router.logit_bias`` (a fixed (E,) fp32 bias on the logits) and
    ``mode`` ("fused" MFMA K-extension or "sparse" dispatch/grouped/combine).
  * Mixed parameter/activation dtypes follow MLX type promotion op by op
    (``_dtype_plan``): the reference's fine-tune layer (fp16 x and base, fp32
    router gate and adapters) runs its base in fp16, its router on the fp32
    gate as stored, casts the gates to fp16 and computes the delta and the
    output in fp32; a bf16 base with fp32 adapters (the adapters and gate
    LoRAMoE_CMix creates, moe.py:47, 121-125, on a bf16 base) likewise, its
    delta as fp32 adapter rows (SPARSE).  One combination the reference's
    tools do not produce is computed wholly in fp32 instead (which skips
    MLX's rounding of shift(x) - x to x's dtype): base weights of another
    dtype than x.
"""
from __future__ import annotations

import math

import torch
from torch import nn

from . import _lib
from .model import _WS, RWKV_CMix_x070, RWKVConfig, require_device

__all__ = ["Router", "LoRAMoE_CMix", "MoE_CMix", "RWKV_CMix_x070", "RWKVConfig", "channel_mixing_rnn"]


def _promote(*dts: torch.dtype) -> torch.dtype:
    out = dts[0]
    for d in dts[1:]:
        out = torch.promote_types(out, d)
    if out not in _lib.TORCH_DTYPE_CODE:
        raise TypeError(f"unsupported dtype {out}; use float32, float16 or bfloat16")
    return out


def _gate_plan(dt: torch.dtype, gate_dtype: torch.dtype):
    """(dtype W_gate is passed in, flag) for a layer computing in dt: the
    gate as stored when it matches, else fp32 with GATE_F32 (fp32(x)·fp32(W),
    moe.py:56; a 16-bit gate converts to fp32 exactly)."""
    if dt == torch.float32 or gate_dtype == dt:
        return dt, 0
    return torch.float32, _lib.GATE_F32


def _dtype_plan(x_dtype, base_dtypes, gate_dtype, adapter_dtypes):
    """MLX promotion of LoRAMoE_CMix's operands onto the library's dtypes.

    Returns (dt, gate_dt, adapter_dt, flags, out_dt): dt for x and the base
    (promote(x, x_k, W_key, W_value), model.py:259-263); the dtypes W_gate and
    lora_A / lora_B are passed in; the RWKVMOE_* dtype flags; and the output
    dtype promote(dt, lora_A, lora_B) (moe.py:138-147)."""
    dt = _promote(x_dtype, *base_dtypes)
    if dt == torch.float32:
        return dt, dt, dt, 0, dt
    gdt, flags = _gate_plan(dt, gate_dtype)
    odt = _promote(dt, *adapter_dtypes)
    if odt == dt:
        return dt, gdt, dt, flags, dt
    # a 16-bit base with fp32 adapters (or with those of the other 16-bit
    # type, which promote to fp32 with it): the delta and out in fp32
    return dt, gdt, torch.float32, flags | _lib.ADAPTERS_F32, torch.float32


class _RouterFunction(torch.autograd.Function):
    """Autograd node of the standalone Router: forward through
    rwkvmoe_router_topk (logits kept for the VJP), VJP through
    rwkvmoe_router_backward.  Gradients reach x and router.gate.weight from
    the gates' and the two losses' cotangents; the indices are integers."""

    @staticmethod
    def forward(ctx, x, wg, bias, dims):
        B, T, C, E, k, dt = dims
        flags = _lib.HAS_BIAS if bias is not None else 0
        desc = _lib.make_desc(B, T, C, 64, E, k, 1, dt, _lib.MODE_FUSED, flags)
        nbytes = _lib.workspace_bytes(desc)
        ws = _WS.get(x.device, nbytes)
        inds = torch.empty(B, T, k, dtype=torch.int32, device=x.device)
        gates = torch.empty(B, T, k, dtype=dt, device=x.device)
        losses = torch.empty(2, dtype=torch.float32, device=x.device)
        logits = torch.empty(B * T, E, dtype=torch.float32, device=x.device)
        t = _lib.make_tensors(x=x, w_gate=wg, logit_bias=bias, inds=inds, gates=gates, losses=losses, logits=logits)
        _lib.call("rwkvmoe_router_topk", desc, t, ws, nbytes, _lib.current_stream(x.device))
        ctx.save_for_backward(x, wg, logits, inds)
        ctx.desc = desc
        ctx.mark_non_differentiable(inds)
        return inds, gates, losses

    @staticmethod
    def backward(ctx, d_inds, d_gates, d_losses):
        x, wg, logits, inds = ctx.saved_tensors
        need = ctx.needs_input_grad
        grads = {}
        if need[0]:
            grads["d_x"] = torch.empty_like(x)
        if need[1]:
            grads["d_w_gate"] = torch.empty_like(wg)
        if grads:
            dg = None if d_gates is None else d_gates.to(x.dtype).contiguous()
            dl = None if d_losses is None else d_losses.to(torch.float32).contiguous()
            nbytes = _lib.router_backward_workspace_bytes(ctx.desc)
            ws = _WS.get(x.device, nbytes)
            _lib.router_backward(ctx.desc, ws, nbytes, _lib.current_stream(x.device), x=x, w_gate=wg, logits=logits,
                                 inds=inds, d_gates=dg, d_losses=dl, **grads)
        return grads.get("d_x"), grads.get("d_w_gate"), None, None


class Router(nn.Module):
    """Token router: linear gate, top-k, softmax gates, aux and z losses
    (rwkv_mlx/moe.py:35-86).  Differentiable like the reference's module:
    while autograd records, the call is one node whose VJP
    (rwkvmoe_router_backward) gives x and gate.weight their gradients from
    the gates', aux_loss's and z_loss's cotangents (a gate stored in another
    dtype than x trains on the promoted dtype)."""

    def __init__(self, d_model: int, n_experts: int, top_k: int = 2):
        super().__init__()
        self.gate = nn.Linear(d_model, n_experts, bias=False)
        self.n_experts = n_experts
        self.top_k = top_k
        self.logit_bias: torch.Tensor | None = None  # optional (E,) fp32

    def forward(self, x: torch.Tensor):
        """Returns (inds (B,T,k) int32, weights (B,T,k) x.dtype, aux_loss, z_loss)."""
        require_device(x, "Router")
        if x.dim() != 3:
            raise ValueError(f"Router expects (B, T, C), got {tuple(x.shape)}")
        B, T, C = x.shape
        E, k = self.n_experts, self.top_k
        dt = x.dtype
        if dt not in _lib.TORCH_DTYPE_CODE:
            raise TypeError(f"unsupported dtype {dt}")
        if B * T == 0:  # MLX: empty selections, and means over no tokens are NaN
            nan = torch.full((), float("nan"), dtype=torch.float32, device=x.device)
            return (torch.empty(B, T, k, dtype=torch.int32, device=x.device),
                    torch.empty(B, T, k, dtype=dt, device=x.device), nan, nan.clone())
        if torch.is_grad_enabled() and (x.requires_grad or self.gate.weight.requires_grad):
            ct = _promote(dt, self.gate.weight.dtype)  # one dtype for the VJP
            bias = self.logit_bias
            if bias is not None:
                bias = bias.detach().to(device=x.device, dtype=torch.float32).contiguous()
            inds, gates, losses = _RouterFunction.apply(
                x.to(ct).contiguous(), self.gate.weight.to(device=x.device, dtype=ct).contiguous(), bias,
                (B, T, C, E, k, ct))
            return inds, gates.to(dt), losses[0], losses[1]  # gates in x's dtype (moe.py:86)
        x = x.contiguous()
        gdt, flags = _gate_plan(dt, self.gate.weight.dtype)  # the gate as stored (moe.py:56)
        wg = self.gate.weight.detach().to(device=x.device, dtype=gdt).contiguous()
        bias = self.logit_bias
        if bias is not None:
            bias = bias.detach().to(device=x.device, dtype=torch.float32).contiguous()
            flags |= _lib.HAS_BIAS
        desc = _lib.make_desc(B, T, C, 64, E, k, 1, dt, _lib.MODE_FUSED, flags)
        nbytes = _lib.workspace_bytes(desc)
        ws = _WS.get(x.device, nbytes)
        inds = torch.empty(B, T, k, dtype=torch.int32, device=x.device)
        gates = torch.empty(B, T, k, dtype=dt, device=x.device)
        losses = torch.empty(2, dtype=torch.float32, device=x.device)
        t = _lib.make_tensors(x=x, w_gate=wg, logit_bias=bias, inds=inds, gates=gates, losses=losses)
        _lib.call("rwkvmoe_router_topk", desc, t, ws, nbytes, _lib.current_stream(x.device))
        return inds, gates, losses[0], losses[1]


def _ln_params(ln):
    """(weight, bias, eps) of the Block's ln2: an nn.LayerNorm (model.py:283)
    or a (weight, bias) pair (eps 1e-5, MLX's default)."""
    if isinstance(ln, nn.LayerNorm):
        if ln.weight is None or ln.bias is None:
            raise ValueError("ln2 must be an affine LayerNorm (weight and bias), as nn.LayerNorm(C) in MLX")
        return ln.weight, ln.bias, ln.eps
    w, b = ln
    return w, b, 1e-5


def _ln_torch(x, w, b, eps):
    """ln2 evaluated by torch, for the calls the library does not fuse
    (training, mixed dtypes): fp32 statistics, output in promote(x, w, b)
    (MLX's dtype for mx.fast.layer_norm on these operands)."""
    odt = _promote(x.dtype, w.dtype, b.dtype)
    return torch.nn.functional.layer_norm(x.float(), (x.shape[-1],), w.float(), b.float(), eps=eps).to(odt)


def _ln_fused_ok(x, w, b, eps, dt):
    """The library applies ln2 itself (RWKVMOE_LN_IN) when x, ln2 and the
    layer share one dtype and eps is MLX's 1e-5."""
    return eps == 1e-5 and x.dtype == w.dtype == b.dtype == dt


def _run_forward(x, xp, xk, wk, wv, wg, A, Bm, bias, res, dims, mode, extras, dflags=0, odt=None, ln=None):
    """rwkvmoe_forward on prepared (dtype-converted, contiguous) operands.
    Returns (out, losses (2,) fp32, desc); `extras` (a dict or None)
    receives the tensors it names (logits, inds, gates, x_ln) as optional
    outputs.  dflags: the dtype flags of a mixed layer (GATE_F32,
    ADAPTERS_F32), whose output dtype is odt.  ln: ln2's (weight, bias), run
    in front of the layer (RWKVMOE_LN_IN)."""
    B, T, C, F, E, k, r, dt = dims
    flags = (_lib.HAS_PREV if xp is not None else 0) | (_lib.HAS_BIAS if bias is not None else 0) \
        | (_lib.ADD_RESIDUAL if res is not None else 0) | (_lib.LN_IN if ln is not None else 0) | dflags
    desc = _lib.make_desc(B, T, C, F, E, k, r, dt, mode, flags)
    nbytes = _lib.workspace_bytes(desc)
    ws = _WS.get(x.device, nbytes)
    out = torch.empty(x.shape, dtype=odt or x.dtype, device=x.device)
    losses = torch.empty(2, dtype=torch.float32, device=x.device)
    lnkw = dict(ln_weight=ln[0], ln_bias=ln[1]) if ln is not None else {}
    t = _lib.make_tensors(x=x, x_prev=xp, x_k=xk, w_key=wk, w_value=wv, w_gate=wg, lora_A=A, lora_B=Bm,
                          logit_bias=bias, residual=res, out=out, losses=losses, **lnkw, **(extras or {}))
    _lib.call("rwkvmoe_forward", desc, t, ws, nbytes, _lib.current_stream(x.device))
    return out, losses, desc


def _ln_backward(x, lnw, d_y, d_res, need_x, need_w, need_b, dims):
    """The VJP of ln2 (rwkvmoe_layer_norm_backward) at ln2's input x:
    returns (d_x or None, d_ln_weight or None, d_ln_bias or None), with
    d_res (the residual branch's cotangent, or None) added to d_x.  d_y is
    rounded to x's dtype, the dtype of the layer input LN(x) whose
    cotangent it is."""
    B, T, C, F, E, k, r = dims
    d_y = d_y.to(x.dtype).contiguous()
    g = {}
    if need_x:
        g["d_x"] = d_y  # (written in place: d_x may alias d_y)
    if need_w:
        g["d_ln_weight"] = torch.empty_like(lnw)
    if need_b:
        g["d_ln_bias"] = torch.empty_like(lnw)
    if g:
        desc = _lib.make_desc(B, T, C, F, E, k, r, x.dtype)
        nbytes = _lib.layer_norm_backward_workspace_bytes(desc)
        ws = _WS.get(x.device, nbytes)
        dr = d_res.to(x.dtype).contiguous() if need_x and d_res is not None else None
        _lib.layer_norm_backward(desc, ws, nbytes, _lib.current_stream(x.device), x=x, ln_weight=lnw, d_y=d_y,
                                 d_res=dr, **g)
    return g.get("d_x"), g.get("d_ln_weight"), g.get("d_ln_bias")


class _LoRAMoEFunction(torch.autograd.Function):
    """Autograd node of LoRAMoE_CMix: forward through rwkvmoe_forward, VJP
    through rwkvmoe_backward.  Gradients reach x, lora_A, lora_B and
    router.gate.weight; the base output is under stop_gradient (moe.py:131),
    so x_k, key.weight and value.weight receive none, and a residual receives
    d_out.

    The fine-tune layer (fp16 x and base, fp32 gate and / or adapters; dtype
    flags `dflags`) runs its MLX-promoted forward, and its VJP runs as the
    fp32 backward on x converted to fp32 (exact) with the gates rounded to
    fp16 as that forward kept them (RWKVMOE_GATES_F16); each gradient is
    returned in its input's dtype."""

    @staticmethod
    def forward(ctx, x, A, Bm, wg, xk, wk, wv, bias, xp, res, dims, mode, dflags, odt, lnw=None, lnb=None,
                res_is_x=False):
        N = dims[0] * dims[1]
        E, k = dims[4], dims[5]
        ex = {"logits": torch.empty(N, E, dtype=torch.float32, device=x.device),
              "inds": torch.empty(N, k, dtype=torch.int32, device=x.device)}
        ln = None
        if lnw is not None:  # ln2 in the layer's launches; LN(x) kept as the VJP's layer input
            ex["x_ln"] = torch.empty_like(x)
            ln = (lnw.detach(), lnb.detach())
        out, losses, _ = _run_forward(x, xp, xk, wk, wv, wg, A, Bm, bias, res, dims, mode, ex, dflags, odt, ln)
        xl = ex["x_ln"] if ln is not None else x
        ctx.save_for_backward(xl, A, Bm, wg, ex["logits"], ex["inds"], x if ln is not None else None, lnw)
        B, T, C, F, E, k, r, dt = dims
        if dflags:
            ctx.desc = _lib.make_desc(B, T, C, F, E, k, r, torch.float32, mode, _lib.GATES_F16)
        else:
            ctx.desc = _lib.make_desc(B, T, C, F, E, k, r, dt, mode)
        ctx.dims = (B, T, C, F, E, k, r)
        ctx.mixed = dflags != 0
        ctx.has_res = res is not None
        ctx.ln = ln is not None
        ctx.res_is_x = res_is_x and ln is not None and res is not None
        return out, losses

    @staticmethod
    def backward(ctx, d_out, d_losses):
        x, A, Bm, wg, logits, inds, x0, lnw = ctx.saved_tensors
        need = ctx.needs_input_grad
        # x: the layer's input (LN(x0) with ln2); its cotangent feeds ln2's VJP
        need_ln = ctx.ln and (need[0] or need[14] or need[15])
        # the backward's operands: the layer's own, or fp32 ones for the fine-tune layer
        cdt = torch.float32 if ctx.mixed else x.dtype
        xb, Ab, Bb, wgb = [t.to(cdt).contiguous() for t in (x, A, Bm, wg)]
        grads = {}
        if need[0] or need_ln:
            grads["d_x"] = torch.empty_like(xb)
        if need[1]:
            grads["d_lora_A"] = torch.empty_like(Ab)
        if need[2]:
            grads["d_lora_B"] = torch.empty_like(Bb)
        if need[3]:
            grads["d_w_gate"] = torch.empty_like(wgb)
        if d_out is None:
            d_out = torch.zeros(x.shape, dtype=cdt, device=x.device)
        if grads:
            dob = d_out.to(cdt).contiguous()
            dl = None if d_losses is None else d_losses.to(torch.float32).contiguous()
            nbytes = _lib.backward_workspace_bytes(ctx.desc)
            ws = _WS.get(x.device, nbytes)
            _lib.backward(ctx.desc, ws, nbytes, _lib.current_stream(x.device), x=xb, w_gate=wgb, lora_A=Ab, lora_B=Bb,
                          logits=logits, inds=inds, d_out=dob, d_losses=dl, **grads)
        d_x = grads.get("d_x")
        d_lnw = d_lnb = None
        fuse_res = ctx.res_is_x and need[0]  # x + ffn(ln2(x)): d_out joins d_x inside ln2's VJP
        if need_ln:
            d_x, d_lnw, d_lnb = _ln_backward(x0, lnw, d_x, d_out if fuse_res else None, need[0], need[14], need[15],
                                             ctx.dims)
        d_res = d_out if ctx.has_res and need[9] and not fuse_res else None
        cast = lambda g, like: None if g is None else g.to(like.dtype)
        return (cast(d_x, x0 if ctx.ln else x), cast(grads.get("d_lora_A"), A), cast(grads.get("d_lora_B"), Bm),
                cast(grads.get("d_w_gate"), wg), None, None, None, None, None, d_res, None, None, None, None,
                d_lnw, d_lnb, None)


class _OrthoFunction(torch.autograd.Function):
    """orthogonal_loss (moe.py:149-163) with its gradient through
    rwkvmoe_ortho_backward: d lora_A_i = 2 Σ_{j≠i} A_j (A_jᵀ A_i) · d_ortho."""

    @staticmethod
    def forward(ctx, A, desc):
        nbytes = _lib.workspace_bytes(desc)
        ws = _WS.get(A.device, nbytes)
        out = torch.empty(1, dtype=torch.float32, device=A.device)
        t = _lib.make_tensors(lora_A=A, ortho_loss=out)
        _lib.call("rwkvmoe_ortho_loss", desc, t, ws, nbytes, _lib.current_stream(A.device))
        ctx.save_for_backward(A)
        ctx.desc = desc
        return out

    @staticmethod
    def backward(ctx, d):
        (A,) = ctx.saved_tensors
        dA = torch.empty_like(A)
        nbytes = _lib.backward_workspace_bytes(ctx.desc)
        ws = _WS.get(A.device, nbytes)
        _lib.backward(ctx.desc, ws, nbytes, _lib.current_stream(A.device), entry="rwkvmoe_ortho_backward", lora_A=A,
                      d_lora_A=dA, d_ortho=d.to(torch.float32).contiguous())
        return dA, None


class _SourceKey:
    """What a cached kernel layout was made from: for each source parameter
    a detached alias (it shares the parameter's storage and version counter
    and keeps that storage alive, so no later tensor can take its address),
    its version counter at the time, and the call's own key (compute dtype,
    flags, device).  It matches while every parameter still holds the same
    storage at the same version: ``p.data = t`` swaps the storage, and
    in-place updates through the parameter move the counter."""

    def __init__(self, params, extra):
        self.alias = tuple(p.detach() for p in params)
        self.state = tuple((p._version, p.dtype, tuple(p.shape)) for p in params)
        self.extra = extra

    def matches(self, params, extra) -> bool:
        if extra != self.extra or len(params) != len(self.alias):
            return False
        for p, a, st in zip(params, self.alias, self.state):
            if (p.untyped_storage().data_ptr() != a.untyped_storage().data_ptr() or p.data_ptr() != a.data_ptr()
                    or (p._version, p.dtype, tuple(p.shape)) != st):
                return False
        return True


class LoRAMoE_CMix(nn.Module):
    """ChannelMix with top-k routed LoRA expert adapters on a frozen shared
    base (rwkv_mlx/moe.py:93-163)."""

    def __init__(self, base: nn.Module, n_experts: int, lora_rank: int, top_k: int = 2):
        super().__init__()
        self.base = base
        self.n_experts = n_experts
        self.lora_rank = lora_rank
        self.top_k = top_k
        C = base.key.weight.shape[1]
        r = lora_rank
        # A ~ N(0,1)·0.01, B = 0: the initial delta is zero (moe.py:121-125)
        self.lora_A = nn.Parameter(torch.randn(n_experts, C, r) * 0.01)
        self.lora_B = nn.Parameter(torch.zeros(n_experts, r, C))
        self.router = Router(C, n_experts, top_k)
        self.mode = "fused"
        self._prep = None       # lora_A / lora_B laid out by rwkvmoe_prepare_adapters
        self._prep_src = None   # what it was made from (_SourceKey)
        self._pbase = None      # base W_key / W_value laid out by rwkvmoe_prepare_base (decode steps)
        self._pbase_src = None

    def invalidate_prepared(self) -> None:
        """Drop the cached kernel layouts of lora_A / lora_B and of the base
        weights; the next forward remakes them.  Updates through a
        parameter (``p.add_(...)``, optimizer steps, ``p.data = t``,
        load_state_dict) are detected on their own; an in-place write through
        ``p.data`` (``p.data.add_(...)``) moves no version counter and needs
        this call.  checkpoint.load_moe_layer calls it."""
        self._prep = self._prep_src = None
        self._pbase = self._pbase_src = None

    def _prepared(self, A: torch.Tensor, Bm: torch.Tensor, dt: torch.dtype, flags: int) -> torch.Tensor:
        """The adapters in the layouts the forward's kernels read, made once by
        rwkvmoe_prepare_adapters and reused while lora_A and lora_B are
        unchanged (``_SourceKey``: same storages and version counters, same
        compute dtype and dtype flags)."""
        fl = flags & (_lib.GATE_F32 | _lib.ADAPTERS_F32)
        if self._prep is None or not self._prep_src.matches((self.lora_A, self.lora_B), (dt, fl, A.device)):
            E, C, r = A.shape
            desc = _lib.make_desc(1, 1, C, 64, E, 1, r, dt, _lib.MODE_FUSED, fl)
            buf = torch.empty(_lib.prepared_bytes(desc), dtype=torch.uint8, device=A.device)
            _lib.prepare_adapters(desc, A, Bm, buf, _lib.current_stream(A.device))
            self._prep, self._prep_src = buf, _SourceKey((self.lora_A, self.lora_B), (dt, fl, A.device))
        return self._prep

    def _prepared_base(self, wk: torch.Tensor, wv: torch.Tensor, dt: torch.dtype):
        """The frozen base weights in the fragment order the decode launches
        read (a FUSED forward of at most 64 tokens), made once by
        rwkvmoe_prepare_base and reused while base.key / base.value are
        unchanged (same rule as _prepared)."""
        src = (self.base.key.weight, self.base.value.weight)
        if self._pbase is None or not self._pbase_src.matches(src, (dt, wk.device)):
            F, C = wk.shape
            desc = _lib.make_desc(1, 1, C, F, 1, 1, 1, dt)
            buf = torch.empty(_lib.prepared_base_bytes(desc), dtype=torch.uint8, device=wk.device)
            _lib.prepare_base(desc, wk, wv, buf, _lib.current_stream(wk.device))
            self._pbase, self._pbase_src = buf, _SourceKey(src, (dt, wk.device))
        return self._pbase

    def _operands(self, x: torch.Tensor, differentiable: bool = False, uniform: bool = False):
        """The parameters in the dtypes of the dtype plan (``_dtype_plan``),
        or with `uniform` all in the promoted dtype.  With `differentiable`
        the trainable ones (gate, lora_A, lora_B) stay attached to autograd
        (the base is always detached: stop_gradient).  Returns (dt, flags,
        out_dt, [x_k, W_key, W_value, W_gate, lora_A, lora_B])."""
        base = self.base
        params = [base.x_k, base.key.weight, base.value.weight, self.router.gate.weight, self.lora_A, self.lora_B]
        dt, gdt, adt, flags, odt = _dtype_plan(x.dtype, [p.dtype for p in params[:3]], params[3].dtype,
                                               [params[4].dtype, params[5].dtype])
        if uniform:
            dt = gdt = adt = odt = _promote(x.dtype, *[p.dtype for p in params])
            flags = 0
        want = [dt, dt, dt, gdt, adt, adt]
        ops = [(p if differentiable and i >= 3 else p.detach()).to(device=x.device, dtype=want[i]).contiguous()
               for i, p in enumerate(params)]
        ops[0] = ops[0].reshape(-1)
        return dt, flags, odt, ops

    def forward(self, x: torch.Tensor, x_prev: torch.Tensor | None = None,
                residual: torch.Tensor | None = None, mode: str | None = None,
                extras: dict | None = None, ln=None):
        """(out, aux_loss, z_loss) = LoRAMoE_CMix(x) (moe.py:129-147).

        x_prev (B,C): token before x[:,0] (default: zeros, the reference's
        shift).  residual (B,T,C): returned out is residual + ffn_out.
        extras: if a dict is passed, it receives inds, gates and logits (and
        x_ln with `ln`).  ln: the Block's ln2 (an nn.LayerNorm or a (weight,
        bias) pair); x is then the residual stream and the layer runs on
        ln2(x) (model.py:321), with x_prev in ln2's output space (the RNN
        state of model.py:413-416).  For Block's x + ffn(ln2(x)) pass
        residual=x as well.  ln2 runs inside the layer's launches when x,
        ln2 and the layer's compute dtype agree (eps 1e-5), else in torch;
        under autograd the fused form's VJP is rwkvmoe_layer_norm_backward
        (gradients reach x, ln2.weight and ln2.bias; with residual=x the
        residual's cotangent is added there).
        The output's dtype is MLX's: promote(x, lora_A, lora_B) (fp32 for an
        fp16 layer with fp32 adapters)."""
        require_device(x, "LoRAMoE_CMix")
        if x.dim() != 3:
            raise ValueError(f"LoRAMoE_CMix expects (B, T, C), got {tuple(x.shape)}")
        B, T, C = x.shape
        lnp = _ln_params(ln) if ln is not None else None
        train = torch.is_grad_enabled() and extras is None and B * T > 0 and (
            x.requires_grad or self.lora_A.requires_grad or self.lora_B.requires_grad
            or self.router.gate.weight.requires_grad or (residual is not None and residual.requires_grad)
            or (lnp is not None and (lnp[0].requires_grad or lnp[1].requires_grad)))
        dt, pflags, odt, (xk, wk, wv, wg, A, Bm) = self._operands(x, differentiable=train)
        if train and pflags and dt != torch.float16:
            # (the fp16 layer's mixed forms have an fp32 VJP with fp16 gates; a bf16 layer
            # with an fp32 gate trains on the promoted dtype)
            dt, pflags, odt, (xk, wk, wv, wg, A, Bm) = self._operands(x, differentiable=True, uniform=True)
        lnw = lnb = None
        if ln is not None:
            lnw, lnb, eps = lnp
            if B * T == 0 or not _ln_fused_ok(x, lnw, lnb, eps, dt):
                # torch's ln2, then the layer (autograd records through both)
                xn = _ln_torch(x, lnw, lnb, eps)
                if extras is not None:
                    extras["x_ln"] = xn.detach()
                return self.forward(xn, x_prev, residual, mode, extras)
            # in the layer's launches; under autograd its VJP is rwkvmoe_layer_norm_backward
            lnw = lnw.to(device=x.device).contiguous()
            lnb = lnb.to(device=x.device).contiguous()
            if not train:
                lnw, lnb = lnw.detach(), lnb.detach()
        if B * T == 0:  # MLX: an empty output, and means over no tokens are NaN
            nan = torch.full((), float("nan"), dtype=torch.float32, device=x.device)
            out = torch.empty(B, T, C, dtype=odt, device=x.device)
            return (out if residual is None else residual.to(odt) + out), nan, nan.clone()
        F = wk.shape[0]
        E, k, r = self.n_experts, self.top_k, self.lora_rank
        if train:
            xp = x_prev.detach().to(device=x.device, dtype=dt).contiguous() if x_prev is not None else None
            bias = self.router.logit_bias
            if bias is not None:
                bias = bias.detach().to(device=x.device, dtype=torch.float32).contiguous()
            res = residual.to(dt).contiguous() if residual is not None else None
            out, losses = _LoRAMoEFunction.apply(x.to(dt).contiguous(), A, Bm, wg, xk, wk, wv, bias, xp, res,
                                                 (B, T, C, F, E, k, r, dt), mode or self.mode, pflags, odt, lnw, lnb,
                                                 residual is x)
            return out, losses[0], losses[1]
        x = x.to(dt).contiguous()
        flags = pflags | (_lib.LN_IN if lnw is not None else 0)
        xp = None
        if x_prev is not None:
            xp = x_prev.to(device=x.device, dtype=dt).contiguous()
            flags |= _lib.HAS_PREV
        bias = self.router.logit_bias
        if bias is not None:
            bias = bias.detach().to(device=x.device, dtype=torch.float32).contiguous()
            flags |= _lib.HAS_BIAS
        res = None
        if residual is not None:
            res = residual.to(dt).contiguous()  # in x's dtype; added to the output in out's dtype
            flags |= _lib.ADD_RESIDUAL
        desc = _lib.make_desc(B, T, C, F, E, k, r, dt, mode or self.mode, flags)
        nbytes = _lib.workspace_bytes(desc)
        ws = _WS.get(x.device, nbytes)
        out = torch.empty(B, T, C, dtype=odt, device=x.device)
        losses = torch.empty(2, dtype=torch.float32, device=x.device)
        kw = {}
        if extras is not None:
            kw = {"inds": torch.empty(B * T, k, dtype=torch.int32, device=x.device),
                  "gates": torch.empty(B * T, k, dtype=dt, device=x.device),
                  "logits": torch.empty(B * T, E, dtype=torch.float32, device=x.device)}
            if lnw is not None:
                kw["x_ln"] = torch.empty(B, T, C, dtype=dt, device=x.device)
        if lnw is not None:
            kw.update(ln_weight=lnw, ln_bias=lnb)
        prep = self._prepared(A, Bm, dt, flags)
        # decode-sized calls read the base weights in the decode launches' layout
        # (laid out only when this forward reads them)
        pbase = self._prepared_base(wk, wv, dt) if _lib.reads_prepared_base(desc) else None
        t = _lib.make_tensors(x=x, x_prev=xp, x_k=xk, w_key=wk, w_value=wv, w_gate=wg, lora_A=A, lora_B=Bm,
                              logit_bias=bias, residual=res, out=out, losses=losses, prepared=prep,
                              prepared_base=pbase, **kw)
        _lib.call("rwkvmoe_forward", desc, t, ws, nbytes, _lib.current_stream(x.device))
        if extras is not None:
            extras.update({n: v for n, v in kw.items() if n not in ("ln_weight", "ln_bias")})
        return out, losses[0], losses[1]

    def decode_step(self, x: torch.Tensor, x_prev: torch.Tensor, ln=None):
        """One RNN-mode token per sequence: x (B,C), x_prev (B,C).

        Returns (out (B,C), aux_loss, z_loss, new_state) with new_state = x
        (rwkv_mlx/model.py:498-506 form of the shift), or ln2(x) with `ln`
        (x is then the residual stream, model.py:413-416)."""
        if ln is None:
            out, aux, z = self.forward(x.unsqueeze(1), x_prev=x_prev)
            return out.squeeze(1), aux, z, x
        ex = {}
        out, aux, z = self.forward(x.unsqueeze(1), x_prev=x_prev, extras=ex, ln=ln)
        return out.squeeze(1), aux, z, ex["x_ln"].reshape(x.shape)

    def orthogonal_loss(self) -> torch.Tensor:
        """Σ_{i<j} ||A_iᵀ A_j||_F² (moe.py:149-163), fp32 scalar; differentiable
        with respect to lora_A when autograd is recording."""
        A = self.lora_A
        require_device(A, "orthogonal_loss")
        E, C, r = A.shape
        dt = A.dtype
        desc = _lib.make_desc(1, 1, C, 64, E, 1, r, dt)
        if torch.is_grad_enabled() and A.requires_grad:
            return _OrthoFunction.apply(A.contiguous(), desc)[0]
        A = A.detach().contiguous()
        nbytes = _lib.workspace_bytes(desc)
        ws = _WS.get(A.device, nbytes)
        out = torch.empty(1, dtype=torch.float32, device=A.device)
        t = _lib.make_tensors(lora_A=A, ortho_loss=out)
        _lib.call("rwkvmoe_ortho_loss", desc, t, ws, nbytes, _lib.current_stream(A.device))
        return out[0]


class _ExpertsFunction(torch.autograd.Function):
    """Autograd node of MoE_CMix: forward through rwkvmoe_experts_forward,
    VJP through rwkvmoe_experts_backward (moe.py:218-234; every parameter of
    the layer is trainable).  Gradients reach x, x_prev, x_k, expert_key,
    expert_val and router.gate.weight; a residual receives d_out."""

    @staticmethod
    def forward(ctx, x, xp, xk, wk, wv, wg, bias, res, dims, lnw=None, lnb=None, res_is_x=False):
        B, T, C, F, E, k, dt = dims
        N = B * T
        flags = (_lib.HAS_PREV if xp is not None else 0) | (_lib.HAS_BIAS if bias is not None else 0) | (
            _lib.ADD_RESIDUAL if res is not None else 0) | (_lib.LN_IN if lnw is not None else 0)
        desc = _lib.make_desc(B, T, C, F, E, k, 1, dt, _lib.MODE_FUSED, flags)
        nbytes = _lib.experts_workspace_bytes(desc)
        ws = _WS.get(x.device, nbytes)
        out = torch.empty_like(x)
        losses = torch.empty(2, dtype=torch.float32, device=x.device)
        logits = torch.empty(N, E, dtype=torch.float32, device=x.device)
        inds = torch.empty(N, k, dtype=torch.int32, device=x.device)
        lnkw = {}
        if lnw is not None:  # ln2 in the layer's launches; LN(x) kept as the VJP's layer input
            lnkw = dict(ln_weight=lnw.detach(), ln_bias=lnb.detach(), x_ln=torch.empty_like(x))
        t = _lib.make_tensors(x=x, x_prev=xp, x_k=xk, w_key=wk, w_value=wv, w_gate=wg, logit_bias=bias,
                              residual=res, out=out, losses=losses, logits=logits, inds=inds, **lnkw)
        _lib.call("rwkvmoe_experts_forward", desc, t, ws, nbytes, _lib.current_stream(x.device))
        xl = lnkw["x_ln"] if lnw is not None else x
        ctx.save_for_backward(xl, xp, xk, wk, wv, wg, logits, inds, x if lnw is not None else None, lnw)
        ctx.desc = _lib.make_desc(B, T, C, F, E, k, 1, dt, _lib.MODE_FUSED, flags & ~_lib.LN_IN)
        ctx.dims = (B, T, C, F, E, k, 1)
        ctx.has_res = res is not None
        ctx.ln = lnw is not None
        ctx.res_is_x = res_is_x and lnw is not None and res is not None
        return out, losses

    @staticmethod
    def backward(ctx, d_out, d_losses):
        x, xp, xk, wk, wv, wg, logits, inds, x0, lnw = ctx.saved_tensors
        need = ctx.needs_input_grad
        # x: the layer's input (LN(x0) with ln2); its cotangent feeds ln2's VJP
        need_ln = ctx.ln and (need[0] or need[9] or need[10])
        grads = {}
        for i, name, like in ((0, "d_x", x), (1, "d_x_prev", xp), (2, "d_x_k", xk), (3, "d_w_key", wk),
                              (4, "d_w_value", wv), (5, "d_w_gate", wg)):
            if (need[i] or (i == 0 and need_ln)) and like is not None:
                grads[name] = torch.empty_like(like)
        if d_out is None:
            d_out = torch.zeros_like(x)
        if grads:
            d_out = d_out.to(x.dtype).contiguous()
            dl = None if d_losses is None else d_losses.to(torch.float32).contiguous()
            nbytes = _lib.experts_backward_workspace_bytes(ctx.desc)
            ws = _WS.get(x.device, nbytes)
            _lib.experts_backward(ctx.desc, ws, nbytes, _lib.current_stream(x.device), x=x, x_prev=xp, x_k=xk,
                                  w_key=wk, w_value=wv, w_gate=wg, logits=logits, inds=inds, d_out=d_out,
                                  d_losses=dl, **grads)
        d_x = grads.get("d_x")
        d_lnw = d_lnb = None
        fuse_res = ctx.res_is_x and need[0]  # x + ffn(ln2(x)): d_out joins d_x inside ln2's VJP
        if need_ln:
            d_x, d_lnw, d_lnb = _ln_backward(x0, lnw, d_x, d_out if fuse_res else None, need[0], need[9], need[10],
                                             ctx.dims)
        d_res = d_out if ctx.has_res and need[7] and not fuse_res else None
        return (d_x, grads.get("d_x_prev"), grads.get("d_x_k"), grads.get("d_w_key"), grads.get("d_w_value"),
                grads.get("d_w_gate"), None, d_res, None, d_lnw, d_lnb, None)


class MoE_CMix(nn.Module):
    """Sparse MoE ChannelMix with E full experts and top-k routing
    (rwkv_mlx/moe.py:170-242).  Parameters as the reference:
    ``router.gate.weight (E,C)``, ``x_k (E,1,1,C)``, ``expert_key (E,F,C)``
    (orthogonal init scaled by sqrt(F/C)), ``expert_val (E,C,F)`` (zeros).

    The forward runs rwkvmoe_experts_forward, which computes only the routed
    (token, expert) rows and adds experts in ascending id as the reference's
    dense loop does (moe.py:223-234).  While autograd records, the call is one
    node whose VJP is rwkvmoe_experts_backward: gradients reach x, x_prev,
    x_k, expert_key, expert_val and router.gate.weight (every parameter of
    this layer is trainable), and a residual receives d_out.  A layer whose
    gate dtype differs from the rest trains on the promoted dtype."""

    def __init__(self, config: RWKVConfig, layer_id: int, n_experts: int, top_k: int = 2):
        super().__init__()
        self.n_experts = n_experts
        self.top_k = top_k
        C, D = config.n_embd, config.dim_ffn
        self.router = Router(C, n_experts, top_k)
        self.x_k = nn.Parameter(torch.zeros(n_experts, 1, 1, C))
        keys = []
        for _ in range(n_experts):
            flat = torch.randn(D, C)
            q, _ = torch.linalg.qr(flat if D >= C else flat.T)
            if D < C:
                q = q.T
            keys.append(q[:D, :C] * math.sqrt(D / C))
        self.expert_key = nn.Parameter(torch.stack(keys))
        self.expert_val = nn.Parameter(torch.zeros(n_experts, C, D))

    @torch.no_grad()
    def _forward_nograd(self, x, x_prev, residual, extras, ln):
        return self._run(x, x_prev, residual, extras, ln)

    def forward(self, x: torch.Tensor, x_prev: torch.Tensor | None = None,
                residual: torch.Tensor | None = None, extras: dict | None = None, ln=None):
        """(out, aux_loss, z_loss) = MoE_CMix(x) (moe.py:218-234).  ln: the
        Block's ln2, as for LoRAMoE_CMix.forward."""
        require_device(x, "MoE_CMix")
        if x.dim() != 3:
            raise ValueError(f"MoE_CMix expects (B, T, C), got {tuple(x.shape)}")
        B, T, C = x.shape
        lnp = _ln_params(ln) if ln is not None else None
        train = torch.is_grad_enabled() and extras is None and B * T > 0 and (
            x.requires_grad or any(p.requires_grad for p in self.parameters())
            or (x_prev is not None and x_prev.requires_grad)
            or (residual is not None and residual.requires_grad)
            or (lnp is not None and (lnp[0].requires_grad or lnp[1].requires_grad)))
        if not train:
            return self._forward_nograd(x, x_prev, residual, extras, ln)
        E, k = self.n_experts, self.top_k
        params = [self.x_k, self.expert_key, self.expert_val, self.router.gate.weight]
        dt = _promote(x.dtype, *[p.dtype for p in params])  # one dtype: the backward has no fp32-gate form
        lnw = lnb = None
        if lnp is not None:
            lnw, lnb, eps = lnp
            if not _ln_fused_ok(x, lnw, lnb, eps, dt):  # torch's ln2, then the layer (autograd records both)
                return self.forward(_ln_torch(x, lnw, lnb, eps), x_prev, residual)
            # in the layer's launches; its VJP is rwkvmoe_layer_norm_backward
            lnw, lnb = lnw.to(device=x.device).contiguous(), lnb.to(device=x.device).contiguous()
        xk, wk, wv, wg = [p.to(device=x.device, dtype=dt).contiguous() for p in params]
        xk = xk.reshape(E, C)
        F = wk.shape[1]
        xp = x_prev.to(device=x.device, dtype=dt).contiguous() if x_prev is not None else None
        bias = self.router.logit_bias
        if bias is not None:
            bias = bias.detach().to(device=x.device, dtype=torch.float32).contiguous()
        res = residual.to(dt).contiguous() if residual is not None else None
        out, losses = _ExpertsFunction.apply(x.to(dt).contiguous(), xp, xk, wk, wv, wg, bias, res,
                                             (B, T, C, F, E, k, dt), lnw, lnb, residual is x)
        return out, losses[0], losses[1]

    def _run(self, x, x_prev, residual, extras, ln=None):
        if x.dim() != 3:
            raise ValueError(f"MoE_CMix expects (B, T, C), got {tuple(x.shape)}")
        B, T, C = x.shape
        E, k = self.n_experts, self.top_k
        params = [self.x_k, self.expert_key, self.expert_val]
        dt = _promote(x.dtype, *[p.dtype for p in params])
        lnw = lnb = None
        if ln is not None:
            lnw, lnb, eps = _ln_params(ln)
            if B * T == 0 or not _ln_fused_ok(x, lnw, lnb, eps, dt):
                xn = _ln_torch(x, lnw, lnb, eps)
                if extras is not None:
                    extras["x_ln"] = xn
                return self._run(xn, x_prev, residual, extras)
            lnw = lnw.detach().to(device=x.device).contiguous()
            lnb = lnb.detach().to(device=x.device).contiguous()
        gdt, gflags = _gate_plan(dt, self.router.gate.weight.dtype)  # the gate as stored (moe.py:56)
        xk, wk, wv = [p.detach().to(device=x.device, dtype=dt).contiguous() for p in params]
        wg = self.router.gate.weight.detach().to(device=x.device, dtype=gdt).contiguous()
        xk = xk.reshape(E, C)
        F = wk.shape[1]
        if B * T == 0:
            nan = torch.full((), float("nan"), dtype=torch.float32, device=x.device)
            out = torch.empty(B, T, C, dtype=dt, device=x.device)
            return (out if residual is None else residual.to(dt) + out), nan, nan.clone()
        x = x.to(dt).contiguous()
        flags = gflags | (_lib.LN_IN if lnw is not None else 0)
        xp = None
        if x_prev is not None:
            xp = x_prev.to(device=x.device, dtype=dt).contiguous()
            flags |= _lib.HAS_PREV
        bias = self.router.logit_bias
        if bias is not None:
            bias = bias.detach().to(device=x.device, dtype=torch.float32).contiguous()
            flags |= _lib.HAS_BIAS
        res = None
        if residual is not None:
            res = residual.to(dt).contiguous()
            flags |= _lib.ADD_RESIDUAL
        desc = _lib.make_desc(B, T, C, F, E, k, 1, dt, _lib.MODE_FUSED, flags)
        nbytes = _lib.experts_workspace_bytes(desc)
        ws = _WS.get(x.device, nbytes)
        out = torch.empty_like(x)
        losses = torch.empty(2, dtype=torch.float32, device=x.device)
        kw = {}
        if extras is not None:
            kw = {"inds": torch.empty(B * T, k, dtype=torch.int32, device=x.device),
                  "gates": torch.empty(B * T, k, dtype=dt, device=x.device),
                  "logits": torch.empty(B * T, E, dtype=torch.float32, device=x.device)}
            if lnw is not None:
                kw["x_ln"] = torch.empty(B, T, C, dtype=dt, device=x.device)
        lnkw = dict(ln_weight=lnw, ln_bias=lnb) if lnw is not None else {}
        t = _lib.make_tensors(x=x, x_prev=xp, x_k=xk, w_key=wk, w_value=wv, w_gate=wg, logit_bias=bias,
                              residual=res, out=out, losses=losses, **kw, **lnkw)
        _lib.call("rwkvmoe_experts_forward", desc, t, ws, nbytes, _lib.current_stream(x.device))
        if extras is not None:
            extras.update(kw)
        return out, losses[0], losses[1]

    def orthogonal_loss(self) -> torch.Tensor:
        """No orthogonality loss for full experts (moe.py:240-242)."""
        return torch.zeros((), dtype=torch.float32, device=self.expert_key.device)


def channel_mixing_rnn(x: torch.Tensor, x_prev: torch.Tensor, ffn: nn.Module, ln=None):
    """One RNN-mode ChannelMix step (rwkv_mlx/model.py:498-506): returns
    ``(ffn(x) with the token shift taken from x_prev, x)``, the output and the
    next shift state.  With ``ln`` (the Block's ln2) x is the residual stream
    and the step is model.py:413-416's ``xx = ln2(x); xx, state =
    _channel_mixing_rnn(xx, state, ffn)``: the output and the next state
    ln2(x) (for a LoRA-MoE or MoE layer ln2 runs inside its launches).

    x and x_prev are one token, (C,) as the reference passes them, or one
    token for each of B sequences, (B, C).  ``ffn`` is an RWKV_CMix_x070
    (the reference's case), or a LoRAMoE_CMix / MoE_CMix, whose aux and z
    losses an inference step drops; model.py:498-506 reads ``ffn.x_k``,
    ``ffn.key`` and ``ffn.value``, which only the plain ChannelMix has.  A
    LoRA-MoE step of up to 64 sequences runs as two kernel launches (the
    router with the key product, then the value product with the adapter
    K-extension)."""
    if x.shape != x_prev.shape or x.dim() not in (1, 2):
        raise ValueError(f"channel_mixing_rnn expects x and x_prev of one shape, (C,) or (B, C); "
                         f"got {tuple(x.shape)} and {tuple(x_prev.shape)}")
    xb = x.reshape(-1, 1, x.shape[-1])
    pb = x_prev.reshape(-1, x.shape[-1])
    if isinstance(ffn, (LoRAMoE_CMix, MoE_CMix)):
        if ln is None:
            out = ffn(xb, x_prev=pb)[0]
            return out.reshape(x.shape), x
        ex = {}
        out = ffn(xb, x_prev=pb, extras=ex, ln=ln)[0]
        return out.reshape(x.shape), ex["x_ln"].reshape(x.shape)
    if isinstance(ffn, RWKV_CMix_x070):
        xs = x if ln is None else _ln_torch(x, *_ln_params(ln))
        out = ffn(xs.reshape(-1, 1, x.shape[-1]), x_prev=pb)
        return out.reshape(x.shape), xs
    raise TypeError(f"channel_mixing_rnn: unsupported ffn {type(ffn).__name__}")


def build_layer(C: int, F: int, E: int, k: int, r: int) -> LoRAMoE_CMix:
    """A LoRAMoE_CMix over a fresh base, as Block.__init__ builds it (model.py:292-305)."""
    cfg = RWKVConfig(n_embd=C, dim_ffn=F, moe_num_experts=E, moe_top_k=k, moe_lora_rank=r)
    return LoRAMoE_CMix(RWKV_CMix_x070(cfg, 0), E, r, k)
