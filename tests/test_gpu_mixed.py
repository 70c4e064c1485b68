"""GPU parity of the reference's fine-tune layer: an fp16 x and base
(convert.py writes fp16 weights) with the fp32 router gate and fp32 LoRA
adapters moe.py:47, 124-125 creates, called through the C ABI with
RWKVMOE_GATE_F32 | RWKVMOE_ADAPTERS_F32, against the oracle's MLX-promotion
mode (moe_oracle.moe_forward(..., gate_dtype="f32", adapter_dtype="f32"),
pinned by the Fraction fixture kat_f16base_f32adapters_e4_top2).

MLX runs that layer as: base in fp16 (model.py:259-263), logits from the fp32
gate as stored (moe.py:56), gates cast to fp16 (moe.py:86), and the adapter
products, the gate-weighted delta and out = base + delta in fp32
(moe.py:138-147).  Bars:
  * logits, top-k indices bit-exact; gates within one fp16 ulp;
  * the fp16 base within the fp16 bar (2e-2) of the oracle's: an fp16 GEMM's
    rounding depends on its accumulation order, which no implementation
    shares with another (MLX's included), so it is checked at fp16's bar;
  * the fp32 part at the fp32 bar (1e-5, max- and norm-relative): out against
    fp32(base_gpu + delta_oracle), i.e. the oracle's delta and sum on the
    GPU's own fp16 base and its own gates (already checked to one fp16 ulp:
    the softmax's exp differs from NumPy's in the last fp32 bit, which flips
    an fp16 rounding for about one token in four thousand);
  * the residual add in fp32 bit for bit.

The same layer on a bf16 base (bf16 x and base weights with the fp32 gate
and adapters LoRAMoE_CMix creates) has the same rounding points with bf16
for fp16 (the oracle's moe_forward(..., "bf16", gate_dtype="f32",
adapter_dtype="f32")); the library runs its delta as fp32 adapter rows
(SPARSE: the grouped LoRA in fp32 on fp32 copies of x) whatever the mode,
and the bars are the same with bf16's for fp16's (gates within 2^-7).
"""
from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest

from helpers import assert_close, rel_errs, to_dev, to_np
from oracle import moe_backward as MB
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5


def mixed_inputs(shape, bdt="f16"):
    """The workload's inputs with x and the base in bdt (fp16 or bf16) and
    W_gate, A, B in fp32 (the same draws, rounded to each tensor's dtype)."""
    from rwkv_mlx_amd.workloads import make_inputs
    g16 = make_inputs(replace(shape, dtype=bdt))
    g32 = make_inputs(replace(shape, dtype="f32"))
    g = dict(g16)
    for k in ("Wg", "A", "B"):
        g[k] = g32[k]
    return g


GATE_ULP = {"f16": 2.0 ** -10, "bf16": 2.0 ** -7}  # gates in (0, 1]: one step below 1 (two for fp16)


class Mixed:
    def __init__(self, shape, device, mode="fused", gate32=True, bdt="f16"):
        import torch
        from rwkv_mlx_amd import _lib
        from helpers import torch_dtype
        self.w = shape
        self.dev = device
        self.bdt = bdt
        self.tdt = torch_dtype(bdt)
        self.g = g = mixed_inputs(shape, bdt)
        self.gate32 = gate32
        h = lambda a: to_dev(a, bdt, device)
        f = lambda a: to_dev(a, "f32", device)
        self.x, self.x_k, self.Wk, self.Wv = h(g["x"]), h(g["x_k"]), h(g["Wk"]), h(g["Wv"])
        self.Wg = f(g["Wg"]) if gate32 else h(g["Wg"])
        self.A, self.B = f(g["A"]), f(g["B"])
        self.x_prev = h(g["x_prev"]) if "x_prev" in g else None
        self.bias = torch.from_numpy(g["bias"]).to(device) if "bias" in g else None
        self.flags = _lib.ADAPTERS_F32 | (_lib.GATE_F32 if gate32 else 0)
        if self.x_prev is not None:
            self.flags |= _lib.HAS_PREV
        if self.bias is not None:
            self.flags |= _lib.HAS_BIAS
        self.mode = mode
        self.N = shape.tokens

    def desc(self, flags):
        from rwkv_mlx_amd import _lib
        w = self.w
        return _lib.make_desc(w.batch, w.seq_len, w.d_model, w.d_ffn, w.n_experts, w.top_k, w.lora_rank, self.bdt,
                              self.mode, flags)

    def call(self, entry, flags, **tensors):
        import torch
        from rwkv_mlx_amd import _lib
        d = self.desc(flags)
        n = _lib.workspace_bytes(d)
        ws = torch.empty(n, dtype=torch.uint8, device=self.dev)
        _lib.call(entry, d, _lib.make_tensors(**tensors), ws, n, _lib.current_stream(self.dev))
        torch.cuda.synchronize()

    def forward(self, residual=None):
        import torch
        from rwkv_mlx_amd import _lib
        w = self.w
        out = torch.empty(self.N, w.d_model, dtype=torch.float32, device=self.dev)
        losses = torch.empty(2, dtype=torch.float32, device=self.dev)
        ex = dict(logits=torch.empty(self.N, w.n_experts, dtype=torch.float32, device=self.dev),
                  inds=torch.empty(self.N, w.top_k, dtype=torch.int32, device=self.dev),
                  gates=torch.empty(self.N, w.top_k, dtype=self.tdt, device=self.dev))
        if self.mode == "sparse":
            ex["base_out"] = torch.empty(self.N, w.d_model, dtype=self.tdt, device=self.dev)
        flags = self.flags | (_lib.ADD_RESIDUAL if residual is not None else 0)
        self.call("rwkvmoe_forward", flags, x=self.x, x_prev=self.x_prev, x_k=self.x_k, w_key=self.Wk,
                  w_value=self.Wv, w_gate=self.Wg, lora_A=self.A, lora_B=self.B, logit_bias=self.bias,
                  residual=residual, out=out, losses=losses, **ex)
        return out, losses, ex

    def base(self):
        """The 16-bit base through the stage entry points (the value product's
        plan and accumulation order are the forward's)."""
        import torch
        w = self.w
        hidden = torch.empty(self.N, w.d_ffn, dtype=self.tdt, device=self.dev)
        base = torch.empty(self.N, w.d_model, dtype=self.tdt, device=self.dev)
        fl = self.flags & ~0x18
        self.call("rwkvmoe_cmix_key", fl, x=self.x, x_prev=self.x_prev, x_k=self.x_k, w_key=self.Wk, hidden=hidden)
        self.call("rwkvmoe_cmix_value", fl, hidden=hidden, w_value=self.Wv, base_out=base)
        return base


def _shapes():
    from rwkv_mlx_amd.workloads import BY_NAME, HEADLINE
    return [
        ("headline-fused", HEADLINE, "fused", "f16"),       # router-fused adapters, 128x96 mixed value tiles
        ("headline-sparse", HEADLINE, "sparse", "f16"),
        ("1536tok-fused", HEADLINE.scaled(batch=3, seq_len=512), "fused", "f16"),  # split value plan: SPARSE
        ("decode64", BY_NAME["decode-d768-e8-top2-r16-fp16"], "fused", "f16"),     # 1-token router tiles: SPARSE
        ("skew-e32-top4", BY_NAME["skew-d1024-e32-top4-r16-fp16"].scaled(batch=2, seq_len=512), "fused", "f16"),
        # a bf16 base: fp32 adapter rows (SPARSE) in either mode
        ("bf16-headline-fused", HEADLINE, "fused", "bf16"),
        ("bf16-headline-sparse", HEADLINE, "sparse", "bf16"),
        ("bf16-decode64", BY_NAME["decode-d768-e8-top2-r16-fp16"], "fused", "bf16"),
        ("bf16-skew-e32-top4", BY_NAME["skew-d1024-e32-top4-r16-fp16"].scaled(batch=2, seq_len=512), "fused", "bf16"),
    ]


@pytest.mark.parametrize("name,shape,mode,bdt", _shapes(), ids=[s[0] for s in _shapes()])
def test_mixed_layer_matches_mlx_promotion(device, name, shape, mode, bdt):
    print(f"\n[mixed] {name} tokens={shape.tokens} mode={mode} base={bdt}", flush=True)
    L = Mixed(shape, device, mode, bdt=bdt)
    g = L.g
    w = shape
    C = w.d_model
    x2 = g["x"].reshape(L.N, C)
    out, losses, ex = L.forward()
    assert out.dtype.is_floating_point and out.element_size() == 4
    r = O.router(x2, g["Wg"], w.top_k, bdt, g.get("bias"), gate_dtype="f32")
    assert np.array_equal(to_np(ex["logits"]).view(np.uint32), r["logits"].view(np.uint32)), "logits"
    assert np.array_equal(ex["inds"].cpu().numpy(), r["inds"]), "top-k indices"
    assert np.max(np.abs(to_np(ex["gates"]) - r["gates"])) <= GATE_ULP[bdt]
    la = losses.cpu().numpy()
    assert abs(la[0] - r["aux"]) <= 1e-5 * abs(r["aux"]) and abs(la[1] - r["z"]) <= 1e-5 * abs(r["z"])

    base_gpu = to_np(ex["base_out"] if mode == "sparse" else L.base()).reshape(L.N, C)
    base_ref = O.cmix_base(g["x"], g["x_k"], g["Wk"], g["Wv"], bdt, g.get("x_prev")).reshape(L.N, C)
    assert_close(base_gpu, base_ref, bdt, f"{bdt} base")
    gates_gpu = to_np(ex["gates"])
    delta_ref = O.lora_delta_dense(x2, g["A"], g["B"], r["inds"], gates_gpu, "f32")
    got = to_np(out).reshape(L.N, C)
    ref = O.round_to(base_gpu + delta_ref, "f32")
    emax, enorm = rel_errs(got, ref)
    print(f"  fp32 part: max-rel {emax:.2e} norm-rel {enorm:.2e}", flush=True)
    assert emax <= F32_TOL and enorm <= F32_TOL, f"out vs fp32(base_gpu + delta): {emax:.3e} {enorm:.3e}"
    # against the oracle's whole output the gap is the fp16 base's rounding only
    full = O.round_to(base_ref + delta_ref, "f32")
    assert_close(got, full, bdt, "out vs oracle")
    # and the layer is not the all-one-dtype function: the delta kept fp32 precision
    d16 = O.lora_delta_dense(x2, O.round_to(g["A"], bdt), O.round_to(g["B"], bdt), r["inds"], r["gates"], bdt)
    assert np.max(np.abs(got - (base_gpu + d16))) > 10 * np.max(np.abs(got - ref))


@pytest.mark.parametrize("mode,bdt", [("fused", "f16"), ("sparse", "f16"), ("fused", "bf16")])
def test_mixed_residual_in_fp32(device, mode, bdt):
    """Block's x = x + ffn_out with a 16-bit residual stream and an fp32
    ffn_out is fp32 (model.py:321-322 under MLX promotion), bit for bit."""
    import torch
    from rwkv_mlx_amd.workloads import HEADLINE
    L = Mixed(HEADLINE.scaled(batch=2, seq_len=512), device, mode, bdt=bdt)
    res = torch.randn(L.N, L.w.d_model, device=device).to(L.tdt)
    out, _, _ = L.forward()
    out_r, _, _ = L.forward(residual=res)
    assert out_r.dtype == torch.float32
    assert torch.equal(out_r, res.float() + out)


def test_gate_f32_alone(device):
    """An fp32 gate with fp16 adapters: the router reads the fp32 gate; the
    delta stays fp16 (promote(fp16, fp16)) and so does out."""
    import torch
    from rwkv_mlx_amd import _lib
    from rwkv_mlx_amd.workloads import HEADLINE
    w = HEADLINE.scaled(batch=2, seq_len=256)
    g = mixed_inputs(w)
    h = lambda a: to_dev(a, "f16", device)
    A16, B16 = O.round_to(g["A"], "f16"), O.round_to(g["B"], "f16")
    N, C = w.tokens, w.d_model
    out = torch.empty(N, C, dtype=torch.float16, device=device)
    losses = torch.empty(2, dtype=torch.float32, device=device)
    inds = torch.empty(N, w.top_k, dtype=torch.int32, device=device)
    d = _lib.make_desc(w.batch, w.seq_len, C, w.d_ffn, w.n_experts, w.top_k, w.lora_rank, "f16", "fused",
                       _lib.GATE_F32)
    n = _lib.workspace_bytes(d)
    ws = torch.empty(n, dtype=torch.uint8, device=device)
    t = _lib.make_tensors(x=h(g["x"]), x_k=h(g["x_k"]), w_key=h(g["Wk"]), w_value=h(g["Wv"]),
                          w_gate=to_dev(g["Wg"], "f32", device), lora_A=h(A16), lora_B=h(B16), out=out,
                          losses=losses, inds=inds)
    _lib.call("rwkvmoe_forward", d, t, ws, n, _lib.current_stream(device))
    torch.cuda.synchronize()
    p = {**g, "A": A16, "B": B16}
    parts = O.moe_forward(g["x"], p, w.top_k, "f16", return_parts=True, gate_dtype="f32")
    assert np.array_equal(inds.cpu().numpy(), parts["inds"])
    assert_close(to_np(out).reshape(N, C), parts["out"].reshape(N, C), "f16", "gate-f32 layer")


def test_gate_f32_sparse_forms(device):
    """SPARSE with an fp32 gate and fp16 adapters at the D=768 layer's full
    size (4096 tokens), where the forward keeps the adapters on chip (the
    router's u, the value product's rank slices): the routing equals the
    oracle's, and the output matches the oracle and the grouped form (the
    same call with adapter rows asked for) at the fp16 tolerance."""
    import torch
    from rwkv_mlx_amd import _lib
    from rwkv_mlx_amd.workloads import HEADLINE
    w = HEADLINE
    print(f"\n[gate f32 sparse] {w.name}", flush=True)
    g = mixed_inputs(w)
    h = lambda a: to_dev(a, "f16", device)
    A16, B16 = O.round_to(g["A"], "f16"), O.round_to(g["B"], "f16")
    N, C = w.tokens, w.d_model
    d = _lib.make_desc(w.batch, w.seq_len, C, w.d_ffn, w.n_experts, w.top_k, w.lora_rank, "f16", "sparse",
                       _lib.GATE_F32)
    n = _lib.workspace_bytes(d)
    ws = torch.empty(n, dtype=torch.uint8, device=device)
    common = dict(x=h(g["x"]), x_k=h(g["x_k"]), w_key=h(g["Wk"]), w_value=h(g["Wv"]),
                  w_gate=to_dev(g["Wg"], "f32", device), lora_A=h(A16), lora_B=h(B16))
    outs = []
    for rows in (False, True):
        out = torch.empty(N, C, dtype=torch.float16, device=device)
        losses = torch.empty(2, dtype=torch.float32, device=device)
        inds = torch.empty(N, w.top_k, dtype=torch.int32, device=device)
        extra = {"adapter_rows": torch.empty(N * w.top_k, C, dtype=torch.float16, device=device)} if rows else {}
        t = _lib.make_tensors(out=out, losses=losses, inds=inds, **common, **extra)
        _lib.call("rwkvmoe_forward", d, t, ws, n, _lib.current_stream(device))
        torch.cuda.synchronize()
        outs.append((to_np(out).reshape(N, C), inds.cpu().numpy()))
    p = {**g, "A": A16, "B": B16}
    parts = O.moe_forward(g["x"], p, w.top_k, "f16", return_parts=True, gate_dtype="f32")
    for (o, ind), form in zip(outs, ("on chip", "grouped")):
        assert np.array_equal(ind, parts["inds"]), form
        assert_close(o, parts["out"].reshape(N, C), "f16", f"gate-f32 sparse {form}")
    assert_close(outs[0][0], outs[1][0], "f16", "gate-f32 sparse forms")


def test_module_fine_tune_layer(device):
    """LoRAMoE_CMix as build_moe_from_base leaves it: fp16 base, fp32
    lora_A / lora_B / router.gate (moe.py:47, 124-125; finetune_moe.py:75)."""
    import torch
    from rwkv_mlx_amd.moe import build_layer
    torch.manual_seed(3)
    C, F, E, k, r = 256, 512, 8, 2, 16
    m = build_layer(C, F, E, k, r).cuda()
    with torch.no_grad():
        m.base.x_k.uniform_(0, 1)
        m.lora_B.normal_(0, 0.02)
    m.base.half()  # the converted checkpoint's fp16 base; adapters and gate stay fp32
    assert m.lora_A.dtype == torch.float32 and m.router.gate.weight.dtype == torch.float32
    x = torch.randn(4, 256, C, device="cuda").half()
    with torch.no_grad():
        ex = {}
        out, aux, z = m(x, extras=ex)
    assert out.dtype == torch.float32
    f = lambda t: t.detach().float().cpu().numpy()
    p = {"x_k": f(m.base.x_k).reshape(-1), "Wk": f(m.base.key.weight), "Wv": f(m.base.value.weight),
         "Wg": f(m.router.gate.weight), "A": f(m.lora_A), "B": f(m.lora_B)}
    xr = f(x)
    parts = O.moe_forward(xr, p, k, "f16", return_parts=True, gate_dtype="f32", adapter_dtype="f32")
    assert np.array_equal(ex["inds"].cpu().numpy(), parts["inds"])
    assert abs(float(aux) - parts["aux"]) <= 1e-5 * abs(parts["aux"])
    assert abs(float(z) - parts["z"]) <= 1e-5 * abs(parts["z"])
    assert_close(f(out).reshape(-1, C), parts["out"].reshape(-1, C), "f16", "module out")
    # the fp32 part on the module's own base (the base alone through the fp16
    # ChannelMix) and its own gates (within one fp16 ulp of the oracle's)
    assert np.max(np.abs(f(ex["gates"]) - parts["gates"])) <= 2.0 ** -10
    with torch.no_grad():
        base = m.base(x)
    xr2 = xr.reshape(-1, C)
    delta = O.lora_delta_dense(xr2, p["A"], p["B"], parts["inds"], f(ex["gates"]), "f32")
    ref = O.round_to(f(base).reshape(-1, C) + delta, "f32")
    emax, enorm = rel_errs(f(out).reshape(-1, C), ref)
    assert emax <= F32_TOL and enorm <= F32_TOL, (emax, enorm)


def test_module_bf16_base_fp32_adapters(device):
    """LoRAMoE_CMix on a bf16 base with the fp32 adapters and gate it
    creates: the base in bf16, the delta and out in fp32 (MLX promotion),
    through the module's dtype plan (ADAPTERS_F32 on a bf16 layer) and its
    prepared-adapter cache, in both modes."""
    import torch
    from rwkv_mlx_amd.moe import build_layer
    torch.manual_seed(4)
    C, F, E, k, r = 256, 512, 8, 2, 16
    m = build_layer(C, F, E, k, r).cuda()
    with torch.no_grad():
        m.base.x_k.uniform_(0, 1)
        m.lora_B.normal_(0, 0.02)
    m.base.bfloat16()
    assert m.lora_A.dtype == torch.float32 and m.router.gate.weight.dtype == torch.float32
    x = torch.randn(4, 256, C, device="cuda").bfloat16()
    f = lambda t: t.detach().float().cpu().numpy()
    p = {"x_k": f(m.base.x_k).reshape(-1), "Wk": f(m.base.key.weight), "Wv": f(m.base.value.weight),
         "Wg": f(m.router.gate.weight), "A": f(m.lora_A), "B": f(m.lora_B)}
    xr = f(x)
    parts = O.moe_forward(xr, p, k, "bf16", return_parts=True, gate_dtype="f32", adapter_dtype="f32")
    with torch.no_grad():
        base = f(m.base(x)).reshape(-1, C)
    outs = []
    for mode in ("fused", "sparse"):
        with torch.no_grad():
            ex = {}
            out, aux, z = m(x, extras=ex, mode=mode)
        assert out.dtype == torch.float32
        assert np.array_equal(ex["inds"].cpu().numpy(), parts["inds"])
        assert abs(float(aux) - parts["aux"]) <= 1e-5 * abs(parts["aux"])
        assert_close(f(out).reshape(-1, C), parts["out"].reshape(-1, C), "bf16", f"module out ({mode})")
        assert np.max(np.abs(f(ex["gates"]) - parts["gates"])) <= GATE_ULP["bf16"]
        delta = O.lora_delta_dense(xr.reshape(-1, C), p["A"], p["B"], parts["inds"], f(ex["gates"]), "f32")
        emax, enorm = rel_errs(f(out).reshape(-1, C), O.round_to(base + delta, "f32"))
        assert emax <= F32_TOL and enorm <= F32_TOL, (mode, emax, enorm)
        outs.append(out)
    assert torch.equal(outs[0], outs[1])  # both modes run the fp32-rows form


def test_router_module_reads_fp32_gate(device):
    """Router with its default fp32 gate on fp16 x: logits from the gate as
    stored (moe.py:56), not from a gate rounded to fp16."""
    import torch
    from rwkv_mlx_amd.moe import Router
    torch.manual_seed(9)
    C, E, k = 512, 8, 2
    rt = Router(C, E, k).cuda()
    x = torch.randn(2, 300, C, device="cuda").half()
    with torch.no_grad():
        inds, gates, aux, z = rt(x)
    wg = rt.gate.weight.detach().float().cpu().numpy()
    ref = O.router(x.float().cpu().numpy().reshape(-1, C), wg, k, "f16", gate_dtype="f32")
    assert np.array_equal(inds.cpu().numpy().reshape(-1, k), ref["inds"])
    assert gates.dtype == torch.float16
    assert abs(float(aux) - ref["aux"]) <= 1e-5 * abs(ref["aux"]) and abs(float(z) - ref["z"]) <= 1e-5 * abs(ref["z"])
    # under autograd (the gate requires grad) the call trains on the promoted
    # dtype, fp32 (the backward has one element type); gates still come back
    # in x's dtype, and the gate's gradient matches the float64 VJP of the fp32
    # router on x converted to fp32 (exact)
    inds2, gates2, aux2, z2 = rt(x)
    assert gates2.dtype == torch.float16 and gates2.requires_grad
    (gates2.float().sum() + 0.5 * aux2 + 0.25 * z2).backward()
    ref2 = MB.router_backward(x.float().cpu().numpy().reshape(-1, C), wg, k, "f32",
                              np.ones((x.shape[0] * x.shape[1], k)), 0.5, 0.25)
    assert np.array_equal(inds2.cpu().numpy().reshape(-1, k), ref2["inds"])
    emax, enorm = rel_errs(rt.gate.weight.grad.cpu().numpy(), ref2["dWg"])
    assert emax <= 1e-4 and enorm <= 1e-4, (emax, enorm)


def test_module_fine_tune_layer_training(device):
    """Training the fine-tune layer (fp16 x and base, fp32 gate and adapters):
    the forward under autograd is the MLX-promoted one (fp32 out, the same
    values as without autograd), and the gradients of lora_A, lora_B and the
    gate (fp32) match the float64 VJP of that layer (gates rounded to fp16,
    s_e and a_e in fp32: moe_backward(..., gate_dtype="f32",
    adapter_dtype="f32")) at the fp32 bar; dx (fp16, x's dtype) at the fp16
    bar.  Only the adapters and gate are trained: the base is under
    stop_gradient (moe.py:131)."""
    import torch
    from rwkv_mlx_amd.moe import build_layer
    torch.manual_seed(5)
    C, F, E, k, r = 256, 512, 8, 2, 16
    m = build_layer(C, F, E, k, r).cuda()
    with torch.no_grad():
        m.base.x_k.uniform_(0, 1)
        m.lora_B.normal_(0, 0.02)
    m.base.half()
    m.base.requires_grad_(False)
    x = torch.randn(2, 128, C, device="cuda").half().requires_grad_(True)
    dO = torch.randn(2, 128, C, device="cuda", dtype=torch.float32)
    out, aux, z = m(x)
    assert out.dtype == torch.float32
    with torch.no_grad():
        out0, aux0, z0 = m(x)
    assert torch.equal(out.detach(), out0)
    d_aux, d_z = 0.01, 0.001
    ((out * dO).sum() + d_aux * aux + d_z * z).backward()
    f = lambda t: t.detach().float().cpu().numpy()
    N = 2 * 128
    ref = MB.moe_backward(f(x).reshape(N, C), f(m.router.gate.weight), f(m.lora_A), f(m.lora_B), k, "f16",
                          f(dO).reshape(N, C), d_aux, d_z, gate_dtype="f32", adapter_dtype="f32")
    for name, got, tol in (("dA", m.lora_A.grad, F32_TOL), ("dB", m.lora_B.grad, F32_TOL),
                           ("dWg", m.router.gate.weight.grad, F32_TOL), ("dx", x.grad, 2e-2)):
        assert got is not None and got.dtype == (torch.float16 if name == "dx" else torch.float32), name
        emax, enorm = rel_errs(f(got).reshape(ref[name].shape), ref[name])
        assert emax <= tol and enorm <= tol, f"{name}: max-rel {emax:.3e} norm-rel {enorm:.3e}"
    assert m.base.key.weight.grad is None
