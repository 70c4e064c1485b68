"""GPU parity of ln2 in front of the layer (RWKVMOE_LN_IN: x is the Block's
residual stream, the layer runs on LN(x), model.py:321 / 413-416).

* x_ln (the LN output the forward writes) equals the oracle's layer_norm bit
  for bit; routing on it is bit-exact and the output is within the dtype
  tolerance of the oracle forward on LN(x) (1e-5 fp32, 2e-2 fp16 / bf16).
* The forward with the flag gives the same bits as the forward without it
  on the x_ln it wrote (FUSED, SPARSE, the two-launch decode and the
  full-expert layer), and with residual = x it is round(x + ffn(LN(x))).
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import Layer, assert_close, oracle_rows, sample_rows, to_dev, to_np
from oracle import moe_oracle as O
from rwkv_mlx_amd.workloads import BY_NAME, LayerShape

pytestmark = pytest.mark.gpu

CASES = [
    LayerShape("ln-c128-e4-k2-r8-f32", "f32", 2, 40, 128, 256, 4, 2, 8, seed=9401),
    LayerShape("ln-c256-e8-k2-r16-f16", "f16", 2, 48, 256, 512, 8, 2, 16, seed=9402),
    LayerShape("ln-c192-e5-k3-r3-bf16", "bf16", 3, 21, 192, 320, 5, 3, 3, seed=9403),
    BY_NAME["cmix-d768-e8-top2-r16-fp16"],
    BY_NAME["decode-d768-e8-top2-r16-fp16"],
]


def _stream(L, seed):
    """A residual stream (before ln2) and ln2's parameters, in the layer dtype."""
    rng = np.random.default_rng(seed)
    g, d, C = L.np, L.w.dtype, L.w.d_model
    N = L.N
    raw = O.round_to(g["x"].reshape(N, C) * 1.7 + 0.3 + rng.standard_normal((N, 1)), d)
    w = O.round_to(1.0 + 0.1 * rng.standard_normal(C), d)
    b = O.round_to(0.05 * rng.standard_normal(C), d)
    return raw, w, b


def _run(L, entry, desc, x, **kw):
    import torch
    w = L.w
    out = torch.empty_like(L.x)
    losses = torch.empty(2, dtype=torch.float32, device=L.dev)
    inds = torch.empty(L.N, w.top_k, dtype=torch.int32, device=L.dev)
    ins = L.inputs()
    ins["x"] = x
    L.call(entry, desc, out=out, losses=losses, inds=inds, **ins, **kw)
    torch.cuda.synchronize()
    return out, losses, inds


@pytest.mark.parametrize("mode", ["fused", "sparse"])
@pytest.mark.parametrize("shape", CASES, ids=lambda s: s.name)
def test_forward_with_ln(device, shape, mode):
    import torch
    from rwkv_mlx_amd import _lib
    if shape.decode and mode == "sparse":
        pytest.skip("the decode workload runs FUSED")
    print(f"\n[ln case] {shape.name} {mode}", flush=True)
    L = Layer(shape, device)
    d, N, C = shape.dtype, L.N, shape.d_model
    raw, w, b = _stream(L, shape.seed + 7)
    x_raw, lw, lb = to_dev(raw, d, device), to_dev(w, d, device), to_dev(b, d, device)
    xln = torch.empty_like(x_raw)
    desc = L.make_desc(mode=mode, flags=L.flags | _lib.LN_IN)
    entry = "rwkvmoe_decode" if shape.decode else "rwkvmoe_forward"
    out, losses, inds = _run(L, entry, desc, x_raw, ln_weight=lw, ln_bias=lb, x_ln=xln)
    # LN(x) itself
    ref_ln = O.layer_norm(raw, w, b, d)
    got_ln = to_np(xln).reshape(N, C)
    assert np.array_equal(got_ln, ref_ln), f"x_ln: {np.sum(got_ln != ref_ln)} elements differ"
    # the layer on LN(x): routing and output against the oracle
    g2 = dict(L.np, x=ref_ln.reshape(L.np["x"].shape))
    rt = O.router(ref_ln, g2["Wg"], shape.top_k, d, g2.get("bias"))
    assert np.array_equal(inds.cpu().numpy(), rt["inds"])
    rows = np.arange(N) if N <= 1024 else sample_rows(N, shape.seq_len, n=192)
    _, _, ref, _ = oracle_rows(g2, shape, rows, rt)
    assert_close(to_np(out).reshape(N, C)[rows], ref, d, shape.name)
    # the same bits as the forward without the flag on the x_ln it wrote
    out0, losses0, inds0 = _run(L, entry, L.make_desc(mode=mode), xln)
    assert torch.equal(out, out0) and torch.equal(inds, inds0) and torch.equal(losses, losses0)
    # Block: x + ffn(ln2(x))
    desc_r = L.make_desc(mode=mode, flags=L.flags | _lib.LN_IN | _lib.ADD_RESIDUAL)
    out_r, _, _ = _run(L, entry, desc_r, x_raw, ln_weight=lw, ln_bias=lb, residual=x_raw)
    assert torch.equal(out_r, (x_raw.float().reshape(out.shape) + out.float()).to(L.dt))


@pytest.mark.parametrize("shape", [CASES[1], CASES[2]], ids=lambda s: s.name)
def test_experts_forward_with_ln(device, shape):
    """The full-expert layer (rwkvmoe_experts_forward) with ln2 in front."""
    import torch
    from rwkv_mlx_amd import _lib
    print(f"\n[ln experts case] {shape.name}", flush=True)
    L = Layer(shape, device)
    d, N, C, F, E = shape.dtype, L.N, shape.d_model, shape.d_ffn, shape.n_experts
    rng = np.random.default_rng(shape.seed + 11)
    x_k = to_dev(rng.uniform(0, 1, (E, C)), d, device)
    Wk = to_dev(rng.standard_normal((E, F, C)) / np.sqrt(C), d, device)
    Wv = to_dev(rng.standard_normal((E, C, F)) / np.sqrt(F), d, device)
    raw, w, b = _stream(L, shape.seed + 13)
    x_raw, lw, lb = to_dev(raw, d, device), to_dev(w, d, device), to_dev(b, d, device)
    xln = torch.empty_like(x_raw)

    def run(x, flags, **kw):
        desc = _lib.make_desc(shape.batch, shape.seq_len, C, F, E, shape.top_k, 1, d, "fused", flags)
        nbytes = _lib.experts_workspace_bytes(desc)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
        out = torch.empty_like(L.x)
        losses = torch.empty(2, dtype=torch.float32, device=device)
        inds = torch.empty(N, shape.top_k, dtype=torch.int32, device=device)
        t = _lib.make_tensors(x=x, x_prev=L.x_prev, x_k=x_k, w_key=Wk, w_value=Wv, w_gate=L.Wg, logit_bias=L.bias,
                              out=out, losses=losses, inds=inds, **kw)
        _lib.call("rwkvmoe_experts_forward", desc, t, ws, nbytes, _lib.current_stream(device))
        torch.cuda.synchronize()
        return out, losses, inds

    out, losses, inds = run(x_raw, L.flags | _lib.LN_IN, ln_weight=lw, ln_bias=lb, x_ln=xln)
    assert np.array_equal(to_np(xln).reshape(N, C), O.layer_norm(raw, w, b, d))
    out0, losses0, inds0 = run(xln, L.flags)
    assert torch.equal(out, out0) and torch.equal(inds, inds0) and torch.equal(losses, losses0)


def test_module_ln(device):
    """LoRAMoE_CMix.forward(x, ln=ln2) and channel_mixing_rnn(..., ln=ln2):
    the layer's own LN(x) (extras["x_ln"]) is the oracle's bit for bit, the
    call equals the call on that x_ln, RNN steps from a zero state track the
    sequence forward and end in the state ln2(x[:, -1]), and under autograd
    ln2 runs in torch with gradients reaching x and ln2's parameters."""
    import torch
    from torch import nn
    from rwkv_mlx_amd.moe import build_layer, channel_mixing_rnn
    torch.manual_seed(0)
    C, T = 256, 12
    ffn = build_layer(C, 512, 8, 2, 16).to(device).half()
    ln = nn.LayerNorm(C).to(device).half()
    with torch.no_grad():
        ffn.lora_B.normal_(0.0, 0.05)
        ln.weight.normal_(1.0, 0.1)
        ln.bias.normal_(0.0, 0.05)
    x = (torch.randn(2, T, C, device=device) * 2 + 0.3).half()
    with torch.no_grad():
        ex = {}
        out, aux, z = ffn(x, ln=ln, extras=ex, residual=x)
        xl = ex["x_ln"]
        ref = O.layer_norm(to_np(x).reshape(-1, C), to_np(ln.weight), to_np(ln.bias), "f16")
        assert np.array_equal(to_np(xl).reshape(-1, C), ref)
        out0, aux0, z0 = ffn(xl, extras={}, residual=x)
        assert torch.equal(out, out0) and torch.equal(aux, aux0) and torch.equal(z, z0)
        seq, _, _ = ffn(x, ln=ln)
        state = torch.zeros(2, C, device=device, dtype=torch.float16)
        steps = []
        for t in range(T):
            o, state = channel_mixing_rnn(x[:, t], state, ffn, ln=ln)
            steps.append(o)
        assert_close(to_np(torch.stack(steps, 1)), to_np(seq), "f16", "rnn steps vs sequence")
        assert torch.equal(state, xl[:, -1])
    x2 = x.clone().requires_grad_(True)
    out, aux, z = ffn(x2, ln=ln)
    (out.float().square().mean() + aux + z).backward()
    assert x2.grad is not None and torch.isfinite(x2.grad.float()).all()
    assert ln.weight.grad is not None and torch.isfinite(ln.weight.grad.float()).all()
