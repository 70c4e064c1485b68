"""The decode path: a FUSED forward of at most 64 tokens (one RNN-mode step
of up to 64 sequences, or a few short sequences) runs as two launches, the
decode front (the router, key tiles computing relu(xk·W_keyᵀ)² with the
token shift, adapter tiles computing x·A_allᵀ) and the decode value launch
(h·W_valueᵀ plus the gated adapter K-extension, K split over the 16 waves of
a workgroup and summed in a fixed order, plus the loss reduction).

Checks, through the C ABI against the oracle: router logits, indices, dense
gates and the dispatch bit-exact, the output within the dtype's tolerance,
the losses within 1e-5, on token counts 1 to 64, fp16 and bf16, an fp32
router gate, a logit bias, the residual add and multi-token sequences (the
shift inside a sequence); the base weights laid out by rwkvmoe_prepare_base
give the same bits as the weights as stored; repeated calls on one workspace
with changing token counts match fresh workspaces bit for bit; and 16
successive RNN steps with a carried shift state against the 16-token
forward (rwkv_mlx/model.py:498-506 against model.py:258-263)."""
from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest

from helpers import Layer, assert_close, oracle_rows, to_dev, to_np
from oracle import moe_oracle as O
from rwkv_mlx_amd.workloads import LayerShape, make_inputs

pytestmark = pytest.mark.gpu

D768 = dict(d_model=768, d_ffn=3072, n_experts=8, top_k=2, lora_rank=16)


def _shape(name, dtype, batch, seq_len, decode=True, seed=8000, **kw):
    dims = dict(D768)
    dims.update(kw)
    return LayerShape(name, dtype, batch, seq_len, dims["d_model"], dims["d_ffn"], dims["n_experts"], dims["top_k"],
                      dims["lora_rank"], decode=decode, seed=seed)


CASES = [
    _shape("n1-f16", "f16", 1, 1, seed=8001),
    _shape("n5-f16", "f16", 5, 1, seed=8002),
    _shape("n16-bf16", "bf16", 16, 1, seed=8003),
    _shape("n17-f16", "f16", 17, 1, seed=8004),
    _shape("n64-bf16", "bf16", 64, 1, seed=8005),
    # E·r = 128 at E = 16, a wider d_model and a ragged last router block
    _shape("n33-c1024-e16-r8-f16", "f16", 33, 1, seed=8006, d_model=1024, d_ffn=2048, n_experts=16, top_k=3,
           lora_rank=8),
    # 12 sequences of 4 tokens, no carried state: the shift inside a sequence
    _shape("b12-t4-f16", "f16", 12, 4, decode=False, seed=8007),
    # the smallest layer: C = F = 64, one expert, rank 1
    _shape("n3-c64-e1-r1-bf16", "bf16", 3, 1, seed=8008, d_model=64, d_ffn=64, n_experts=1, top_k=1, lora_rank=1),
]


def _layer(shape, device, gate32=False, bias=False):
    g = make_inputs(shape)
    if gate32:
        g["Wg"] = make_inputs(replace(shape, dtype="f32"))["Wg"]
    if bias:
        g["bias"] = np.random.default_rng(shape.seed).normal(0, 0.5, shape.n_experts).astype(np.float32)
    L = Layer(shape, device, inputs=g)
    if gate32:
        from rwkv_mlx_amd import _lib
        L.Wg = to_dev(g["Wg"], "f32", device)
        L.flags |= _lib.GATE_F32
    if bias and L.bias is None:
        import torch
        from rwkv_mlx_amd import _lib
        L.bias = torch.from_numpy(g["bias"]).to(device)
        L.flags |= _lib.HAS_BIAS
    L.desc = L.make_desc()
    L.router_ref = O.router(g["x"].reshape(L.N, -1), g["Wg"], shape.top_k, shape.dtype, g.get("bias"),
                            gate_dtype="f32" if gate32 else None)
    L.ref = oracle_rows(g, shape, np.arange(L.N), L.router_ref)
    return L


def _check(L, out, losses, ex, what, residual=None):
    base_ref, delta_ref, out_ref, r = L.ref
    ref = out_ref if residual is None else O.round_to(out_ref + to_np(residual).reshape(L.N, -1), L.w.dtype)
    assert_close(to_np(out).reshape(L.N, -1), ref, L.w.dtype, what)
    lg = ex["logits"].cpu().numpy()
    assert np.array_equal(lg.view(np.uint32), r["logits"].astype(np.float32).view(np.uint32)), what
    assert np.array_equal(ex["inds"].cpu().numpy(), r["inds"]), what
    assert np.array_equal(to_np(ex["gates"]), np.asarray(r["gates"], np.float32)), what
    p, i, o = O.dispatch(r["inds"], L.w.n_experts)
    assert np.array_equal(ex["perm"].cpu().numpy(), p), what
    assert np.array_equal(ex["inv_perm"].cpu().numpy(), i), what
    assert np.array_equal(ex["offsets"].cpu().numpy(), o), what
    l = losses.cpu().numpy()
    assert abs(l[0] - r["aux"]) <= 1e-5 * abs(r["aux"]) + 1e-7, what
    assert abs(l[1] - r["z"]) <= 1e-5 * abs(r["z"]) + 1e-7, what


@pytest.mark.parametrize("shape", CASES, ids=[c.name for c in CASES])
def test_decode_path_matches_oracle(device, shape):
    print(f"\n[decode] {shape.name}", flush=True)
    L = _layer(shape, device)
    entry = "rwkvmoe_decode" if shape.decode else "rwkvmoe_forward"
    out, losses, ex = L.forward(extras=True, entry=entry)
    _check(L, out, losses, ex, shape.name)


@pytest.mark.parametrize("shape", CASES, ids=[c.name for c in CASES])
def test_prepared_base_is_bit_identical(device, shape):
    """W_key / W_value read in fragment order from rwkvmoe_prepare_base's
    buffer give the same bits as reading them as stored."""
    import torch
    from rwkv_mlx_amd import _lib
    print(f"\n[decode prepared base] {shape.name}", flush=True)
    L = _layer(shape, device)
    pb = torch.empty(_lib.prepared_base_bytes(L.desc), dtype=torch.uint8, device=device)
    assert pb.numel() == 2 * shape.d_model * shape.d_ffn * 2
    stream = _lib.current_stream(device)
    _lib.prepare_base(L.desc, L.Wk, L.Wv, pb, stream)
    entry = "rwkvmoe_decode" if shape.decode else "rwkvmoe_forward"
    res = []
    for use in (None, pb):
        out = torch.empty_like(L.x)
        losses = torch.empty(2, dtype=torch.float32, device=device)
        L.call(entry, out=out, losses=losses, prepared_base=use, **L.inputs())
        torch.cuda.synchronize()
        res.append((to_np(out), losses.cpu().numpy()))
    assert np.array_equal(res[0][0], res[1][0]) and np.array_equal(res[0][1], res[1][1])


def test_module_base_cache_follows_updates(device):
    """The module lays the base out once for decode-sized calls and again
    after an in-place update of base.value."""
    import torch
    from rwkv_mlx_amd.moe import build_layer
    torch.manual_seed(6)
    m = build_layer(256, 512, 8, 2, 16).cuda().half()
    with torch.no_grad():
        m.base.x_k.uniform_(0, 1)
        m.base.value.weight.normal_(0, 0.05)
        m.lora_B.normal_(0, 0.02)
    x = torch.randn(12, 1, 256, device="cuda").half()
    xp = torch.randn(12, 256, device="cuda").half()
    with torch.no_grad():
        a, _, _ = m(x, x_prev=xp)
        src = m._pbase_src
        assert src is not None
        b, _, _ = m(x, x_prev=xp)
        assert m._pbase_src is src and torch.equal(a, b)
        m.base.value.weight.mul_(-2.0)
        c, _, _ = m(x, x_prev=xp)
        assert m._pbase_src is not src
        fresh = build_layer(256, 512, 8, 2, 16).cuda().half()
        fresh.load_state_dict(m.state_dict())
        d, _, _ = fresh(x, x_prev=xp)
    assert torch.equal(c, d) and not torch.equal(a, c)


@pytest.mark.parametrize("gate32,bias,resid", [(True, False, False), (False, True, True), (True, True, True)],
                         ids=["gate32", "bias-resid", "gate32-bias-resid"])
def test_decode_path_options(device, gate32, bias, resid):
    import torch
    shape = _shape("n40-f16", "f16", 40, 1, seed=8010)
    print(f"\n[decode options] gate32={gate32} bias={bias} residual={resid}", flush=True)
    L = _layer(shape, device, gate32=gate32, bias=bias)
    residual = None
    if resid:
        residual = to_dev(np.random.default_rng(5).normal(0, 1, (L.N, shape.d_model)), "f16", device)
        residual = residual.reshape(shape.batch, 1, shape.d_model)
    out, losses, ex = L.forward(extras=True, residual=residual, entry="rwkvmoe_decode")
    _check(L, out, losses, ex, f"gate32={gate32} bias={bias}", residual=residual)
    if resid:
        # the residual is added to the rounded output: round(residual + out), bit for bit
        plain, _, _ = L.forward(entry="rwkvmoe_decode")
        assert torch.equal(out, (residual.float() + plain.float()).to(out.dtype))


def test_repeated_calls_share_one_workspace(device):
    """Calls at 64, 5, 64 and 1 tokens on one workspace (sized for 64):
    every call's output equals a call on a fresh workspace, bit for bit."""
    import torch
    from rwkv_mlx_amd import _lib
    big = _layer(_shape("n64-f16", "f16", 64, 1, seed=8020), device)
    small = _layer(_shape("n5-f16", "f16", 5, 1, seed=8021), device)
    one = _layer(_shape("n1-f16", "f16", 1, 1, seed=8022), device)
    ws_bytes = _lib.workspace_bytes(big.desc)
    assert ws_bytes >= max(_lib.workspace_bytes(small.desc), _lib.workspace_bytes(one.desc))
    shared = torch.empty(ws_bytes, dtype=torch.uint8, device=device)

    def run(L, ws):
        out = torch.empty_like(L.x)
        losses = torch.empty(2, dtype=torch.float32, device=device)
        t = _lib.make_tensors(out=out, losses=losses, **L.inputs())
        _lib.call("rwkvmoe_decode", L.desc, t, ws, ws.numel(), _lib.current_stream(device))
        torch.cuda.synchronize()
        return to_np(out), losses.cpu().numpy()

    fresh = {id(L): run(L, torch.zeros(_lib.workspace_bytes(L.desc), dtype=torch.uint8, device=device))
             for L in (big, small, one)}
    for L in (big, small, big, one, big):
        got = run(L, shared)
        ref = fresh[id(L)]
        assert np.array_equal(got[0], ref[0]) and np.array_equal(got[1], ref[1]), L.w.name
    _, _, out_ref, _ = big.ref
    assert_close(run(big, shared)[0].reshape(big.N, -1), out_ref, "f16", "n64 after reuse")


def test_rnn_steps_match_sequence_forward(device):
    """16 RNN steps of 8 sequences (channel_mixing_rnn, state carried) against
    the forward of the 16-token sequences: indices bit-exact, every step's
    output within 2e-2 of the forward's, and the final state equal to the
    last token."""
    import torch
    from rwkv_mlx_amd import channel_mixing_rnn
    from rwkv_mlx_amd.moe import build_layer
    torch.manual_seed(3)
    m = build_layer(768, 3072, 8, 2, 16).cuda().half()
    with torch.no_grad():
        m.base.x_k.uniform_(0, 1)
        m.lora_B.normal_(0, 0.02)
        m.base.value.weight.normal_(0, 0.02)
    B, T = 8, 16
    x = torch.randn(B, T, 768, device="cuda").half()
    with torch.no_grad():
        ex = {}
        full, _, _ = m(x, extras=ex)          # 128 tokens: the many-token kernels
        inds_full = ex["inds"].reshape(B, T, -1)
        state = torch.zeros(B, 768, device="cuda", dtype=torch.half)
        for t in range(T):
            exs = {}
            m(x[:, t:t + 1], x_prev=state, extras=exs)
            assert torch.equal(exs["inds"].reshape(B, -1), inds_full[:, t]), f"step {t}: routing differs"
            out, state = channel_mixing_rnn(x[:, t], state, m)
            assert out.shape == (B, 768)
            assert_close(to_np(out), to_np(full[:, t]), "f16", f"step {t}")
        assert torch.equal(state, x[:, -1])


def test_rnn_step_single_token_plain_cmix(device):
    """The reference's form: one (C,) token through a plain ChannelMix, against
    the oracle's RNN-mode ChannelMix."""
    import torch
    from rwkv_mlx_amd import RWKV_CMix_x070, RWKVConfig, channel_mixing_rnn
    torch.manual_seed(4)
    ffn = RWKV_CMix_x070(RWKVConfig(n_embd=256, dim_ffn=1024)).cuda().half()
    with torch.no_grad():
        ffn.x_k.uniform_(0, 1)
    x = torch.randn(256, device="cuda").half()
    xp = torch.randn(256, device="cuda").half()
    with torch.no_grad():
        out, st = channel_mixing_rnn(x, xp, ffn)
    ref = O.cmix_decode(to_np(x)[None], to_np(xp)[None], to_np(ffn.x_k).reshape(-1), to_np(ffn.key.weight),
                        to_np(ffn.value.weight), "f16")[0]
    assert out.shape == (256,) and torch.equal(st, x)
    assert_close(to_np(out)[None], ref, "f16", "plain cmix rnn step")
