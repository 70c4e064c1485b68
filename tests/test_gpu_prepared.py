"""Prepared adapters (rwkvmoe_prepare_adapters + rwkvmoe_tensors.prepared):
the forward reading lora_A / lora_B from a prepared buffer is bit-identical
to the forward that lays them out itself, on every path that reads them (the
router's fused adapter product, the key GEMM's adapter tiles, the SPARSE
grouped LoRA, the value GEMM's K-extension, fp32 adapters as fp16 pairs), and
the module's cache of the buffer follows in-place updates of the adapters."""
from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest

from helpers import Layer, to_dev

pytestmark = pytest.mark.gpu


def _cases():
    from rwkv_mlx_amd.workloads import BY_NAME, HEADLINE
    return [
        ("headline-fused", HEADLINE, "fused", 0),
        ("headline-sparse", HEADLINE, "sparse", 0),
        ("decode64-keyad", BY_NAME["decode-d768-e8-top2-r16-fp16"], "fused", 0),
        ("skew-e32-keyad", BY_NAME["skew-d1024-e32-top4-r16-fp16"].scaled(batch=1, seq_len=1024), "fused", 0),
        ("fp32-512", BY_NAME["cmix-d512-e4-top1-r8-fp32"], "fused", 0),
        ("bf16-d2048", BY_NAME["cmix-d2048-e16-top2-r32-bf16"].scaled(batch=1, seq_len=512), "fused", 0),
        ("mixed-fused", HEADLINE, "fused", 1),
        ("mixed-sparse", HEADLINE, "sparse", 1),
    ]


@pytest.mark.parametrize("name,shape,mode,mixed", _cases(), ids=[c[0] for c in _cases()])
def test_prepared_matches_unprepared(device, name, shape, mode, mixed):
    import torch
    from rwkv_mlx_amd import _lib
    from rwkv_mlx_amd.workloads import make_inputs
    print(f"\n[prepared] {name}", flush=True)
    L = Layer(shape, device, mode=mode)
    flags = L.flags
    ins = L.inputs()
    out_dt = L.dt
    if mixed:
        g32 = make_inputs(replace(shape, dtype="f32"))
        ins.update(w_gate=to_dev(g32["Wg"], "f32", device), lora_A=to_dev(g32["A"], "f32", device),
                   lora_B=to_dev(g32["B"], "f32", device))
        flags |= _lib.GATE_F32 | _lib.ADAPTERS_F32
        out_dt = torch.float32
    desc = L.make_desc(mode=mode, flags=flags)
    nbytes = _lib.workspace_bytes(desc)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    prep = torch.empty(_lib.prepared_bytes(desc), dtype=torch.uint8, device=device)
    stream = _lib.current_stream(device)
    _lib.prepare_adapters(desc, ins["lora_A"], ins["lora_B"], prep, stream)
    res = []
    for use in (None, prep):
        out = torch.empty(L.N, shape.d_model, dtype=out_dt, device=device)
        losses = torch.empty(2, dtype=torch.float32, device=device)
        inds = torch.empty(L.N, shape.top_k, dtype=torch.int32, device=device)
        ortho = torch.empty(1, dtype=torch.float32, device=device)
        t = _lib.make_tensors(out=out, losses=losses, inds=inds, ortho_loss=ortho, prepared=use, **ins)
        _lib.call("rwkvmoe_forward", desc, t, ws, nbytes, stream)
        torch.cuda.synchronize()
        res.append([a.cpu().numpy() for a in (out.float(), losses, inds, ortho)])
    for a, b, what in zip(res[0], res[1], ("out", "losses", "inds", "ortho")):
        assert np.array_equal(a, b), f"{what} differs with prepared adapters"


def test_module_cache_follows_updates(device):
    """The module's cache of the prepared adapters is reused while lora_A /
    lora_B are unchanged and remade after: an in-place update through the
    parameter (version counter), ``p.data = t``, two checkpoint loads in a
    row between forwards (the old storage cannot hand its address to the new
    one: the cache keeps it alive), and an in-place write through ``p.data``
    followed by invalidate_prepared()."""
    import torch
    from rwkv_mlx_amd.checkpoint import load_moe_layer, moe_state
    from rwkv_mlx_amd.moe import build_layer
    torch.manual_seed(1)
    m = build_layer(256, 512, 8, 2, 16).cuda().half()
    with torch.no_grad():
        m.base.x_k.uniform_(0, 1)
        m.lora_B.normal_(0, 0.02)
    x = torch.randn(2, 300, 256, device="cuda").half()

    def fresh_out():
        f = build_layer(256, 512, 8, 2, 16).cuda().half()
        f.load_state_dict(m.state_dict())
        return f(x)[0]

    with torch.no_grad():
        a, _, _ = m(x)
        src = m._prep_src
        b, _, _ = m(x)
        assert m._prep_src is src and torch.equal(a, b)    # reused
        m.lora_B.mul_(-1.5)                                 # in place: version counter moves
        c, _, _ = m(x)
        assert m._prep_src is not src
        assert torch.equal(c, fresh_out()) and not torch.equal(a, c)
        # p.data = t with new values
        m.lora_B.data = (m.lora_B.detach() * 0.5).clone()
        d, _, _ = m(x)
        assert torch.equal(d, fresh_out()) and not torch.equal(c, d)
        # two checkpoint loads between forwards: the second may reuse the
        # first's freed allocation, never the cached storage's
        sd1 = moe_state({0: m})
        sd2 = {k: (v * 2 if k.endswith("lora_B") else v) for k, v in sd1.items()}
        load_moe_layer(m, {k: v * 3 if k.endswith("lora_B") else v for k, v in sd1.items()}, 0)
        load_moe_layer(m, sd2, 0)
        e, _, _ = m(x)
        assert torch.equal(e, fresh_out()) and not torch.equal(d, e)
        # in place through .data: no version counter moves; invalidate_prepared() is the documented remedy
        m.lora_B.data.mul_(-1.0)
        m.invalidate_prepared()
        f, _, _ = m(x)
        assert torch.equal(f, fresh_out()) and not torch.equal(e, f)
