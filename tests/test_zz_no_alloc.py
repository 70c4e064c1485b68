"""rwkvmoe_forward_noalloc (the forward on the library's own device scratch)
against rwkvmoe_forward with a caller workspace, through the C ABI: two calls
in a row on the same GPU, the second on a smaller layer, each bit-identical to
the workspace forward (same kernels, same inputs), on the many-token FUSED
and SPARSE paths, the two-launch decode path (at most 64 tokens, whose
scratch regions the many-token calls never touch) and ln2 in front of the
layer (RWKVMOE_LN_IN, with LN(x) kept in the scratch); the forward captured
into a HIP graph after an eager call and replayed; and the host-side
rejection of a layer whose workspace exceeds the scratch.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import Layer, to_dev

pytestmark = pytest.mark.gpu


def _ln_params(layer):
    rng = np.random.default_rng(21)
    C = layer.w.d_model
    return (to_dev(1.0 + 0.1 * rng.standard_normal(C), layer.w.dtype, layer.dev),
            to_dev(0.05 * rng.standard_normal(C), layer.w.dtype, layer.dev))


def _run_both(layer, mode, ln=False):
    import torch
    from rwkv_mlx_amd import _lib
    w = layer.w
    outs = []
    extra = {}
    flags = layer.flags
    if ln:
        lw, lb = _ln_params(layer)
        extra = dict(ln_weight=lw, ln_bias=lb)
        flags |= _lib.LN_IN
    for entry in ("ws", "noalloc"):
        out = torch.empty_like(layer.x)
        losses = torch.empty(2, dtype=torch.float32, device=layer.dev)
        inds = torch.empty(layer.N, w.top_k, dtype=torch.int32, device=layer.dev)
        desc = layer.make_desc(mode=mode, flags=flags)
        t = _lib.make_tensors(out=out, losses=losses, inds=inds, **layer.inputs(), **extra)
        if entry == "ws":
            nbytes = _lib.workspace_bytes(desc)
            ws = torch.empty(nbytes, dtype=torch.uint8, device=layer.dev)
            _lib.call("rwkvmoe_forward", desc, t, ws, nbytes, _lib.current_stream(layer.dev))
        else:
            _lib.forward_noalloc(desc, t, _lib.current_stream(layer.dev))
        torch.cuda.synchronize()
        outs.append((out.float().cpu().numpy(), losses.cpu().numpy(), inds.cpu().numpy()))
    return outs


def _assert_same(res):
    (o1, l1, i1), (o2, l2, i2) = res
    assert np.array_equal(i1, i2), "router indices differ"
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32)), "outputs differ"
    assert np.array_equal(l1.view(np.uint32), l2.view(np.uint32)), "losses differ"


@pytest.mark.parametrize("mode", ["fused", "sparse"])
def test_noalloc_matches_workspace_forward(device, mode):
    from rwkv_mlx_amd.workloads import HEADLINE
    # the headline layer (4096 tokens), then a smaller one reusing the scratch
    for shape in (HEADLINE, HEADLINE.scaled(batch=3, seq_len=100)):
        print(f"noalloc {mode} {shape.name} tokens={shape.tokens}", flush=True)
        _assert_same(_run_both(Layer(shape, device, mode=mode), mode))


def test_noalloc_decode_and_ln(device):
    """The two-launch decode path (64 then 19 sequences with a carried state:
    its h / u / gate regions of the scratch) and ln2 in front of the layer
    (LN(x) in the scratch), each after the other on the same scratch."""
    from rwkv_mlx_amd.workloads import BY_NAME, HEADLINE
    dec = BY_NAME["decode-d768-e8-top2-r16-fp16"]
    cases = [(dec, False), (dec.scaled(batch=19, seq_len=1), False), (dec, True),
             (HEADLINE.scaled(batch=2, seq_len=512), True), (HEADLINE.scaled(batch=1, seq_len=40), True)]
    for shape, ln in cases:
        print(f"noalloc {shape.name} tokens={shape.tokens} ln={ln}", flush=True)
        _assert_same(_run_both(Layer(shape, device, mode="fused"), "fused", ln=ln))


@pytest.mark.parametrize("name", ["cmix-d768-e8-top2-r16-fp16", "decode-d768-e8-top2-r16-fp16"])
def test_noalloc_graph_replay(device, name):
    """rwkvmoe_forward_noalloc captured into a HIP graph after an eager call
    (which resolves the scratch address outside the capture), replayed three
    times with the program's own work between replays: every replay equals
    the eager call bit for bit."""
    import torch
    from rwkv_mlx_amd import _lib
    from rwkv_mlx_amd.workloads import BY_NAME
    print(f"noalloc graph {name}", flush=True)
    L = Layer(BY_NAME[name], device, mode="fused")
    out = torch.empty_like(L.x)
    losses = torch.empty(2, dtype=torch.float32, device=device)
    inds = torch.empty(L.N, L.w.top_k, dtype=torch.int32, device=device)
    desc = L.make_desc()
    t = _lib.make_tensors(out=out, losses=losses, inds=inds, **L.inputs())

    def run():
        _lib.forward_noalloc(desc, t, _lib.current_stream(device))

    run()
    torch.cuda.synchronize()
    ref = [a.clone() for a in (out, losses, inds)]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    torch.cuda.synchronize()
    for rep in range(3):
        out.fill_(float("nan"))
        losses.fill_(float("nan"))
        inds.fill_(-7)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip((out, losses, inds), ref):
            assert torch.equal(a.view(torch.uint8) if a.dtype != torch.int32 else a,
                               b.view(torch.uint8) if b.dtype != torch.int32 else b), f"replay {rep} differs"
    del g


def test_noalloc_rejects_layers_beyond_scratch(device):
    import torch
    from rwkv_mlx_amd import _lib
    from rwkv_mlx_amd.workloads import BY_NAME
    w = BY_NAME["cmix-d2048-e16-top2-r32-bf16"]  # 341 MiB of workspace
    desc = _lib.make_desc(w.batch, w.seq_len, w.d_model, w.d_ffn, w.n_experts, w.top_k, w.lora_rank, w.dtype)
    assert _lib.workspace_bytes(desc) > _lib.NOALLOC_SCRATCH_BYTES
    dummy = torch.empty(16, dtype=torch.bfloat16, device=device)  # never read: rejected on the host
    t = _lib.make_tensors(x=dummy, x_k=dummy, w_key=dummy, w_value=dummy, w_gate=dummy, lora_A=dummy,
                          lora_B=dummy, out=dummy, losses=torch.empty(2, device=device))
    with pytest.raises(_lib.RwkvMoeError) as ei:
        _lib.forward_noalloc(desc, t, _lib.current_stream(device))
    assert ei.value.status == -11
