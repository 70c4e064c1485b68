"""HIP graph capture of the C ABI entry points.

A serving or training loop can capture a layer call in a graph
(torch.cuda.CUDAGraph over the stream the library launches on) and replay
it: the library allocates nothing, issues no memset and no host
synchronisation, and every counter a kernel relies on is cleared by an
earlier kernel of the same call.  Each case runs the entry point eagerly,
captures the same call on static buffers, then replays it three times with
the program's own eager work (outputs overwritten with NaN / -7) and device
synchronisations between the replays; every replay must reproduce the eager
outputs bit for bit (the kernels are deterministic).  Then new inputs are
copied into the static input buffers, the graph is replayed, and the result
must equal an eager call on those inputs.  Cases: the D=768, E=8, top-2
layer at 4096 tokens in FUSED and SPARSE mode, the decode batch of 64
tokens, the layer's backward (dx, dA, dB, dW_gate), and the full-expert
layer.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import Layer, to_dev
from rwkv_mlx_amd.workloads import BY_NAME

pytestmark = pytest.mark.gpu

REPLAYS = 3


def _bytes(t):
    import torch
    return t.detach().contiguous().view(-1).view(torch.uint8).cpu().numpy()


def _poison(outs):
    for o in outs:
        if o.dtype.is_floating_point:
            o.fill_(float("nan"))
        else:
            o.fill_(-7)


def _check_graph(run, outs, refresh):
    """run(): the call on static buffers (launches on the current stream);
    outs: its outputs; refresh(): copies new inputs into the static inputs."""
    import torch
    run()
    torch.cuda.synchronize()
    ref = [_bytes(o) for o in outs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    torch.cuda.synchronize()
    for rep in range(REPLAYS):
        _poison(outs)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (o, r) in enumerate(zip(outs, ref)):
            assert np.array_equal(_bytes(o), r), f"replay {rep}: output {i} differs from the eager call"
    refresh()
    g.replay()
    torch.cuda.synchronize()
    got = [_bytes(o) for o in outs]
    _poison(outs)
    run()
    torch.cuda.synchronize()
    for i, (o, r) in enumerate(zip(outs, got)):
        assert np.array_equal(_bytes(o), r), f"new inputs: output {i} of the replay differs from the eager call"
    assert not np.array_equal(got[0], ref[0]), "new inputs gave the old outputs"


def _refresher(L, seed):
    import torch

    def refresh():
        rng = np.random.default_rng(seed)
        x2 = to_dev(rng.standard_normal(tuple(L.x.shape)).astype(np.float32), L.w.dtype, L.dev)
        L.x.copy_(x2)
        torch.cuda.synchronize()
    return refresh


@pytest.mark.parametrize("name,mode", [("cmix-d768-e8-top2-r16-fp16", "fused"),
                                       ("cmix-d768-e8-top2-r16-fp16", "sparse"),
                                       ("decode-d768-e8-top2-r16-fp16", "fused")])
def test_forward_graph_replays_match_eager(device, name, mode):
    import torch
    from rwkv_mlx_amd import _lib
    print(f"\n[graph forward] {name} {mode}", flush=True)
    shape = BY_NAME[name]
    L = Layer(shape, device, mode=mode)
    w = L.w
    out = torch.empty_like(L.x)
    losses = torch.empty(2, dtype=torch.float32, device=device)
    ex = dict(logits=torch.empty(L.N, w.n_experts, dtype=torch.float32, device=device),
              inds=torch.empty(L.N, w.top_k, dtype=torch.int32, device=device),
              perm=torch.empty(L.N * w.top_k, dtype=torch.int32, device=device),
              inv_perm=torch.empty(L.N * w.top_k, dtype=torch.int32, device=device),
              offsets=torch.empty(w.n_experts + 1, dtype=torch.int32, device=device))
    entry = "rwkvmoe_decode" if shape.decode else "rwkvmoe_forward"
    t = _lib.make_tensors(out=out, losses=losses, **L.inputs(), **ex)

    def run():
        _lib.call(entry, L.desc, t, L.ws, L.ws_bytes, _lib.current_stream(device))

    _check_graph(run, [out, losses] + list(ex.values()), _refresher(L, 4242))


def test_backward_graph_replays_match_eager(device):
    import torch
    from rwkv_mlx_amd import _lib
    print("\n[graph backward] cmix-d768-e8-top2-r16-fp16", flush=True)
    L = Layer(BY_NAME["cmix-d768-e8-top2-r16-fp16"], device)
    w = L.w
    _, _, ex = L.forward(extras=True)
    rng = np.random.default_rng(77)
    dO = to_dev(rng.standard_normal((L.N, w.d_model)).astype(np.float32), w.dtype, device)
    d_losses = torch.tensor([0.01, 0.001], dtype=torch.float32, device=device)
    outs = dict(d_x=torch.empty(L.N, w.d_model, dtype=L.dt, device=device),
                d_lora_A=torch.empty(w.n_experts, w.d_model, w.lora_rank, dtype=L.dt, device=device),
                d_lora_B=torch.empty(w.n_experts, w.lora_rank, w.d_model, dtype=L.dt, device=device),
                d_w_gate=torch.empty(w.n_experts, w.d_model, dtype=L.dt, device=device))
    nbytes = _lib.backward_workspace_bytes(L.desc)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)

    def run():
        _lib.backward(L.desc, ws, nbytes, _lib.current_stream(device), x=L.x, w_gate=L.Wg, lora_A=L.A,
                      lora_B=L.B, logits=ex["logits"], inds=ex["inds"], d_out=dO, d_losses=d_losses, **outs)

    def refresh():
        dO.copy_(to_dev(np.random.default_rng(78).standard_normal((L.N, w.d_model)).astype(np.float32), w.dtype,
                        device))
        torch.cuda.synchronize()

    _check_graph(run, list(outs.values()), refresh)


def test_experts_graph_replays_match_eager(device):
    import torch
    from rwkv_mlx_amd import _lib
    print("\n[graph experts] D=768 F=3072 E=8 top-2 fp16, 4096 tokens", flush=True)
    B, T, C, F, E, k = 8, 512, 768, 3072, 8, 2
    N = B * T
    gen = torch.Generator(device=device).manual_seed(5151)
    rn = lambda *s, scale=1.0: (torch.randn(*s, generator=gen, device=device) * scale).to(torch.float16)
    x = rn(B, T, C)
    x_k = torch.rand(E, C, generator=gen, device=device).to(torch.float16)
    wk = rn(E, F, C, scale=C ** -0.5)
    wv = rn(E, C, F, scale=F ** -0.5)
    wg = rn(E, C, scale=C ** -0.5)
    desc = _lib.make_desc(B, T, C, F, E, k, 1, "f16", _lib.MODE_FUSED, 0)
    nbytes = _lib.experts_workspace_bytes(desc)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    out = torch.empty_like(x)
    losses = torch.empty(2, dtype=torch.float32, device=device)
    ex = dict(logits=torch.empty(N, E, dtype=torch.float32, device=device),
              inds=torch.empty(N, k, dtype=torch.int32, device=device),
              perm=torch.empty(N * k, dtype=torch.int32, device=device),
              offsets=torch.empty(E + 1, dtype=torch.int32, device=device))
    t = _lib.make_tensors(x=x, x_k=x_k, w_key=wk, w_value=wv, w_gate=wg, out=out, losses=losses, **ex)

    def run():
        _lib.call("rwkvmoe_experts_forward", desc, t, ws, nbytes, _lib.current_stream(device))

    def refresh():
        x.copy_(rn(B, T, C))
        torch.cuda.synchronize()

    _check_graph(run, [out, losses] + list(ex.values()), refresh)
