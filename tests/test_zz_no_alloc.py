"""rwkvmoe_forward_noalloc (the forward on the library's own device scratch)
against rwkvmoe_forward with a caller workspace, through the C ABI: two calls
in a row on the same GPU, the second on a smaller layer, each bit-identical to
the workspace forward (same kernels, same inputs).  Also the host-side
rejection of a layer whose workspace exceeds the scratch.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import Layer

pytestmark = pytest.mark.gpu


def _run_both(layer, mode):
    import torch
    from rwkv_mlx_amd import _lib
    w = layer.w
    outs = []
    for entry in ("ws", "noalloc"):
        out = torch.empty_like(layer.x)
        losses = torch.empty(2, dtype=torch.float32, device=layer.dev)
        inds = torch.empty(layer.N, w.top_k, dtype=torch.int32, device=layer.dev)
        desc = layer.make_desc(mode=mode)
        t = _lib.make_tensors(out=out, losses=losses, inds=inds, **layer.inputs())
        if entry == "ws":
            nbytes = _lib.workspace_bytes(desc)
            ws = torch.empty(nbytes, dtype=torch.uint8, device=layer.dev)
            _lib.call("rwkvmoe_forward", desc, t, ws, nbytes, _lib.current_stream(layer.dev))
        else:
            _lib.forward_noalloc(desc, t, _lib.current_stream(layer.dev))
        torch.cuda.synchronize()
        outs.append((out.float().cpu().numpy(), losses.cpu().numpy(), inds.cpu().numpy()))
    return outs


@pytest.mark.parametrize("mode", ["fused", "sparse"])
def test_noalloc_matches_workspace_forward(device, mode):
    from rwkv_mlx_amd.workloads import HEADLINE
    # the headline layer (4096 tokens), then a smaller one reusing the scratch
    for shape in (HEADLINE, HEADLINE.scaled(batch=3, seq_len=100)):
        print(f"noalloc {mode} {shape.name} tokens={shape.tokens}", flush=True)
        (o1, l1, i1), (o2, l2, i2) = _run_both(Layer(shape, device, mode=mode), mode)
        assert np.array_equal(i1, i2), "router indices differ"
        assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32)), "outputs differ"
        assert np.array_equal(l1.view(np.uint32), l2.view(np.uint32)), "losses differ"


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
