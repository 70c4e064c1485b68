"""GPU dispatch against the oracle's stable counting sort, bit-exact, over
assignment counts on both sides of the single-workgroup limit (2048) and
of the switch to 1024-assignment blocks (65536), and expert counts from 1 to
64, including skewed routing where most assignments
go to one expert."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

CASES = [  # (assignments, experts, skew)
    (1, 1, 0.0), (63, 5, 0.0), (64, 8, 0.0), (65, 8, 0.0), (128, 8, 0.0), (1000, 3, 0.0), (2048, 64, 0.0),
    (2048, 8, 0.9), (2049, 8, 0.0), (8192, 8, 0.0), (8192, 64, 0.0), (8192, 32, 0.9), (16384, 1, 0.0),
    (40000, 8, 0.5), (65536, 16, 0.0), (65537, 64, 0.3), (200000, 8, 0.0),
]


def _call(inds_np, E):
    import torch
    from rwkv_mlx_amd import _lib
    dev = torch.device("cuda", 0)
    nk = inds_np.size
    inds = torch.from_numpy(inds_np.astype(np.int32)).to(dev)
    perm = torch.full((nk,), -7, dtype=torch.int32, device=dev)
    inv = torch.full((nk,), -7, dtype=torch.int32, device=dev)
    offs = torch.full((E + 1,), -7, dtype=torch.int32, device=dev)
    # the layer shape only fixes N*k and E here: N = nk tokens, top-1
    desc = _lib.make_desc(batch=1, seq_len=nk, d_model=64, d_ffn=64, n_experts=E, top_k=1, lora_rank=1, dtype="f16")
    nws = _lib.workspace_bytes(desc)
    ws = torch.empty(nws, dtype=torch.uint8, device=dev)
    t = _lib.make_tensors(inds=inds, perm=perm, inv_perm=inv, offsets=offs)
    _lib.call("rwkvmoe_dispatch", desc, t, ws, nws, _lib.current_stream(dev))
    torch.cuda.synchronize()
    return perm.cpu().numpy(), inv.cpu().numpy(), offs.cpu().numpy()


@pytest.mark.parametrize("nk,E,skew", CASES)
def test_dispatch_matches_stable_sort(nk, E, skew):
    print(f"\n[dispatch] nk={nk} E={E} skew={skew}", flush=True)
    rng = np.random.default_rng(nk * 131 + E)
    inds = rng.integers(0, E, size=nk)
    if skew > 0:
        inds = np.where(rng.random(nk) < skew, E - 1, inds)
    p, i, o = _call(inds, E)
    rp, ri, ro = O.dispatch(inds.reshape(nk, 1), E)
    assert np.array_equal(o, ro)
    assert np.array_equal(p, rp)
    assert np.array_equal(i, ri)
