"""The expert adapters' contribution checked at its own scale (moe.py:138-145).

The layer's output is base + delta with max|base| 8-14x max|delta| on the
seeded workloads, so an output-level bar of 2e-2 (or a delta bar scaled by
max|base| / max|delta|) leaves room for a wrong delta.  Here the base is
taken out of the comparison:

* W_value = 0 makes the base exactly zero (h · 0), so the forward's output
  IS the delta, computed by the same kernels as ever: FUSED through the
  router's gated adapter product U and the value product's K-extension,
  SPARSE through the router's unscaled adapter product u and the value
  product's rank slices where the layer has E·r <= 128 (the D=768 cases),
  else through dispatch, the MFMA grouped LoRA and combine.  It must match
  the oracle's delta (moe.py's dense expert loop, MLX's rounding points)
  within 2e-2 of max|delta| element-wise and 2e-2 in norm: the dtype
  tolerance, at the delta's own scale.
* The SPARSE forward's two forms agree at the same bar: on chip (above)
  and through dispatch, the grouped LoRA and the fused combine (the form
  taken when the caller asks for the adapter rows).
* The MFMA grouped LoRA kernel's adapter rows (rwkvmoe_lora_grouped, no
  RWKVMOE_LORA_VALU) must match (x·A_e)·B_e per routed row within 2e-2 of
  max|rows|.

Shapes: the D=768 E=8 top-2 r=16 layer in fp16 and in bf16, the skewed
E=32 top-4 layer (fp16) and the wide D=2048 E=16 r=32 layer (bf16): k >= 2
with unequal gates (the tests check that most tokens' two largest gates
differ by more than 0.1).

A planted mistake shows the bars' reach (CPU, oracle only): the slot gates
swapped on the tokens whose two gates differ by less than 0.1 — a mistake
that only shows on near-tied pairs — moves the delta by 13-15% of max|delta|
(5-7% in norm).  The own-scale bars reject it; the old output-scaled bar,
2e-2 · max|base| / max|delta| ≈ 0.21-0.24, would not.
"""
from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest

from helpers import Layer, rel_errs, sample_rows, to_np
from oracle import moe_oracle as O
from rwkv_mlx_amd.workloads import BY_NAME, HEADLINE, make_inputs

DELTA_MAX_REL = 2e-2      # element-wise, relative to max|delta| (measured: <= 4.4e-3, FUSED bf16)
DELTA_NORM_REL = 2e-2     # ||got - ref|| / ||ref||
ROWS_REL = 2e-2           # adapter rows, relative to max|rows| (max and norm)

SHAPES = [
    HEADLINE,
    replace(HEADLINE, name="cmix-d768-e8-top2-r16-bf16", dtype="bf16", seed=1011),
    BY_NAME["skew-d1024-e32-top4-r16-fp16"],
    BY_NAME["cmix-d2048-e16-top2-r32-bf16"],
]
IDS = [s.name for s in SHAPES]


def _rows(shape, n=384):
    return np.arange(shape.tokens) if shape.tokens <= 4096 else sample_rows(shape.tokens, shape.seq_len, n=n)


def _oracle_delta(g, shape, rows, gates=None):
    x = g["x"].reshape(shape.tokens, -1)
    rt = O.router(x[rows], g["Wg"], shape.top_k, shape.dtype, g.get("bias"))
    gt = rt["gates"] if gates is None else gates
    return O.lora_delta_dense(x[rows], g["A"], g["B"], rt["inds"], gt, shape.dtype), rt


def _swap_near_tied(gates, thr=0.1):
    """The planted mistake: slots 0 and 1 swap gates on tokens whose gates
    differ by less than thr."""
    gs = gates.copy()
    sel = np.abs(gates[:, 0] - gates[:, 1]) < thr
    gs[sel, 0], gs[sel, 1] = gates[sel, 1], gates[sel, 0]
    return gs


# ---- the planted mistake (CPU: the oracle against itself) ------------------------------

@pytest.mark.parametrize("shape", SHAPES, ids=IDS)
def test_planted_gate_swap_is_caught_at_own_scale(shape):
    g = make_inputs(shape)
    rows = sample_rows(shape.tokens, shape.seq_len, n=256)
    ref, rt = _oracle_delta(g, shape, rows)
    bad = O.lora_delta_dense(g["x"].reshape(shape.tokens, -1)[rows], g["A"], g["B"], rt["inds"],
                             _swap_near_tied(rt["gates"]), shape.dtype)
    emax, enorm = rel_errs(bad, ref)
    assert emax > DELTA_MAX_REL and enorm > DELTA_NORM_REL, (emax, enorm)
    # the output-scaled bar of a delta check against the full layer would let it pass
    C = shape.d_model
    x = g["x"].reshape(shape.tokens, C)
    prev = np.zeros((rows.size, C), np.float32)
    for i, r in enumerate(rows):
        if r % shape.seq_len:
            prev[i] = x[r - 1]
    base = O.cmix_base(x[rows][:, None, :], g["x_k"], g["Wk"], g["Wv"], shape.dtype, x_prev=prev).reshape(-1, C)
    old_bar = 2e-2 * max(1.0, float(np.max(np.abs(base))) / float(np.max(np.abs(ref))))
    assert emax < old_bar, (emax, old_bar)


# ---- the GPU kernels -----------------------------------------------------------------

@pytest.fixture(scope="module", params=SHAPES, ids=IDS)
def case(request, device):
    shape = request.param
    print(f"\n[adapter delta] {shape.name}", flush=True)
    L = Layer(shape, device)
    L.Wv.zero_()  # base = h · 0 = 0 exactly: the output is the adapter delta alone
    rows = _rows(shape)
    ref, rt = _oracle_delta(L.np, shape, rows)
    gates = rt["gates"]
    gap = np.abs(gates[:, 0] - gates[:, 1])
    assert np.mean(gap > 0.1) > 0.5, "the check needs unequal gates"
    return L, rows, ref, rt


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["fused", "sparse"])
def test_delta_at_its_own_scale(case, mode):
    L, rows, ref, rt = case
    out, _, ex = L.forward(mode=mode, extras=True)
    assert np.array_equal(ex["inds"].cpu().numpy()[rows], rt["inds"]), "routing differs"
    got = to_np(out).reshape(L.N, -1)[rows]
    emax, enorm = rel_errs(got, ref)
    print(f"  {mode}: delta max-rel {emax:.2e} norm-rel {enorm:.2e}", flush=True)
    assert np.all(np.isfinite(got))
    assert emax <= DELTA_MAX_REL and enorm <= DELTA_NORM_REL, \
        f"{L.w.name}/{mode}: delta max-rel {emax:.3e} norm-rel {enorm:.3e}"


@pytest.mark.gpu
def test_grouped_lora_rows_at_their_own_scale(case):
    """The MFMA grouped LoRA kernel (the SPARSE default) per routed row."""
    import torch
    L, _, _, _ = case
    shape = L.w
    k, C = shape.top_k, shape.d_model
    _, _, ex = L.forward(mode="sparse", extras=True)
    ag = torch.empty(L.N * k, C, dtype=L.dt, device=L.dev)
    L.call("rwkvmoe_lora_grouped", L.make_desc(mode="sparse"), x=L.x, lora_A=L.A, lora_B=L.B, perm=ex["perm"],
           offsets=ex["offsets"], adapter_rows=ag)
    torch.cuda.synchronize()
    pm = ex["perm"].cpu().numpy()
    inds = ex["inds"].cpu().numpy().reshape(-1)
    pick = np.random.default_rng(3).choice(pm.size, min(pm.size, 1024), replace=False)
    x = L.np["x"].reshape(-1, C)
    a = pm[pick]
    e = inds[a]
    want = np.empty((pick.size, C), np.float32)
    for ee in np.unique(e):
        m = e == ee
        want[m] = O.lora_adapter(x[a[m] // k], L.np["A"][ee], L.np["B"][ee], shape.dtype)
    got = to_np(ag)[a]  # (rows in assignment order)
    emax, enorm = rel_errs(got, want)
    print(f"  rows: max-rel {emax:.2e} norm-rel {enorm:.2e}", flush=True)
    assert emax <= ROWS_REL and enorm <= ROWS_REL, f"{shape.name}: rows max-rel {emax:.3e} norm-rel {enorm:.3e}"


@pytest.mark.gpu
def test_sparse_forms_agree(case):
    """The SPARSE forward on chip (router u + rank slices, where the layer
    allows it) against the same forward through dispatch, the grouped LoRA
    and the fused combine (requested adapter rows select it): the deltas
    agree within the own-scale bar, and the second form's adapter rows are
    written."""
    import torch
    L, rows, ref, rt = case
    shape = L.w
    out_a, _, _ = L.forward(mode="sparse")
    out_b = torch.empty_like(L.x)
    losses = torch.empty(2, dtype=torch.float32, device=L.dev)
    ag = torch.full((L.N * shape.top_k, shape.d_model), float("nan"), dtype=L.dt, device=L.dev)
    L.call("rwkvmoe_forward", L.make_desc(mode="sparse"), out=out_b, losses=losses, adapter_rows=ag, **L.inputs())
    torch.cuda.synchronize()
    a = to_np(out_a).reshape(L.N, -1)[rows]
    b = to_np(out_b).reshape(L.N, -1)[rows]
    emax, enorm = rel_errs(a, b)
    print(f"  forms: max-rel {emax:.2e} norm-rel {enorm:.2e}", flush=True)
    assert np.all(np.isfinite(to_np(ag))), "the grouped form's adapter rows were not all written"
    assert emax <= DELTA_MAX_REL and enorm <= DELTA_NORM_REL, f"{shape.name}: forms max-rel {emax:.3e}"
    ea, _ = rel_errs(a, ref)
    eb, _ = rel_errs(b, ref)
    print(f"  vs oracle: on chip {ea:.2e}, grouped {eb:.2e}", flush=True)
