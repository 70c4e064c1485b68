"""The C ABI of librwkvmoe.so without a GPU: the library loads, exports every
entry point include/rwkvmoe.h declares, its ctypes mirror matches the
header's structs, and every argument error is reported with its status code
on the host before any HIP call.

No test here launches a kernel: every forward / stage call is built to fail
validation (and the whole module is skipped where a GPU is visible, so a
mistake in a test can never send the fake addresses used here to a device).
"""
from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "rwkvmoe.h"


def _gpu_visible() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


pytestmark = pytest.mark.skipif(_gpu_visible(), reason="host-only argument checks use fake device addresses")


@pytest.fixture(scope="module")
def L():
    from rwkv_mlx_amd import _lib
    if not _lib.LIB_PATH.exists():
        from rwkv_mlx_amd import build
        build.build(verbose=False)
    return _lib


def header_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(rwkvmoe_\w+)\s*\(", text, flags=re.M)))


def header_struct_fields(name: str) -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), text, flags=re.S).group(1)
    return re.findall(r"(\w+)\s*;", body)


def header_define(name: str) -> int:
    m = re.search(r"#define\s+%s\s+(-?\d+)" % name, HEADER.read_text())
    return int(m.group(1))


# ---- library and header ---------------------------------------------------------

def test_every_declared_symbol_is_exported(L):
    declared = header_functions()
    assert len(declared) >= 13, declared
    h = L.lib()
    for name in declared:
        assert hasattr(h, name), f"{name} declared in rwkvmoe.h but not exported"
    nm = subprocess.run(["nm", "-D", "--defined-only", str(L.LIB_PATH)], capture_output=True, text=True)
    if nm.returncode == 0:
        exported = set(re.findall(r"\b(rwkvmoe_\w+)\b", nm.stdout))
        assert set(declared) == exported, f"exported-but-undeclared: {exported - set(declared)}"


def test_python_binding_lists_every_entry_point(L):
    assert sorted(L.ENTRY_POINTS) == header_functions()


def test_ctypes_structs_match_header(L):
    assert [f[0] for f in L.Desc._fields_] == header_struct_fields("rwkvmoe_desc")
    assert [f[0] for f in L.Tensors._fields_] == header_struct_fields("rwkvmoe_tensors")
    assert ctypes.sizeof(L.Desc) == 10 * 4
    assert ctypes.sizeof(L.Tensors) == len(L.Tensors._fields_) * 8
    assert [f[0] for f in L.Grads._fields_] == header_struct_fields("rwkvmoe_grads")
    assert ctypes.sizeof(L.Grads) == len(L.Grads._fields_) * 8
    assert [f[0] for f in L.ExpertsGrads._fields_] == header_struct_fields("rwkvmoe_experts_grads")
    assert ctypes.sizeof(L.ExpertsGrads) == len(L.ExpertsGrads._fields_) * 8
    assert [f[0] for f in L.RouterGrads._fields_] == header_struct_fields("rwkvmoe_router_grads")
    assert ctypes.sizeof(L.RouterGrads) == len(L.RouterGrads._fields_) * 8
    assert [f[0] for f in L.LnGrads._fields_] == header_struct_fields("rwkvmoe_ln_grads")
    assert ctypes.sizeof(L.LnGrads) == len(L.LnGrads._fields_) * 8


def test_status_codes_match_header(L):
    for code, name in L.STATUS.items():
        assert header_define(name) == code
    assert header_define("RWKVMOE_MAX_KERNELS") == L.MAX_KERNELS
    assert header_define("RWKVMOE_TIMED_PAIR_EVENTS") == L.TIMED_PAIR_EVENTS


def test_status_strings(L):
    texts = {c: L.status_string(c) for c in L.STATUS}
    assert texts[0] == "success"
    assert len(set(texts.values())) == len(texts), "status strings must be distinct"
    assert L.status_string(-1234) == "unknown status"


def test_version(L):
    assert L.lib().rwkvmoe_version() == 200


def test_tensors_struct_size_is_checked(L):
    """rwkvmoe_tensors leads with struct_size; any other value than the
    library's sizeof(rwkvmoe_tensors) is RWKVMOE_ERR_VERSION before anything
    else of the struct is read — including a caller built against the
    previous layout, whose first field was the x pointer."""
    d = desc(L)
    assert L.Tensors.struct_size.offset == 0
    for bad in (0, ctypes.sizeof(L.Tensors) - 8, ctypes.sizeof(L.Tensors) + 8, FAKE):
        t = fake_tensors(L)
        t.struct_size = bad
        for name in ("rwkvmoe_forward", "rwkvmoe_decode", "rwkvmoe_router_topk", "rwkvmoe_experts_forward"):
            assert call_status(L, name, d, t, ws_bytes=1 << 34) == -12, (name, bad)
        assert L.lib().rwkvmoe_forward_noalloc(ctypes.byref(d), ctypes.byref(t), None) == -12


@pytest.mark.parametrize("kw,reads", [
    (dict(batch=64, seq_len=1), 1),                             # decode step of 64 sequences
    (dict(batch=4, seq_len=16), 1),                             # 64 tokens
    (dict(batch=65, seq_len=1), 0),                             # past the decode path
    (dict(), 0),                                                # the 4096-token layer
    (dict(batch=64, seq_len=1, mode=1), 0),                     # SPARSE
    (dict(batch=64, seq_len=1, dtype=0), 0),                    # fp32
    (dict(batch=64, seq_len=1, n_experts=32), 0),               # more than 16 experts
    (dict(batch=64, seq_len=1, flags=16), 0),                   # fp32 adapters
    (dict(batch=64, seq_len=1, dtype=2, flags=8), 0),           # bf16 layer with an fp32 gate
    (dict(batch=64, seq_len=1, flags=8), 1),                    # fp16 layer with an fp32 gate
])
def test_reads_prepared_base(L, kw, reads):
    d = desc(L, **kw)
    n = ctypes.c_int(-1)
    assert L.lib().rwkvmoe_reads_prepared_base(ctypes.byref(d), ctypes.byref(n)) == 0
    assert n.value == reads
    assert L.reads_prepared_base(d) == bool(reads)
    assert L.lib().rwkvmoe_reads_prepared_base(ctypes.byref(d), None) == -4
    assert L.lib().rwkvmoe_reads_prepared_base(None, ctypes.byref(n)) == -1


# ---- descriptor validation (host only) ------------------------------------------

HEADLINE = dict(batch=8, seq_len=512, d_model=768, d_ffn=3072, n_experts=8, top_k=2, lora_rank=16, dtype="f16")


def desc(L, **kw):
    a = {**HEADLINE, **kw}
    return L.make_desc(a["batch"], a["seq_len"], a["d_model"], a["d_ffn"], a["n_experts"], a["top_k"],
                       a["lora_rank"], a["dtype"], a.get("mode", 0), a.get("flags", 0))


def ws_status(L, d):
    n = ctypes.c_size_t(0)
    return L.lib().rwkvmoe_workspace_bytes(ctypes.byref(d), ctypes.byref(n)), n.value


@pytest.mark.parametrize("kw,code", [
    (dict(dtype=3), -3), (dict(dtype=-1), -3),
    (dict(mode=2), -9), (dict(flags=32), -8),
    (dict(batch=0), -2), (dict(seq_len=0), -2),
    (dict(d_model=96), -2), (dict(d_model=0), -2), (dict(d_model=8256), -2),
    (dict(d_ffn=100), -2), (dict(d_ffn=65600), -2),
    (dict(n_experts=0), -2), (dict(n_experts=65), -2),
    (dict(lora_rank=0), -2), (dict(lora_rank=33), -2),
    (dict(top_k=0), -7), (dict(top_k=9, n_experts=16), -7), (dict(top_k=3, n_experts=2), -7),
    (dict(batch=1 << 14, seq_len=1 << 12), -2),   # N * F beyond 2^31
])
def test_workspace_rejects_bad_desc(L, kw, code):
    st, _ = ws_status(L, desc(L, **kw))
    assert st == code, (kw, st)


def test_workspace_null_arguments(L):
    n = ctypes.c_size_t(0)
    assert L.lib().rwkvmoe_workspace_bytes(None, ctypes.byref(n)) == -1
    d = desc(L)
    assert L.lib().rwkvmoe_workspace_bytes(ctypes.byref(d), None) == -4


def test_workspace_sizes(L):
    st, fused = ws_status(L, desc(L))
    assert st == 0
    st, sparse = ws_status(L, desc(L, mode=1))
    assert st == 0
    N, C, F, E, k, r, s = 4096, 768, 3072, 8, 2, 16, 2
    # at least: hidden (N,F), xk (N,C); fused adds U (N, 128); sparse adds base (N,C) and adapter rows (N*k,C)
    assert fused >= N * F * s + N * C * s + N * 128 * s
    assert sparse >= N * F * s + N * C * s + N * C * s + N * k * C * s
    assert fused % 256 == 0 and sparse % 256 == 0
    # grows with the token count
    assert ws_status(L, desc(L, batch=16))[1] > fused
    # fp32 needs about twice the bytes of fp16
    assert ws_status(L, desc(L, dtype="f32"))[1] > 1.9 * fused * 0.9


# ---- entry point validation (fails before any HIP call) -------------------------

FAKE = 1 << 40  # 256-byte aligned, never dereferenced: every call below fails validation first


def fake_tensors(L, **override):
    names = ("x", "x_k", "w_key", "w_value", "w_gate", "lora_A", "lora_B", "out", "losses")
    kw = {n: FAKE + (i << 24) for i, n in enumerate(names)}
    kw.update(override)
    return L.make_tensors(**{k: v for k, v in kw.items() if v is not None})


def call_status(L, name, d, t, ws=FAKE + (1 << 32), ws_bytes=None):
    if ws_bytes is None:
        ws_bytes = ws_status(L, d)[1] if ws_status(L, d)[0] == 0 else 0
    fn = getattr(L.lib(), name)
    return fn(ctypes.byref(d) if d is not None else None, ctypes.byref(t) if t is not None else None,
              ws, ctypes.c_size_t(ws_bytes), None)


def test_forward_null_desc_and_tensors(L):
    d = desc(L)
    assert call_status(L, "rwkvmoe_forward", None, fake_tensors(L), ws_bytes=1 << 30) == -1
    assert call_status(L, "rwkvmoe_forward", d, None) == -1


@pytest.mark.parametrize("missing", ["x", "x_k", "w_key", "w_value", "w_gate", "lora_A", "lora_B", "out", "losses"])
def test_forward_missing_tensor(L, missing):
    assert call_status(L, "rwkvmoe_forward", desc(L), fake_tensors(L, **{missing: None})) == -4


@pytest.mark.parametrize("field,offset", [("x", 8), ("w_key", 2), ("out", 4), ("losses", 2), ("lora_A", 1)])
def test_forward_misaligned(L, field, offset):
    assert call_status(L, "rwkvmoe_forward", desc(L), fake_tensors(L, **{field: FAKE + offset})) == -5


def test_forward_workspace(L):
    d = desc(L)
    need = ws_status(L, d)[1]
    t = fake_tensors(L)
    assert call_status(L, "rwkvmoe_forward", d, t, ws=None, ws_bytes=need) == -6
    assert call_status(L, "rwkvmoe_forward", d, t, ws_bytes=need - 1) == -6
    assert call_status(L, "rwkvmoe_forward", d, t, ws=FAKE + 128, ws_bytes=need) == -6


def test_forward_flag_without_tensor(L):
    for flag in (1, 2, 4):
        assert call_status(L, "rwkvmoe_forward", desc(L, flags=flag), fake_tensors(L)) == -8


def test_decode_needs_single_token_and_state(L):
    t = fake_tensors(L, x_prev=FAKE + (64 << 24))
    assert call_status(L, "rwkvmoe_decode", desc(L, flags=1), t) == -9          # T = 512
    assert call_status(L, "rwkvmoe_decode", desc(L, seq_len=1), fake_tensors(L)) == -9  # no HAS_PREV


def test_forward_timed_needs_events(L):
    d = desc(L)
    t = fake_tensors(L)
    n = ctypes.c_int(-1)
    names = (ctypes.c_char_p * L.MAX_KERNELS)()
    few = (ctypes.c_void_p * L.MAX_KERNELS)(*([FAKE] * L.MAX_KERNELS))
    enough_null = (ctypes.c_void_p * (L.MAX_KERNELS + 1))()
    f = L.lib().rwkvmoe_forward_timed
    ws_bytes = ws_status(L, d)[1]
    assert f(ctypes.byref(d), ctypes.byref(t), FAKE, ws_bytes, None, few, L.MAX_KERNELS, names, ctypes.byref(n)) == -10
    assert f(ctypes.byref(d), ctypes.byref(t), FAKE, ws_bytes, None, enough_null, L.MAX_KERNELS + 1, names,
             ctypes.byref(n)) == -10
    assert f(ctypes.byref(d), ctypes.byref(t), FAKE, ws_bytes, None, few, L.MAX_KERNELS, None, None) == -10
    # argument errors of the forward itself pass through, with no kernel recorded
    ev = (ctypes.c_void_p * (L.MAX_KERNELS + 1))(*([FAKE] * (L.MAX_KERNELS + 1)))
    bad = fake_tensors(L, out=None)
    assert f(ctypes.byref(d), ctypes.byref(bad), FAKE, ws_bytes, None, ev, L.MAX_KERNELS + 1, names,
             ctypes.byref(n)) == -4
    assert n.value == 0
    # the per-launch pair form: every one of its 2·RWKVMOE_MAX_KERNELS events must be given
    pairs_null = (ctypes.c_void_p * L.TIMED_PAIR_EVENTS)(*([FAKE] * (L.TIMED_PAIR_EVENTS - 1)))
    assert f(ctypes.byref(d), ctypes.byref(t), FAKE, ws_bytes, None, pairs_null, L.TIMED_PAIR_EVENTS, names,
             ctypes.byref(n)) == -10
    pairs = (ctypes.c_void_p * L.TIMED_PAIR_EVENTS)(*([FAKE] * L.TIMED_PAIR_EVENTS))
    assert f(ctypes.byref(d), ctypes.byref(bad), FAKE, ws_bytes, None, pairs, L.TIMED_PAIR_EVENTS, names,
             ctypes.byref(n)) == -4
    assert n.value == 0


@pytest.mark.parametrize("name,required", [
    ("rwkvmoe_router_topk", ("x", "w_gate")),
    ("rwkvmoe_dispatch", ("inds", "perm", "inv_perm", "offsets")),
    ("rwkvmoe_cmix_key", ("x", "x_k", "w_key", "hidden")),
    ("rwkvmoe_cmix_value", ("hidden", "w_value", "base_out")),
    ("rwkvmoe_lora_grouped", ("x", "lora_A", "lora_B", "perm", "offsets", "adapter_rows")),
    ("rwkvmoe_combine", ("base_out", "adapter_rows", "inds", "gates", "out")),
    ("rwkvmoe_ortho_loss", ("lora_A", "ortho_loss")),
])
def test_stage_entry_points_require_their_tensors(L, name, required):
    d = desc(L)
    for miss in required:
        kw = {n: FAKE + (i << 24) for i, n in enumerate(required) if n != miss}
        t = L.make_tensors(**kw)
        assert call_status(L, name, d, t) == -4, (name, miss)
    # and reject a bad descriptor the same way the forward does
    t = L.make_tensors(**{n: FAKE + (i << 24) for i, n in enumerate(required)})
    assert call_status(L, name, desc(L, dtype=7), t, ws_bytes=1 << 30) == -3


def test_error_object_names_status(L):
    e = L.RwkvMoeError(-6, "rwkvmoe_forward")
    assert "RWKVMOE_ERR_WORKSPACE" in str(e) and e.status == -6


# ---- the torch mirror refuses CPU tensors (no CPU fallback) -----------------------

def test_module_refuses_cpu_tensors(L):
    import torch

    from rwkv_mlx_amd.model import RWKV_CMix_x070, RWKVConfig
    from rwkv_mlx_amd.moe import LoRAMoE_CMix, Router
    cfg = RWKVConfig(n_embd=128, dim_ffn=512)
    base = RWKV_CMix_x070(cfg)
    moe = LoRAMoE_CMix(base, n_experts=4, lora_rank=8, top_k=2)
    x = torch.randn(1, 4, 128)
    with pytest.raises(RuntimeError, match="GPU only"):
        moe(x)
    with pytest.raises(RuntimeError, match="GPU only"):
        base(x)
    with pytest.raises(RuntimeError, match="GPU only"):
        Router(128, 4, 2)(x)


def test_module_parameter_layout_matches_reference(L):
    """Parameter names and shapes of moe.py:45-49, 111-127 and model.py:253-257."""
    from rwkv_mlx_amd.model import RWKV_CMix_x070, RWKVConfig
    from rwkv_mlx_amd.moe import LoRAMoE_CMix
    cfg = RWKVConfig(n_embd=128, dim_ffn=512)
    moe = LoRAMoE_CMix(RWKV_CMix_x070(cfg), n_experts=4, lora_rank=8, top_k=2)
    shapes = {n: tuple(p.shape) for n, p in moe.named_parameters()}
    assert shapes == {
        "base.x_k": (1, 1, 128), "base.key.weight": (512, 128), "base.value.weight": (128, 512),
        "lora_A": (4, 128, 8), "lora_B": (4, 8, 128), "router.gate.weight": (4, 128),
    }
    assert float(moe.lora_B.detach().abs().sum()) == 0.0  # moe.py:125 initialises B to zeros


# ---- backward entry point validation (host only) --------------------------------

def fake_grads(L, **override):
    names = ("x", "w_gate", "lora_A", "lora_B", "logits", "inds", "d_out", "d_x", "d_lora_A", "d_lora_B", "d_w_gate")
    kw = {n: FAKE + (i << 24) for i, n in enumerate(names)}
    kw.update(override)
    g = L.Grads()
    for k, v in kw.items():
        if v is not None:
            setattr(g, k, v)
    return g


def bwd_ws(L, d):
    n = ctypes.c_size_t(0)
    return L.lib().rwkvmoe_backward_workspace_bytes(ctypes.byref(d), ctypes.byref(n)), n.value


def bwd_status(L, d, g, ws=FAKE + (1 << 32), ws_bytes=None):
    if ws_bytes is None:
        st, ws_bytes = bwd_ws(L, d)
        ws_bytes = ws_bytes if st == 0 else 0
    return L.lib().rwkvmoe_backward(ctypes.byref(d) if d is not None else None,
                                    ctypes.byref(g) if g is not None else None, ws, ctypes.c_size_t(ws_bytes), None)


def test_backward_workspace_sizes(L):
    st, n = bwd_ws(L, desc(L))
    assert st == 0 and n % 256 == 0
    N, C, kx = 4096, 768, 128
    # 16-bit layer on the fused routing path: at least DSd, SGd, dℓ (row-major) and the expert masks
    assert n >= 2 * N * kx * 2 + N * 128 * 2 + N * 8
    # fp32 layer (dense path): at least the two transposed token operands and S, G, DSd
    st, n32 = bwd_ws(L, desc(L, dtype="f32"))
    assert st == 0 and n32 % 256 == 0
    assert n32 >= 2 * C * N * 4 + 3 * N * kx * 4
    assert bwd_ws(L, desc(L, d_model=96))[0] == -2
    assert L.lib().rwkvmoe_backward_workspace_bytes(None, ctypes.byref(ctypes.c_size_t(0))) == -1
    assert L.lib().rwkvmoe_backward_workspace_bytes(ctypes.byref(desc(L)), None) == -4


def test_backward_argument_errors(L):
    d = desc(L)
    assert bwd_status(L, None, fake_grads(L), ws_bytes=1 << 30) == -1
    assert bwd_status(L, d, None) == -1
    for missing in ("x", "w_gate", "lora_A", "lora_B", "logits", "inds", "d_out"):
        assert bwd_status(L, d, fake_grads(L, **{missing: None})) == -4, missing
    for field, off in (("x", 8), ("d_out", 4), ("logits", 2), ("d_x", 8), ("d_lora_A", 1), ("d_w_gate", 2)):
        assert bwd_status(L, d, fake_grads(L, **{field: FAKE + off})) == -5, field
    need = bwd_ws(L, d)[1]
    assert bwd_status(L, d, fake_grads(L), ws=None, ws_bytes=need) == -6
    assert bwd_status(L, d, fake_grads(L), ws_bytes=need - 1) == -6


# ---- full-expert entry point validation (host only) -----------------------------

def test_experts_entry_validation(L):
    d = desc(L, lora_rank=1)
    n = ctypes.c_size_t(0)
    assert L.lib().rwkvmoe_experts_workspace_bytes(ctypes.byref(d), ctypes.byref(n)) == 0
    N, C, F, k, s = 4096, 768, 3072, 2, 2
    # at least the gathered mixed rows, the hidden rows and the expert outputs
    assert n.value >= N * k * (C + F + C) * s
    assert L.lib().rwkvmoe_experts_workspace_bytes(None, ctypes.byref(n)) == -1
    assert L.lib().rwkvmoe_experts_workspace_bytes(ctypes.byref(d), None) == -4
    big = desc(L, batch=1 << 12, seq_len=1 << 8, d_ffn=4096, lora_rank=1, top_k=2)  # N*k*F >= 2^31
    assert L.lib().rwkvmoe_experts_workspace_bytes(ctypes.byref(big), ctypes.byref(n)) == -2
    ws = n.value if L.lib().rwkvmoe_experts_workspace_bytes(ctypes.byref(d), ctypes.byref(n)) == 0 else 0
    fn = L.lib().rwkvmoe_experts_forward
    for missing in ("x", "x_k", "w_key", "w_value", "w_gate", "out", "losses"):
        t = fake_tensors(L, **{missing: None})
        assert fn(ctypes.byref(d), ctypes.byref(t), FAKE + (1 << 32), ctypes.c_size_t(ws), None) == -4, missing
    t = fake_tensors(L, x=FAKE + 8)
    assert fn(ctypes.byref(d), ctypes.byref(t), FAKE + (1 << 32), ctypes.c_size_t(ws), None) == -5
    t = fake_tensors(L)
    assert fn(ctypes.byref(d), ctypes.byref(t), FAKE + (1 << 32), ctypes.c_size_t(ws - 1), None) == -6
    assert fn(ctypes.byref(d), ctypes.byref(t), None, ctypes.c_size_t(ws), None) == -6


def test_experts_backward_validation(L):
    """rwkvmoe_experts_backward_workspace_bytes and the argument errors of
    rwkvmoe_experts_backward, all found on the host."""
    d = desc(L, lora_rank=1)
    n = ctypes.c_size_t(0)
    assert L.lib().rwkvmoe_experts_backward_workspace_bytes(ctypes.byref(d), ctypes.byref(n)) == 0
    N, C, F, E, k, s = 4096, 768, 3072, 8, 2, 2
    # at least the routed rows' xk, p, u and dk, and two transposed operands over the packed token ranges
    assert n.value % 256 == 0 and n.value >= N * k * (2 * C + 2 * F) * s + 2 * F * N * k * s
    ws = n.value
    assert L.lib().rwkvmoe_experts_backward_workspace_bytes(None, ctypes.byref(n)) == -1
    assert L.lib().rwkvmoe_experts_backward_workspace_bytes(ctypes.byref(d), None) == -4
    dg = desc(L, lora_rank=1, flags=L.GATE_F32)
    assert L.lib().rwkvmoe_experts_backward_workspace_bytes(ctypes.byref(dg), ctypes.byref(n)) == -3
    big = desc(L, batch=1 << 10, seq_len=1 << 9, lora_rank=1)  # (N·k + 128·E) · F beyond 2^31
    assert L.lib().rwkvmoe_experts_backward_workspace_bytes(ctypes.byref(big), ctypes.byref(n)) == -2
    names = ("x", "x_k", "w_key", "w_value", "w_gate", "logits", "inds", "d_out", "d_x", "d_x_k", "d_w_key",
             "d_w_value", "d_w_gate")

    def grads(**override):
        kw = {nm: FAKE + (i << 24) for i, nm in enumerate(names)}
        kw.update(override)
        g = L.ExpertsGrads()
        for key, v in kw.items():
            if v is not None:
                setattr(g, key, v)
        return g

    fn = L.lib().rwkvmoe_experts_backward

    def st(g, dd=d, w=FAKE + (1 << 32), nb=ws):
        return fn(ctypes.byref(dd) if dd is not None else None, ctypes.byref(g) if g is not None else None, w,
                  ctypes.c_size_t(nb), None)

    assert st(grads(), dd=None) == -1
    assert st(None) == -1
    for missing in ("x", "x_k", "w_key", "w_value", "w_gate", "logits", "inds", "d_out"):
        assert st(grads(**{missing: None})) == -4, missing
    for field, off in (("x", 8), ("logits", 2), ("d_out", 4), ("d_w_key", 8), ("d_x_k", 2)):
        assert st(grads(**{field: FAKE + off})) == -5, field
    assert st(grads(d_x_prev=FAKE + (40 << 24))) == -8  # d_x_prev without RWKVMOE_HAS_PREV
    dp = desc(L, lora_rank=1, flags=L.HAS_PREV)
    assert st(grads(), dd=dp) == -4                      # HAS_PREV without x_prev
    assert st(grads(), nb=ws - 1) == -6
    assert st(grads(), w=None) == -6
    assert st(grads(), dd=dg) == -3


def test_gates_f16_flag_is_backward_only(L):
    """RWKVMOE_GATES_F16 (the fine-tune layer's fp32 VJP with fp16 gates):
    accepted by the backward at dtype F32 only; every forward entry point and
    a 16-bit backward reject it."""
    n = ctypes.c_size_t(0)
    d = desc(L, dtype="f32", flags=L.GATES_F16)
    assert L.lib().rwkvmoe_backward_workspace_bytes(ctypes.byref(d), ctypes.byref(n)) == 0
    d16 = desc(L, flags=L.GATES_F16)
    assert L.lib().rwkvmoe_backward_workspace_bytes(ctypes.byref(d16), ctypes.byref(n)) == -8
    assert ws_status(L, d)[0] == -8
    assert L.lib().rwkvmoe_experts_workspace_bytes(ctypes.byref(desc(L, dtype="f32", flags=L.GATES_F16, lora_rank=1)),
                                                   ctypes.byref(n)) == -8
    assert call_status(L, "rwkvmoe_forward", d, fake_tensors(L), ws_bytes=1 << 30) == -8


def test_ln_flag(L):
    """RWKVMOE_LN_IN (ln2 in front of the layer): the forwards need ln_weight
    and ln_bias (16-byte aligned), the workspace holds LN(x) (N·C elements);
    the backwards and the stage entry points reject the flag."""
    n = ctypes.c_size_t(0)
    d = desc(L, flags=L.LN_IN)
    base, ln = ws_status(L, desc(L)), ws_status(L, d)
    N, C = HEADLINE["batch"] * HEADLINE["seq_len"], HEADLINE["d_model"]
    assert base[0] == 0 and ln[0] == 0 and ln[1] - base[1] == (N * C * 2 + 255) // 256 * 256
    assert call_status(L, "rwkvmoe_forward", d, fake_tensors(L)) == -8
    assert call_status(L, "rwkvmoe_forward", d, fake_tensors(L, ln_weight=FAKE + (30 << 24))) == -8
    assert call_status(L, "rwkvmoe_forward", d, fake_tensors(L, ln_weight=FAKE + (30 << 24),
                                                            ln_bias=FAKE + (31 << 24) + 8)) == -5
    assert call_status(L, "rwkvmoe_experts_forward", desc(L, flags=L.LN_IN, lora_rank=1), fake_tensors(L)) == -8
    for entry in ("rwkvmoe_router_topk", "rwkvmoe_lora_grouped", "rwkvmoe_cmix_key"):
        t = fake_tensors(L, ln_weight=FAKE + (30 << 24), ln_bias=FAKE + (31 << 24))
        assert call_status(L, entry, d, t) == -8, entry
    assert L.lib().rwkvmoe_backward_workspace_bytes(ctypes.byref(d), ctypes.byref(n)) == -8
    assert L.lib().rwkvmoe_experts_backward_workspace_bytes(ctypes.byref(desc(L, flags=L.LN_IN, lora_rank=1)),
                                                            ctypes.byref(n)) == -8
    e0, e1 = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert L.lib().rwkvmoe_experts_workspace_bytes(ctypes.byref(desc(L, lora_rank=1)), ctypes.byref(e0)) == 0
    assert L.lib().rwkvmoe_experts_workspace_bytes(ctypes.byref(desc(L, flags=L.LN_IN, lora_rank=1)),
                                                   ctypes.byref(e1)) == 0
    assert e1.value - e0.value == (N * C * 2 + 255) // 256 * 256


def test_lora_valu_flag(L):
    """RWKVMOE_LORA_VALU (the grouped adapter products on the vector ALUs):
    accepted in either mode and every dtype with the same workspace size,
    rejected together with RWKVMOE_ADAPTERS_F32."""
    for dt in ("f32", "f16", "bf16"):
        for mode in (0, 1):
            assert ws_status(L, desc(L, dtype=dt, mode=mode, flags=L.LORA_VALU)) == \
                ws_status(L, desc(L, dtype=dt, mode=mode))
    assert ws_status(L, desc(L, mode=1, flags=L.LORA_VALU | L.ADAPTERS_F32))[0] == -8
    assert ws_status(L, desc(L, mode=1, flags=L.LORA_VALU | L.GATE_F32 | L.ADAPTERS_F32))[0] == -8


def test_ortho_backward_validation(L):
    d = desc(L)
    g = L.Grads()
    assert L.lib().rwkvmoe_ortho_backward(ctypes.byref(d), ctypes.byref(g), FAKE, ctypes.c_size_t(1 << 30), None) == -4
    g.lora_A = FAKE
    assert L.lib().rwkvmoe_ortho_backward(ctypes.byref(d), ctypes.byref(g), FAKE, ctypes.c_size_t(1 << 30), None) == -4
    g.d_lora_A = FAKE + 1
    assert L.lib().rwkvmoe_ortho_backward(ctypes.byref(d), ctypes.byref(g), FAKE, ctypes.c_size_t(1 << 30), None) == -5


def test_mixed_dtype_workspace_and_flags(L):
    """fp32 adapters on an fp16 layer: A_all / B_all / U in their fp16 pair
    forms need more workspace; the flags are no-ops on an fp32 layer."""
    base = ws_status(L, desc(L))
    mixed = ws_status(L, desc(L, flags=L.GATE_F32 | L.ADAPTERS_F32))
    assert base[0] == 0 and mixed[0] == 0 and mixed[1] > base[1]
    f32 = ws_status(L, desc(L, dtype=0))
    f32m = ws_status(L, desc(L, dtype=0, flags=L.GATE_F32 | L.ADAPTERS_F32))
    assert f32 == f32m
    gate_only = ws_status(L, desc(L, flags=L.GATE_F32))
    assert gate_only == base


def test_bf16_fp32_adapters_take_fp32_rows(L):
    """fp32 adapters beside a bf16 base run as fp32 adapter rows (SPARSE)
    whatever the mode: both modes need the same workspace, which holds the
    fp32 copy of x (N·C·4 bytes) and the fp32 rows beyond the bf16 SPARSE
    layer's (less the router's adapter product u, N·kx·2 bytes, which the
    bf16 SPARSE layer holds for its on-chip adapters at E·r = 128 and the
    fp32-adapter layer does not use); the prepared adapters are A_all / B_all
    in fp32."""
    sp = ws_status(L, desc(L, dtype=2, mode=1))
    fu = ws_status(L, desc(L, dtype=2, mode=0, flags=L.GATE_F32 | L.ADAPTERS_F32))
    sp32 = ws_status(L, desc(L, dtype=2, mode=1, flags=L.GATE_F32 | L.ADAPTERS_F32))
    assert sp[0] == fu[0] == sp32[0] == 0 and fu == sp32
    N, C, k = HEADLINE["batch"] * HEADLINE["seq_len"], HEADLINE["d_model"], HEADLINE["top_k"]
    kx_u = -(-HEADLINE["n_experts"] * HEADLINE["lora_rank"] // 128) * 128
    assert sp32[1] >= sp[1] - N * kx_u * 2 + N * C * 4 + N * k * C * 2
    n = ctypes.c_size_t(0)
    assert L.lib().rwkvmoe_prepared_bytes(ctypes.byref(desc(L, dtype=2, flags=L.ADAPTERS_F32)), ctypes.byref(n)) == 0
    kx = -(-HEADLINE["n_experts"] * HEADLINE["lora_rank"] // 128) * 128
    assert n.value >= 2 * kx * C * 4


def test_prepare_base_bytes_and_argument_errors(L):
    """rwkvmoe_prepared_base_bytes: W_key and W_value, 2·F·C elements of the
    16-bit dtype (fp32 layers: RWKVMOE_ERR_DTYPE); rwkvmoe_prepare_base
    reports its argument errors on the host."""
    d = desc(L)
    n = ctypes.c_size_t(0)
    assert L.lib().rwkvmoe_prepared_base_bytes(ctypes.byref(d), ctypes.byref(n)) == 0
    assert n.value == 2 * d.d_model * d.d_ffn * 2
    d32 = desc(L, dtype=0)
    assert L.lib().rwkvmoe_prepared_base_bytes(ctypes.byref(d32), ctypes.byref(n)) == -3
    assert L.lib().rwkvmoe_prepared_base_bytes(ctypes.byref(d), None) == -4
    f = L.lib().rwkvmoe_prepare_base
    fake = 1 << 20  # never dereferenced: every call below fails on the host
    need = 2 * d.d_model * d.d_ffn * 2
    assert f(ctypes.byref(d), None, fake, fake, need, None) == -4
    assert f(ctypes.byref(d), fake, fake, None, need, None) == -4
    assert f(ctypes.byref(d), fake, fake, fake, need - 1, None) == -6
    assert f(ctypes.byref(d), fake, fake, fake + 16, need, None) == -6   # not 256-byte aligned
    assert f(ctypes.byref(d), fake + 2, fake, fake, need, None) == -5    # not 16-byte aligned
    assert f(ctypes.byref(d32), fake, fake, fake, need, None) == -3
    assert f(None, fake, fake, fake, need, None) == -1


def test_prepare_adapters_argument_errors(L):
    """rwkvmoe_prepare_adapters reports its argument errors on the host."""
    d = desc(L)
    n = ctypes.c_size_t(0)
    assert L.lib().rwkvmoe_prepared_bytes(ctypes.byref(d), ctypes.byref(n)) == 0 and n.value > 0
    nm = ctypes.c_size_t(0)
    dm = desc(L, flags=L.ADAPTERS_F32)
    assert L.lib().rwkvmoe_prepared_bytes(ctypes.byref(dm), ctypes.byref(nm)) == 0 and nm.value > n.value
    f = L.lib().rwkvmoe_prepare_adapters
    fake = 1 << 20  # never dereferenced: every call below fails on the host
    assert f(ctypes.byref(d), None, fake, fake, n.value, None) == -4
    assert f(ctypes.byref(d), fake, fake, None, n.value, None) == -4
    assert f(ctypes.byref(d), fake, fake, fake, n.value - 1, None) == -6
    assert f(ctypes.byref(d), fake, fake, fake + 16, n.value, None) == -6   # not 256-byte aligned
    assert f(None, fake, fake, fake, n.value, None) == -1


def test_router_backward_validation(L):
    """rwkvmoe_router_backward: workspace sizes, flags (only HAS_BIAS), the
    required operands and alignment, all on the host."""
    d = desc(L)
    n = ctypes.c_size_t(0)
    f = L.lib().rwkvmoe_router_backward_workspace_bytes
    assert f(ctypes.byref(d), ctypes.byref(n)) == 0 and n.value > 0
    assert f(ctypes.byref(desc(L, flags=L.HAS_BIAS)), ctypes.byref(n)) == 0
    for fl in (L.HAS_PREV, L.ADD_RESIDUAL, L.GATE_F32, L.LN_IN):
        assert f(ctypes.byref(desc(L, flags=fl)), ctypes.byref(n)) == -8, fl
    assert f(ctypes.byref(d), None) == -4
    need = n.value
    b = L.lib().rwkvmoe_router_backward

    def g(**over):
        kw = dict(x=FAKE, w_gate=FAKE + (1 << 24), logits=FAKE + (2 << 24), inds=FAKE + (3 << 24),
                  d_x=FAKE + (4 << 24), d_w_gate=FAKE + (5 << 24))
        kw.update(over)
        gr = L.RouterGrads()
        for k_, v in kw.items():
            setattr(gr, k_, v)
        return gr

    ws = FAKE + (6 << 24)
    f(ctypes.byref(d), ctypes.byref(n))
    for miss in ("x", "w_gate", "logits", "inds"):
        assert b(ctypes.byref(d), ctypes.byref(g(**{miss: None})), ws, need, None) == -4, miss
    assert b(ctypes.byref(d), ctypes.byref(g(x=FAKE + 8)), ws, need, None) == -5
    assert b(ctypes.byref(d), ctypes.byref(g(d_gates=FAKE + 1)), ws, need, None) == -5
    assert b(ctypes.byref(d), ctypes.byref(g()), ws, need - 1, None) == -6
    assert b(ctypes.byref(d), ctypes.byref(g()), None, need, None) == -6
    assert b(None, ctypes.byref(g()), ws, need, None) == -1
    assert b(ctypes.byref(d), None, ws, need, None) == -1


def test_layer_norm_backward_validation(L):
    """rwkvmoe_layer_norm_backward: workspace size (the column partials:
    one fp32 row pair per workgroup, at most 1024 workgroups), any desc the
    forward takes, the required operands and alignment, all on the host."""
    d = desc(L, flags=L.LN_IN | L.ADD_RESIDUAL)
    n = ctypes.c_size_t(0)
    f = L.lib().rwkvmoe_layer_norm_backward_workspace_bytes
    assert f(ctypes.byref(d), ctypes.byref(n)) == 0
    N, C = HEADLINE["batch"] * HEADLINE["seq_len"], HEADLINE["d_model"]
    assert n.value == min((N + 15) // 16, 1024) * 2 * C * 4
    big = desc(L, batch=64, seq_len=4096)
    assert f(ctypes.byref(big), ctypes.byref(n)) == 0 and n.value == 1024 * 2 * C * 4
    assert f(ctypes.byref(desc(L, dtype=7)), ctypes.byref(n)) == -3
    assert f(ctypes.byref(d), None) == -4
    f(ctypes.byref(d), ctypes.byref(n))
    need = n.value
    b = L.lib().rwkvmoe_layer_norm_backward

    def g(**over):
        kw = dict(x=FAKE, ln_weight=FAKE + (1 << 24), d_y=FAKE + (2 << 24), d_x=FAKE + (3 << 24),
                  d_ln_weight=FAKE + (4 << 24), d_ln_bias=FAKE + (5 << 24))
        kw.update(over)
        gr = L.LnGrads()
        for k_, v in kw.items():
            setattr(gr, k_, v)
        return gr

    ws = FAKE + (6 << 24)
    for miss in ("x", "ln_weight", "d_y"):
        assert b(ctypes.byref(d), ctypes.byref(g(**{miss: None})), ws, need, None) == -4, miss
    assert b(ctypes.byref(d), ctypes.byref(g(x=FAKE + 8)), ws, need, None) == -5
    assert b(ctypes.byref(d), ctypes.byref(g(d_res=FAKE + 8)), ws, need, None) == -5
    assert b(ctypes.byref(d), ctypes.byref(g(d_ln_bias=FAKE + 1)), ws, need, None) == -5
    assert b(ctypes.byref(d), ctypes.byref(g()), ws, need - 1, None) == -6
    assert b(ctypes.byref(d), ctypes.byref(g()), None, need, None) == -6
    assert b(ctypes.byref(d), ctypes.byref(g()), ws + 128, need, None) == -6
    # no column sums asked for: no workspace needed; no output at all: nothing to do
    assert b(ctypes.byref(d), ctypes.byref(g(d_x=None, d_ln_weight=None, d_ln_bias=None)), None, 0, None) == 0
    assert b(None, ctypes.byref(g()), ws, need, None) == -1
    assert b(ctypes.byref(d), None, ws, need, None) == -1
