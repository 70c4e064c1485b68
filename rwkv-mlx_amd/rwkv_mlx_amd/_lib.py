"""ctypes binding of librwkvmoe.so (the C ABI declared in include/rwkvmoe.h).

PyTorch is only plumbing here: it owns device memory and the stream.  torch
is imported before the library is loaded so that the library binds to the
HIP runtime torch already has in the process.  There is no CPU fallback:
if the library is missing, every call raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "librwkvmoe.so"

F32, F16, BF16 = 0, 1, 2
MODE_FUSED, MODE_SPARSE = 0, 1
HAS_PREV, HAS_BIAS, ADD_RESIDUAL = 1, 2, 4
GATE_F32, ADAPTERS_F32, GATES_F16, LORA_VALU, LN_IN = 8, 16, 32, 64, 128

TORCH_DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}
NAME_DTYPE_CODE = {"f32": F32, "f16": F16, "bf16": BF16}
MODES = {"fused": MODE_FUSED, "sparse": MODE_SPARSE}

ENTRY_POINTS = (
    "rwkvmoe_status_string",
    "rwkvmoe_version",
    "rwkvmoe_workspace_bytes",
    "rwkvmoe_prepared_bytes",
    "rwkvmoe_prepare_adapters",
    "rwkvmoe_prepared_base_bytes",
    "rwkvmoe_prepare_base",
    "rwkvmoe_reads_prepared_base",
    "rwkvmoe_forward",
    "rwkvmoe_forward_noalloc",
    "rwkvmoe_decode",
    "rwkvmoe_forward_timed",
    "rwkvmoe_router_topk",
    "rwkvmoe_dispatch",
    "rwkvmoe_cmix_key",
    "rwkvmoe_cmix_value",
    "rwkvmoe_lora_grouped",
    "rwkvmoe_combine",
    "rwkvmoe_ortho_loss",
    "rwkvmoe_backward_workspace_bytes",
    "rwkvmoe_backward",
    "rwkvmoe_ortho_backward",
    "rwkvmoe_router_backward_workspace_bytes",
    "rwkvmoe_router_backward",
    "rwkvmoe_layer_norm_backward_workspace_bytes",
    "rwkvmoe_layer_norm_backward",
    "rwkvmoe_experts_workspace_bytes",
    "rwkvmoe_experts_forward",
    "rwkvmoe_experts_backward_workspace_bytes",
    "rwkvmoe_experts_backward",
)
STAGE_ENTRY_POINTS = ("rwkvmoe_forward", "rwkvmoe_decode", "rwkvmoe_router_topk", "rwkvmoe_dispatch",
                      "rwkvmoe_cmix_key", "rwkvmoe_cmix_value", "rwkvmoe_lora_grouped", "rwkvmoe_combine",
                      "rwkvmoe_ortho_loss", "rwkvmoe_experts_forward")
MAX_KERNELS = 16
TIMED_PAIR_EVENTS = 2 * MAX_KERNELS

STATUS = {
    0: "RWKVMOE_OK", -1: "RWKVMOE_ERR_NULL_DESC", -2: "RWKVMOE_ERR_SHAPE", -3: "RWKVMOE_ERR_DTYPE",
    -4: "RWKVMOE_ERR_NULL_PTR", -5: "RWKVMOE_ERR_ALIGN", -6: "RWKVMOE_ERR_WORKSPACE", -7: "RWKVMOE_ERR_TOPK",
    -8: "RWKVMOE_ERR_FLAGS", -9: "RWKVMOE_ERR_MODE", -10: "RWKVMOE_ERR_EVENTS", -11: "RWKVMOE_ERR_SCRATCH",
    -12: "RWKVMOE_ERR_VERSION",
}
NOALLOC_SCRATCH_BYTES = 64 << 20


class Desc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "batch", "seq_len", "d_model", "d_ffn", "n_experts", "top_k", "lora_rank", "dtype", "mode", "flags")]


class Tensors(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint64)] + [(n, ctypes.c_void_p) for n in (
        "x", "x_prev", "x_k", "w_key", "w_value", "w_gate", "lora_A", "lora_B", "logit_bias", "residual",
        "out", "losses", "logits", "inds", "gates", "gate_dense", "perm", "inv_perm", "offsets",
        "hidden", "base_out", "adapter_rows", "ortho_loss", "prepared", "prepared_base",
        "ln_weight", "ln_bias", "x_ln")]


class Grads(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "x", "w_gate", "lora_A", "lora_B", "logits", "inds", "d_out", "d_losses",
        "d_x", "d_lora_A", "d_lora_B", "d_w_gate", "d_ortho")]


class ExpertsGrads(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "x", "x_prev", "x_k", "w_key", "w_value", "w_gate", "logits", "inds", "d_out", "d_losses",
        "d_x", "d_x_prev", "d_x_k", "d_w_key", "d_w_value", "d_w_gate")]


class RouterGrads(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "x", "w_gate", "logits", "inds", "d_gates", "d_losses", "d_x", "d_w_gate")]


class LnGrads(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "x", "ln_weight", "d_y", "d_res", "d_x", "d_ln_weight", "d_ln_bias")]


class RwkvMoeError(RuntimeError):
    def __init__(self, status: int, where: str):
        self.status = status
        name = STATUS.get(status, "hipError" if status > 0 else "unknown")
        super().__init__(f"{where} failed: {name} ({status}): {status_string(status)}")


_LIB: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Load librwkvmoe.so once; raise if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it first (python -m rwkv_mlx_amd.build)")
        h = ctypes.CDLL(str(LIB_PATH))
        h.rwkvmoe_status_string.restype = ctypes.c_char_p
        h.rwkvmoe_status_string.argtypes = [ctypes.c_int]
        h.rwkvmoe_version.restype = ctypes.c_int
        h.rwkvmoe_version.argtypes = []
        h.rwkvmoe_workspace_bytes.restype = ctypes.c_int
        h.rwkvmoe_workspace_bytes.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(ctypes.c_size_t)]
        for name in STAGE_ENTRY_POINTS:
            f = getattr(h, name)
            f.restype = ctypes.c_int
            f.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(Tensors), ctypes.c_void_p, ctypes.c_size_t,
                          ctypes.c_void_p]
        h.rwkvmoe_experts_workspace_bytes.restype = ctypes.c_int
        h.rwkvmoe_experts_workspace_bytes.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(ctypes.c_size_t)]
        for name in ("rwkvmoe_backward_workspace_bytes", "rwkvmoe_experts_backward_workspace_bytes",
                     "rwkvmoe_router_backward_workspace_bytes", "rwkvmoe_layer_norm_backward_workspace_bytes"):
            f = getattr(h, name)
            f.restype = ctypes.c_int
            f.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(ctypes.c_size_t)]
        h.rwkvmoe_experts_backward.restype = ctypes.c_int
        h.rwkvmoe_experts_backward.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(ExpertsGrads), ctypes.c_void_p,
                                               ctypes.c_size_t, ctypes.c_void_p]
        h.rwkvmoe_router_backward.restype = ctypes.c_int
        h.rwkvmoe_router_backward.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(RouterGrads), ctypes.c_void_p,
                                              ctypes.c_size_t, ctypes.c_void_p]
        h.rwkvmoe_layer_norm_backward.restype = ctypes.c_int
        h.rwkvmoe_layer_norm_backward.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(LnGrads), ctypes.c_void_p,
                                                  ctypes.c_size_t, ctypes.c_void_p]
        for name in ("rwkvmoe_backward", "rwkvmoe_ortho_backward"):
            f = getattr(h, name)
            f.restype = ctypes.c_int
            f.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(Grads), ctypes.c_void_p, ctypes.c_size_t,
                          ctypes.c_void_p]
        for name in ("rwkvmoe_prepared_bytes", "rwkvmoe_prepared_base_bytes"):
            f = getattr(h, name)
            f.restype = ctypes.c_int
            f.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(ctypes.c_size_t)]
        for name in ("rwkvmoe_prepare_adapters", "rwkvmoe_prepare_base"):
            f = getattr(h, name)
            f.restype = ctypes.c_int
            f.argtypes = [ctypes.POINTER(Desc), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                          ctypes.c_void_p]
        h.rwkvmoe_reads_prepared_base.restype = ctypes.c_int
        h.rwkvmoe_reads_prepared_base.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(ctypes.c_int)]
        h.rwkvmoe_forward_noalloc.restype = ctypes.c_int
        h.rwkvmoe_forward_noalloc.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(Tensors), ctypes.c_void_p]
        h.rwkvmoe_forward_timed.restype = ctypes.c_int
        h.rwkvmoe_forward_timed.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(Tensors), ctypes.c_void_p,
                                            ctypes.c_size_t, ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p),
                                            ctypes.c_int, ctypes.POINTER(ctypes.c_char_p),
                                            ctypes.POINTER(ctypes.c_int)]
        _LIB = h
    return _LIB


def status_string(status: int) -> str:
    return lib().rwkvmoe_status_string(status).decode()


def make_desc(batch, seq_len, d_model, d_ffn, n_experts, top_k, lora_rank, dtype, mode=MODE_FUSED, flags=0) -> Desc:
    if isinstance(dtype, torch.dtype):
        dtype = TORCH_DTYPE_CODE[dtype]
    elif isinstance(dtype, str):
        dtype = NAME_DTYPE_CODE[dtype]
    if isinstance(mode, str):
        mode = MODES[mode]
    return Desc(batch, seq_len, d_model, d_ffn, n_experts, top_k, lora_rank, dtype, mode, flags)


def workspace_bytes(desc: Desc) -> int:
    n = ctypes.c_size_t(0)
    st = lib().rwkvmoe_workspace_bytes(ctypes.byref(desc), ctypes.byref(n))
    if st != 0:
        raise RwkvMoeError(st, "rwkvmoe_workspace_bytes")
    return int(n.value)


def prepared_bytes(desc: Desc) -> int:
    n = ctypes.c_size_t(0)
    st = lib().rwkvmoe_prepared_bytes(ctypes.byref(desc), ctypes.byref(n))
    if st != 0:
        raise RwkvMoeError(st, "rwkvmoe_prepared_bytes")
    return int(n.value)


def prepare_adapters(desc: Desc, lora_A, lora_B, prepared, stream) -> None:
    """rwkvmoe_prepare_adapters into the uint8 device tensor `prepared`."""
    st = lib().rwkvmoe_prepare_adapters(ctypes.byref(desc), ptr(lora_A), ptr(lora_B), ptr(prepared),
                                        ctypes.c_size_t(prepared.numel()), stream)
    if st != 0:
        raise RwkvMoeError(st, "rwkvmoe_prepare_adapters")


def prepared_base_bytes(desc: Desc) -> int:
    n = ctypes.c_size_t(0)
    st = lib().rwkvmoe_prepared_base_bytes(ctypes.byref(desc), ctypes.byref(n))
    if st != 0:
        raise RwkvMoeError(st, "rwkvmoe_prepared_base_bytes")
    return int(n.value)


def prepare_base(desc: Desc, w_key, w_value, prepared, stream) -> None:
    """rwkvmoe_prepare_base into the uint8 device tensor `prepared`."""
    st = lib().rwkvmoe_prepare_base(ctypes.byref(desc), ptr(w_key), ptr(w_value), ptr(prepared),
                                    ctypes.c_size_t(prepared.numel()), stream)
    if st != 0:
        raise RwkvMoeError(st, "rwkvmoe_prepare_base")


def reads_prepared_base(desc: Desc) -> bool:
    """Whether a forward of `desc` reads rwkvmoe_tensors.prepared_base
    (rwkvmoe_reads_prepared_base; host only)."""
    n = ctypes.c_int(0)
    st = lib().rwkvmoe_reads_prepared_base(ctypes.byref(desc), ctypes.byref(n))
    if st != 0:
        raise RwkvMoeError(st, "rwkvmoe_reads_prepared_base")
    return n.value != 0


def experts_workspace_bytes(desc: Desc) -> int:
    n = ctypes.c_size_t(0)
    st = lib().rwkvmoe_experts_workspace_bytes(ctypes.byref(desc), ctypes.byref(n))
    if st != 0:
        raise RwkvMoeError(st, "rwkvmoe_experts_workspace_bytes")
    return int(n.value)


def backward_workspace_bytes(desc: Desc) -> int:
    n = ctypes.c_size_t(0)
    st = lib().rwkvmoe_backward_workspace_bytes(ctypes.byref(desc), ctypes.byref(n))
    if st != 0:
        raise RwkvMoeError(st, "rwkvmoe_backward_workspace_bytes")
    return int(n.value)


def backward(desc: Desc, ws, ws_bytes: int, stream, entry: str = "rwkvmoe_backward", **kw) -> None:
    """rwkvmoe_backward (or rwkvmoe_ortho_backward) with the named
    rwkvmoe_grads fields."""
    g = Grads()
    for k, v in kw.items():
        setattr(g, k, ptr(v))
    st = getattr(lib(), entry)(ctypes.byref(desc), ctypes.byref(g), ptr(ws), ctypes.c_size_t(ws_bytes), stream)
    if st != 0:
        raise RwkvMoeError(st, entry)


def router_backward_workspace_bytes(desc: Desc) -> int:
    n = ctypes.c_size_t(0)
    st = lib().rwkvmoe_router_backward_workspace_bytes(ctypes.byref(desc), ctypes.byref(n))
    if st != 0:
        raise RwkvMoeError(st, "rwkvmoe_router_backward_workspace_bytes")
    return int(n.value)


def router_backward(desc: Desc, ws, ws_bytes: int, stream, **kw) -> None:
    """rwkvmoe_router_backward with the named rwkvmoe_router_grads fields."""
    g = RouterGrads()
    for k, v in kw.items():
        setattr(g, k, ptr(v))
    st = lib().rwkvmoe_router_backward(ctypes.byref(desc), ctypes.byref(g), ptr(ws), ctypes.c_size_t(ws_bytes), stream)
    if st != 0:
        raise RwkvMoeError(st, "rwkvmoe_router_backward")


def layer_norm_backward_workspace_bytes(desc: Desc) -> int:
    n = ctypes.c_size_t(0)
    st = lib().rwkvmoe_layer_norm_backward_workspace_bytes(ctypes.byref(desc), ctypes.byref(n))
    if st != 0:
        raise RwkvMoeError(st, "rwkvmoe_layer_norm_backward_workspace_bytes")
    return int(n.value)


def layer_norm_backward(desc: Desc, ws, ws_bytes: int, stream, **kw) -> None:
    """rwkvmoe_layer_norm_backward with the named rwkvmoe_ln_grads fields."""
    g = LnGrads()
    for k, v in kw.items():
        setattr(g, k, ptr(v))
    st = lib().rwkvmoe_layer_norm_backward(ctypes.byref(desc), ctypes.byref(g), ptr(ws), ctypes.c_size_t(ws_bytes),
                                           stream)
    if st != 0:
        raise RwkvMoeError(st, "rwkvmoe_layer_norm_backward")


def experts_backward_workspace_bytes(desc: Desc) -> int:
    n = ctypes.c_size_t(0)
    st = lib().rwkvmoe_experts_backward_workspace_bytes(ctypes.byref(desc), ctypes.byref(n))
    if st != 0:
        raise RwkvMoeError(st, "rwkvmoe_experts_backward_workspace_bytes")
    return int(n.value)


def experts_backward(desc: Desc, ws, ws_bytes: int, stream, **kw) -> None:
    """rwkvmoe_experts_backward with the named rwkvmoe_experts_grads fields."""
    g = ExpertsGrads()
    for k, v in kw.items():
        setattr(g, k, ptr(v))
    st = lib().rwkvmoe_experts_backward(ctypes.byref(desc), ctypes.byref(g), ptr(ws), ctypes.c_size_t(ws_bytes),
                                        stream)
    if st != 0:
        raise RwkvMoeError(st, "rwkvmoe_experts_backward")


def ptr(t) -> int | None:
    """Device address of a tensor (None for None)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def make_tensors(**kw) -> Tensors:
    t = Tensors()
    t.struct_size = ctypes.sizeof(Tensors)
    for k, v in kw.items():
        setattr(t, k, ptr(v))
    return t


def forward_noalloc(desc: Desc, tensors: Tensors, stream) -> None:
    """rwkvmoe_forward_noalloc: the forward on the library's own device scratch."""
    st = lib().rwkvmoe_forward_noalloc(ctypes.byref(desc), ctypes.byref(tensors), stream)
    if st != 0:
        raise RwkvMoeError(st, "rwkvmoe_forward_noalloc")


def call(name: str, desc: Desc, tensors: Tensors, ws, ws_bytes: int, stream) -> None:
    """Invoke a stage entry point; raise RwkvMoeError on a non-zero status."""
    fn = getattr(lib(), name)
    st = fn(ctypes.byref(desc), ctypes.byref(tensors), ptr(ws), ctypes.c_size_t(ws_bytes), stream)
    if st != 0:
        raise RwkvMoeError(st, name)


class KernelTimer:
    """Runs rwkvmoe_forward_timed with `slots` sets of timing events on one
    stream and accumulates per-kernel durations (microseconds).

    pairs=True (default): each launch records its own begin and end
    timestamps (RWKVMOE_TIMED_PAIR_EVENTS events), so a duration is the
    kernel's alone, as a kernel trace reports it; launches of one step that
    share a name are summed.  pairs=False: events recorded on the stream
    between the steps; an interval then also holds the event records."""

    def __init__(self, stream, slots: int, pairs: bool = True):
        self.stream = stream
        self.pairs = pairs
        self.n_events = TIMED_PAIR_EVENTS if pairs else MAX_KERNELS + 1
        self.sets = []
        for _ in range(slots):
            evs = [torch.cuda.Event(enable_timing=True) for _ in range(self.n_events)]
            for e in evs:  # torch creates the HIP event on first record
                e.record(stream)
            self.sets.append(evs)
        torch.cuda.synchronize()
        self.used = []  # (set, names) per recorded forward

    def forward(self, desc: Desc, tensors: Tensors, ws, ws_bytes: int) -> None:
        evs = self.sets[len(self.used)]
        handles = (ctypes.c_void_p * self.n_events)(*[e.cuda_event for e in evs])
        names = (ctypes.c_char_p * MAX_KERNELS)()
        n = ctypes.c_int(0)
        st = lib().rwkvmoe_forward_timed(ctypes.byref(desc), ctypes.byref(tensors), ptr(ws), ctypes.c_size_t(ws_bytes),
                                         self.stream.cuda_stream, handles, self.n_events, names, ctypes.byref(n))
        if st != 0:
            raise RwkvMoeError(st, "rwkvmoe_forward_timed")
        self.used.append((evs, [names[i].decode() for i in range(n.value)]))

    def summary(self) -> list[tuple[str, float]]:
        """[(kernel name, mean microseconds per forward)] in launch order."""
        torch.cuda.synchronize()
        order: list[str] = []
        tot: dict[str, float] = {}
        for evs, names in self.used:
            for i, nm in enumerate(names):
                if nm not in tot:
                    order.append(nm)
                    tot[nm] = 0.0
                a, b = (evs[2 * i], evs[2 * i + 1]) if self.pairs else (evs[i], evs[i + 1])
                tot[nm] += a.elapsed_time(b) * 1e3
        return [(nm, tot[nm] / len(self.used)) for nm in order]


def current_stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
