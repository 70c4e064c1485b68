"""Shared helpers for the parity tests: device upload, C-ABI calls, oracle
evaluation on sampled token rows, and the tolerance checks.

Tolerances (outputs vs the oracle): max|got-ref| / max|ref| and
||got-ref||_2 / ||ref||_2 must both be <= 1e-5 for fp32 layers and
<= 2e-2 for fp16/bf16 layers.  Integer outputs (router indices, dispatch
permutation, offsets) and router logits must be bit-exact.
"""
from __future__ import annotations

import numpy as np

from oracle import moe_oracle as O

TOL = {"f32": 1e-5, "f16": 2e-2, "bf16": 2e-2}


def torch_dtype(name):
    import torch
    return {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[name]


def to_dev(a, dtype, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device=device, dtype=torch_dtype(dtype))


def to_np(t):
    return t.detach().float().cpu().numpy()


def rel_errs(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    mx = max(float(np.max(np.abs(ref))), 1e-30)
    nrm = max(float(np.linalg.norm(ref)), 1e-30)
    return float(np.max(d)) / mx, float(np.linalg.norm(got - ref)) / nrm


def assert_close(got, ref, dtype, what=""):
    tol = TOL[dtype]
    assert np.all(np.isfinite(got)), f"{what}: non-finite values"
    emax, enorm = rel_errs(got, ref)
    assert emax <= tol and enorm <= tol, f"{what}: max-rel {emax:.3e} norm-rel {enorm:.3e} > {tol}"
    return emax, enorm


class Layer:
    """One workload's inputs on the device plus a C-ABI runner."""

    def __init__(self, shape, device, inputs=None, mode="fused"):
        import torch
        from rwkv_mlx_amd import _lib
        from rwkv_mlx_amd.workloads import make_inputs
        self.w = shape
        self.dev = device
        self.np = inputs if inputs is not None else make_inputs(shape)
        d = shape.dtype
        self.dt = torch_dtype(d)
        g = self.np
        self.x = to_dev(g["x"], d, device)
        self.x_k = to_dev(g["x_k"], d, device)
        self.Wk = to_dev(g["Wk"], d, device)
        self.Wv = to_dev(g["Wv"], d, device)
        self.Wg = to_dev(g["Wg"], d, device)
        self.A = to_dev(g["A"], d, device)
        self.B = to_dev(g["B"], d, device)
        self.x_prev = to_dev(g["x_prev"], d, device) if "x_prev" in g else None
        self.bias = (torch.from_numpy(g["bias"]).to(device) if "bias" in g else None)
        flags = 0
        if self.x_prev is not None:
            flags |= _lib.HAS_PREV
        if self.bias is not None:
            flags |= _lib.HAS_BIAS
        self.flags = flags
        self.mode = mode
        self.desc = self.make_desc()
        self.ws_bytes = _lib.workspace_bytes(self.desc)
        self.ws = torch.empty(self.ws_bytes, dtype=torch.uint8, device=device)

    def make_desc(self, mode=None, flags=None):
        from rwkv_mlx_amd import _lib
        w = self.w
        return _lib.make_desc(w.batch, w.seq_len, w.d_model, w.d_ffn, w.n_experts, w.top_k, w.lora_rank, w.dtype,
                              mode or self.mode, self.flags if flags is None else flags)

    @property
    def N(self):
        return self.w.tokens

    def inputs(self):
        return dict(x=self.x, x_prev=self.x_prev, x_k=self.x_k, w_key=self.Wk, w_value=self.Wv, w_gate=self.Wg,
                    lora_A=self.A, lora_B=self.B, logit_bias=self.bias)

    def call(self, entry, desc=None, **tensors):
        import torch
        from rwkv_mlx_amd import _lib
        desc = desc or self.desc
        nbytes = _lib.workspace_bytes(desc)
        ws = self.ws if nbytes <= self.ws_bytes else torch.empty(nbytes, dtype=torch.uint8, device=self.dev)
        t = _lib.make_tensors(**tensors)
        _lib.call(entry, desc, t, ws, nbytes, _lib.current_stream(self.dev))

    def forward(self, mode=None, extras=False, residual=None, entry="rwkvmoe_forward"):
        import torch
        from rwkv_mlx_amd import _lib
        w = self.w
        out = torch.empty_like(self.x)
        losses = torch.empty(2, dtype=torch.float32, device=self.dev)
        ex = {}
        if extras:
            ex = dict(logits=torch.empty(self.N, w.n_experts, dtype=torch.float32, device=self.dev),
                      inds=torch.empty(self.N, w.top_k, dtype=torch.int32, device=self.dev),
                      gates=torch.empty(self.N, w.top_k, dtype=self.dt, device=self.dev),
                      perm=torch.empty(self.N * w.top_k, dtype=torch.int32, device=self.dev),
                      inv_perm=torch.empty(self.N * w.top_k, dtype=torch.int32, device=self.dev),
                      offsets=torch.empty(w.n_experts + 1, dtype=torch.int32, device=self.dev))
        flags = self.flags | (_lib.ADD_RESIDUAL if residual is not None else 0)
        desc = self.make_desc(mode=mode, flags=flags)
        self.call(entry, desc, out=out, losses=losses, residual=residual, **self.inputs(), **ex)
        torch.cuda.synchronize()
        return out, losses, ex


def sample_rows(N, T, n=256, seed=0):
    """Token rows to check at full size: sequence starts, ends and random rows."""
    rng = np.random.default_rng(seed)
    rows = set(rng.choice(N, size=min(n, N), replace=False).tolist())
    for s in range(0, N, T):
        if len(rows) > n + 64:
            break
        rows.add(s)
        rows.add(min(N - 1, s + T - 1))
    return np.array(sorted(rows))


def oracle_rows(g, shape, rows, router_out=None):
    """Oracle outputs (base, delta, out) for the given flat token rows.

    Each row is evaluated as a one-token sequence whose carried shift state
    is its true predecessor (zeros at a sequence start), which is exactly the
    reference's shift for that row."""
    w = shape
    C = w.d_model
    x = g["x"].reshape(-1, C)
    T = w.seq_len
    prev = np.zeros((rows.size, C), np.float32)
    for i, rr in enumerate(rows):
        t = rr % T
        if t > 0:
            prev[i] = x[rr - 1]
        elif "x_prev" in g:
            prev[i] = g["x_prev"][rr // T]
    xs = x[rows][:, None, :]
    base = O.cmix_base(xs, g["x_k"], g["Wk"], g["Wv"], w.dtype, x_prev=prev).reshape(-1, C)
    r = router_out or O.router(x, g["Wg"], w.top_k, w.dtype, g.get("bias"))
    delta = O.lora_delta_dense(x[rows], g["A"], g["B"], r["inds"][rows], r["gates"][rows], w.dtype)
    out = O.round_to(base + delta, w.dtype)
    return base, delta, out, r
