"""Layer shapes of the LoRA-MoE ChannelMix forward and their seeded synthetic
inputs.

The five workloads are the shapes the path is measured and checked on: a
small fp32 layer, the 184M-model layer (D=768), a batched decode step, a wide
bf16 layer and a skewed-routing stress case.  Inputs follow the reference's
parameter shapes (rwkv_mlx/moe.py:113-127, rwkv_mlx/model.py:253-257) with
fixed distributions; draws are made in float64 in a fixed order from
``numpy.random.default_rng(seed)`` and then rounded to the layer dtype on the
host, so every consumer sees identical bits.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, replace

import numpy as np


@dataclass(frozen=True)
class LayerShape:
    name: str
    dtype: str          # "f32" | "f16" | "bf16"
    batch: int
    seq_len: int
    d_model: int
    d_ffn: int
    n_experts: int
    top_k: int
    lora_rank: int
    decode: bool = False          # RNN-mode step: seq_len == 1 with a carried shift state
    zipf_s: float | None = None   # router logit bias beta*ln(p_e), p_e ∝ (e+1)^-s
    bias_beta: float = 1.0
    seed: int = 1000

    @property
    def tokens(self) -> int:
        return self.batch * self.seq_len

    def scaled(self, batch: int | None = None, seq_len: int | None = None) -> "LayerShape":
        """Same layer with fewer tokens (for oracle-sized checks)."""
        return replace(self, batch=batch or self.batch, seq_len=seq_len or self.seq_len)


WORKLOADS: list[LayerShape] = [
    LayerShape("cmix-d512-e4-top1-r8-fp32", "f32", 1, 512, 512, 2048, 4, 1, 8, seed=1000),
    LayerShape("cmix-d768-e8-top2-r16-fp16", "f16", 8, 512, 768, 3072, 8, 2, 16, seed=1001),
    LayerShape("decode-d768-e8-top2-r16-fp16", "f16", 64, 1, 768, 3072, 8, 2, 16, decode=True, seed=1002),
    LayerShape("cmix-d2048-e16-top2-r32-bf16", "bf16", 16, 1024, 2048, 8192, 16, 2, 32, seed=1003),
    LayerShape("skew-d1024-e32-top4-r16-fp16", "f16", 8, 1024, 1024, 4096, 32, 4, 16, zipf_s=1.2, seed=1004),
]
BY_NAME = {w.name: w for w in WORKLOADS}
HEADLINE = WORKLOADS[1]


def _round_host(a: np.ndarray, dtype: str) -> np.ndarray:
    """Round float64 draws to the layer dtype on the host, returned as float32."""
    a32 = np.asarray(a, np.float32)
    if dtype == "f32":
        return a32
    if dtype == "f16":
        return a32.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        import torch
        return torch.from_numpy(np.ascontiguousarray(a32)).to(torch.bfloat16).to(torch.float32).numpy()
    raise ValueError(dtype)


def zipf_bias(E: int, s: float, beta: float = 1.0) -> np.ndarray:
    """bias_e = beta * ln p_e with p_e ∝ (e+1)^-s (one popular expert)."""
    p = np.array([(e + 1.0) ** -s for e in range(E)])
    p /= p.sum()
    return (beta * np.log(p)).astype(np.float32)


def make_inputs(w: LayerShape, seed: int | None = None) -> dict[str, np.ndarray]:
    """Seeded inputs: x, x_k, Wk, Wv, Wg, A, B (+ x_prev or bias), as float32
    arrays holding values exactly representable in ``w.dtype``.

    x ~ N(0,1); x_k ~ U(0,1); Wk ~ N(0, 1/√C); Wv ~ N(0, 1/√F);
    Wg ~ N(0, 1/√C); A ~ N(0, 1/√C); B ~ N(0, 0.02); x_prev ~ N(0,1)."""
    rng = np.random.default_rng(w.seed if seed is None else seed)
    B, T, C, F, E, r = w.batch, w.seq_len, w.d_model, w.d_ffn, w.n_experts, w.lora_rank
    d = w.dtype
    out = {
        "x": _round_host(rng.standard_normal((B, T, C)), d),
        "x_k": _round_host(rng.uniform(0.0, 1.0, (C,)), d),
        "Wk": _round_host(rng.standard_normal((F, C)) / math.sqrt(C), d),
        "Wv": _round_host(rng.standard_normal((C, F)) / math.sqrt(F), d),
        "Wg": _round_host(rng.standard_normal((E, C)) / math.sqrt(C), d),
        "A": _round_host(rng.standard_normal((E, C, r)) / math.sqrt(C), d),
        "B": _round_host(rng.standard_normal((E, r, C)) * 0.02, d),
    }
    if w.decode:
        out["x_prev"] = _round_host(rng.standard_normal((B, C)), d)
    if w.zipf_s is not None:
        out["bias"] = zipf_bias(E, w.zipf_s, w.bias_beta)
    return out
