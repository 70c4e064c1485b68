"""The base ChannelMix of RWKV-v7 on MI355X: a PyTorch mirror of the
reference's ``RWKV_CMix_x070`` (rwkv_mlx/model.py:243-263) and of the MoE
fields of ``RWKVConfig`` (rwkv_mlx/model.py:18-47), computing through
librwkvmoe's HIP kernels.

Parameter names and shapes are the reference's: ``x_k (1,1,C)``,
``key.weight (F,C)``, ``value.weight (C,F)``.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import nn

from . import _lib


@dataclass
class RWKVConfig:
    """The fields of rwkv_mlx/model.py:18-47 the ChannelMix path reads."""
    n_layer: int = 12
    n_embd: int = 768
    dim_ffn: int = 0                 # 0 -> int((n_embd * 3.5) // 32 * 32) (model.py:46-47)
    moe_num_experts: int = 0
    moe_top_k: int = 2
    moe_mode: str = "lora"
    moe_lora_rank: int = 64
    moe_layers: tuple = ()
    moe_aux_loss_coeff: float = 0.01
    moe_z_loss_coeff: float = 0.001
    moe_ortho_coeff: float = 0.001

    def __post_init__(self):
        if self.dim_ffn <= 0:
            self.dim_ffn = int((self.n_embd * 3.5) // 32 * 32)


def require_device(x: torch.Tensor, what: str) -> None:
    if not x.is_cuda:
        raise RuntimeError(f"{what}: rwkv_mlx_amd runs on the GPU only (got a {x.device} tensor); "
                           "there is no CPU fallback")


class Workspace:
    """Scratch buffer per (device, stream), reused across calls and grown on
    demand.  Every kernel of a call runs on the caller's current stream, so
    calls on one stream reuse the buffer in order; calls on different streams
    get different buffers and never race on scratch memory."""

    def __init__(self):
        self._buf: dict[tuple, torch.Tensor] = {}

    def get(self, device: torch.device, nbytes: int) -> torch.Tensor:
        key = (device, torch.cuda.current_stream(device).cuda_stream)
        b = self._buf.get(key)
        if b is None or b.numel() < nbytes:
            b = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
            self._buf[key] = b
        return b


_WS = Workspace()


class RWKV_CMix_x070(nn.Module):
    """RWKV-7 ChannelMix: value(relu(key(x + (shift(x) - x) * x_k)) ** 2).

    Mirrors rwkv_mlx/model.py:243-263; ``forward`` runs the shift-fused MFMA
    key GEMM (relu² epilogue) and the value GEMM of librwkvmoe."""

    def __init__(self, config: RWKVConfig, layer_id: int = 0):
        super().__init__()
        self.config = config
        self.layer_id = layer_id
        C = config.n_embd
        self.x_k = nn.Parameter(torch.zeros(1, 1, C))
        self.key = nn.Linear(C, config.dim_ffn, bias=False)
        self.value = nn.Linear(config.dim_ffn, C, bias=False)

    def forward(self, x: torch.Tensor, x_prev: torch.Tensor | None = None) -> torch.Tensor:
        require_device(x, "RWKV_CMix_x070")
        if x.dim() != 3:
            raise ValueError(f"RWKV_CMix_x070 expects (B, T, C), got {tuple(x.shape)}")
        B, T, C = x.shape
        # MLX type promotion: fp32 weights with an fp16 input compute in fp32
        dt = x.dtype
        for prm in (self.x_k, self.key.weight, self.value.weight):
            dt = torch.promote_types(dt, prm.dtype)
        if dt not in _lib.TORCH_DTYPE_CODE:
            raise TypeError(f"unsupported dtype {dt}; use float32, float16 or bfloat16")
        F = self.key.weight.shape[0]
        if B * T == 0:
            return torch.empty(B, T, C, dtype=dt, device=x.device)
        x = x.to(dt).contiguous()
        xk = self.x_k.detach().to(dt).reshape(C).contiguous()
        wk = self.key.weight.detach().to(dt).contiguous()
        wv = self.value.weight.detach().to(dt).contiguous()
        flags = _lib.HAS_PREV if x_prev is not None else 0
        desc = _lib.make_desc(B, T, C, F, 1, 1, 1, dt, _lib.MODE_FUSED, flags)
        nbytes = _lib.workspace_bytes(desc)
        ws = _WS.get(x.device, nbytes)
        hidden = torch.empty(B * T, F, dtype=dt, device=x.device)
        out = torch.empty_like(x)
        xp = x_prev.to(device=x.device, dtype=dt).contiguous() if x_prev is not None else None
        stream = _lib.current_stream(x.device)
        t = _lib.make_tensors(x=x, x_prev=xp, x_k=xk, w_key=wk, hidden=hidden)
        _lib.call("rwkvmoe_cmix_key", desc, t, ws, nbytes, stream)
        t = _lib.make_tensors(hidden=hidden, w_value=wv, base_out=out)
        _lib.call("rwkvmoe_cmix_value", desc, t, ws, nbytes, stream)
        return out
