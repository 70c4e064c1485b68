"""rwkv_mlx_amd — the LoRA-MoE ChannelMix forward of RWKV-v7 (reference:
rwkv_mlx/moe.py, rwkv_mlx/model.py) on AMD Instinct MI355X.

The compute path is librwkvmoe.so: hand-written gfx950 HIP kernels behind the
C ABI in include/rwkvmoe.h, called through ctypes (``_lib``).  PyTorch-ROCm
provides device memory and the stream.
"""
from .model import RWKV_CMix_x070, RWKVConfig  # noqa: F401
from .moe import LoRAMoE_CMix, MoE_CMix, Router, build_layer, channel_mixing_rnn  # noqa: F401

__version__ = "0.1.0"
