"""CPU oracle (test infrastructure only): a NumPy restatement of the
reference's LoRA-MoE ChannelMix forward.  Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg import it; the product never does."""
from .moe_oracle import *  # noqa: F401,F403
