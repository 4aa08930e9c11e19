"""MI355X (gfx950) attention path for KempnerForge.

Drop-in replacements for ``kempnerforge.model.attention.Attention``,
``KVCache`` and ``kempnerforge.model.mot.MoTAttention`` whose attention math (RoPE, GQA, causal softmax attention and its
backward, KV-cache decode, weight capture) runs in hand-written HIP kernels
behind the C ABI in ``include/kf_attn.h``.
"""

from kempnerforge_amd.attention import Attention, KVCache  # noqa: F401
from kempnerforge_amd.mot import MoTAttention  # noqa: F401
from kempnerforge_amd.norm import RMSNorm  # noqa: F401
from kempnerforge_amd.position import precompute_rope_frequencies  # noqa: F401

__version__ = "0.1.0"
