"""flashloop_amd -- MI355X (gfx950) quantized cross-loop KV decode path of FlashLoop.

Host side in Python over PyTorch-ROCm (device memory and streams); the work runs in
hand-written HIP kernels of ``libflashloop_amd.so`` behind a C ABI
(include/flashloop_amd.h).  There is no CPU fallback.
"""

from .cache import (  # noqa: F401
    AttentionStep,
    CrossLoopKVCache,
    CrossLoopKVLayer,
    LayerGeometry,
    decode_attention_step,
    packed_prefix_tokens,
)
from .config import FlashLoopConfig  # noqa: F401
from .batch_engine import FlashLoopBatchEngine
from .batch_engine import FlashLoopBatchEngine  # noqa: F401
from .engine import FlashLoopEngine  # noqa: F401
from .hooks import flashloop  # noqa: F401

__all__ = [
    "AttentionStep",
    "CrossLoopKVCache",
    "CrossLoopKVLayer",
    "LayerGeometry",
    "decode_attention_step",
    "packed_prefix_tokens",
    "FlashLoopConfig",
    "FlashLoopBatchEngine",
    "FlashLoopEngine",
    "flashloop",
]
