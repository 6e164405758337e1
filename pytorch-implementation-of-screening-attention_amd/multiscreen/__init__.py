"""multiscreen for MI355X: Screening Attention with fused gfx950 HIP kernels.

Same public API as the reference package (multiscreen/__init__.py:13-24):
ScreeningAttention, MultiscreenBlock, MultiscreenDecoderLayer, MultiscreenLM,
TanhNorm.  On GPU tensors the attention core runs in libmsa.so (built by
build_lib.py); `ops` exposes the operator boundary and the decode step.
"""

from .attention import ScreeningAttention, KVCache
from .layers import MultiscreenBlock, MultiscreenDecoderLayer
from .model import MultiscreenLM
from .norm import TanhNorm
from . import ops

__all__ = [
    "ScreeningAttention",
    "MultiscreenBlock",
    "MultiscreenDecoderLayer",
    "MultiscreenLM",
    "TanhNorm",
]

__version__ = "0.1.0"
