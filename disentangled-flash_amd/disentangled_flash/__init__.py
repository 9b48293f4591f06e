"""DisentangledFlash for MI355X: fused DeBERTa-v2/v3 disentangled attention in HIP.

Drop-in for the reference package's public API (``__init__.py:3-19``):
``optimize_deberta``, ``enable_deberta_inference``, ``compile_deberta_buckets``,
``DebertaV2InferenceEncoder`` and the ``DisentangledFlashAttention`` module,
plus ``capture_deberta_buckets`` (HIP-graph replay of prepared buckets).
"""

from .deberta import (
    DebertaV2InferenceEncoder,
    compile_deberta_buckets,
    enable_deberta_inference,
    optimize_deberta,
)
from .graphs import DebertaGraphBucket, capture_deberta_buckets
from .kernel import DisentangledFlashAttention

__version__ = "0.1.0"

__all__ = [
    "DebertaGraphBucket",
    "DebertaV2InferenceEncoder",
    "capture_deberta_buckets",
    "DisentangledFlashAttention",
    "compile_deberta_buckets",
    "enable_deberta_inference",
    "optimize_deberta",
]
