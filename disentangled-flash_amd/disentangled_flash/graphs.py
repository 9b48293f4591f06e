"""HIP-graph buckets: replay a prepared encoder forward without host launch cost.

At small batches the eager encoder is bound by the host, not the GPU: each
layer issues four hipBLASLt GEMMs (about 20 us of host time each on ROCm), the
attention and LayerNorm ops and a few torch elementwise kernels, so a 12-layer
forward costs about 1.9 ms of host time whatever the batch.  A HIP graph
records the whole launch sequence of one (batch, bucket length) once and
replays it with a single host call.

This is the MI355X-side counterpart of ``compile_deberta_buckets`` (reference
``deberta.py:349-427``), which uses ``torch.compile`` with CUDA graphs turned
off: instead of a tracing compiler, the prepared layer loop itself is captured.

Inputs are copied into static buffers before each replay; the returned tensor
is the graph's static output and is overwritten by the next replay of the same
bucket (``clone()`` it to keep it).  Each bucket owns its memory pool, so
replaying one bucket never disturbs another bucket's output.
"""

from __future__ import annotations

from collections.abc import Iterable

import torch

from . import layers
from .deberta import DebertaV2InferenceEncoder


class DebertaGraphBucket:
    """One captured encoder forward for a fixed ``(batch, seq_len)``."""

    def __init__(self, encoder: DebertaV2InferenceEncoder, batch: int, seq_len: int,
                 mask_dtype: torch.dtype = torch.long, warmup: int = 2) -> None:
        if seq_len not in encoder.prepared_lengths:
            raise ValueError(f"sequence length {seq_len} is not a prepared bucket")
        if batch < 1:
            raise ValueError("batch must be positive")
        attention = encoder.layer[0].attention.self
        weight = attention.query_proj.weight
        if weight.device.type != "cuda":
            raise RuntimeError("HIP graph buckets need the encoder on a GPU")
        self.encoder = encoder
        self.batch = batch
        self.seq_len = seq_len
        hidden = weight.shape[1]
        self.hidden_states = torch.zeros(batch, seq_len, hidden, device=weight.device,
                                         dtype=weight.dtype)
        self.attention_mask = torch.ones(batch, seq_len, device=weight.device, dtype=mask_dtype)
        plans = encoder.plans_for(seq_len)

        def run() -> torch.Tensor:
            return encoder.forward_prepared(self.hidden_states, self.attention_mask, plans,
                                            output_hidden_states=False).last_hidden_state

        self.pool = torch.cuda.graph_pool_handle()
        self.graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(device=weight.device)
        side.wait_stream(torch.cuda.current_stream(weight.device))
        with torch.inference_mode(), torch.cuda.stream(side):
            # Library handles and workspaces exist before capture: the warm-up runs the
            # kernels the capture will record (capture picks hipBLASLt for few rows).
            with layers.graph_gemm_choice():
                for _ in range(max(1, warmup)):
                    run()
            with torch.cuda.graph(self.graph, pool=self.pool, stream=side):
                self.output = run()
        torch.cuda.current_stream(weight.device).wait_stream(side)

    def __call__(self, hidden_states: torch.Tensor, attention_mask: torch.Tensor) -> torch.Tensor:
        if tuple(hidden_states.shape) != tuple(self.hidden_states.shape):
            raise ValueError(
                f"bucket expects hidden states {tuple(self.hidden_states.shape)}, "
                f"got {tuple(hidden_states.shape)}"
            )
        if tuple(attention_mask.shape) != tuple(self.attention_mask.shape):
            raise ValueError(
                f"bucket expects a mask of shape {tuple(self.attention_mask.shape)}, "
                f"got {tuple(attention_mask.shape)}"
            )
        self.hidden_states.copy_(hidden_states)
        self.attention_mask.copy_(attention_mask)
        self.graph.replay()
        return self.output


def capture_deberta_buckets(
    encoder: DebertaV2InferenceEncoder,
    shapes: Iterable[tuple[int, int]],
    *,
    mask_dtype: torch.dtype = torch.long,
    warmup: int = 2,
) -> dict[tuple[int, int], DebertaGraphBucket]:
    """Capture one HIP graph per ``(batch, seq_len)``; every length must be a prepared bucket.

    The encoder must stay prepared (no ``clear_inference_cache`` or weight changes) while
    the buckets are in use: the graphs hold its cached weights and plans by address.
    """

    buckets: dict[tuple[int, int], DebertaGraphBucket] = {}
    for batch, seq_len in dict.fromkeys((int(b), int(s)) for b, s in shapes):
        buckets[(batch, seq_len)] = DebertaGraphBucket(encoder, batch, seq_len,
                                                       mask_dtype=mask_dtype, warmup=warmup)
    return buckets


__all__ = ["DebertaGraphBucket", "capture_deberta_buckets"]
