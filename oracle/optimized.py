"""torch CPU restatement of the prepared "optimized" forward (test infrastructure only).

Follows ``/root/reference/src/disentangled_flash/_torch.py:316-387``: fused QKV
linear, head reshape, ``QK^T / scale``, active-slot c2p/p2c products divided by
the scale and gathered through the dense ``[L, L]`` slot map, ``finfo.min``
mask fill, softmax and PV.  ``bench.py`` times it on the host CPU as the
reported baseline; tests pin it against ``attention.original_attention``.
"""

from __future__ import annotations

import math

import torch


def optimized_attention(hidden: torch.Tensor, qkv_weight: torch.Tensor,
                        qkv_bias: torch.Tensor | None, pos_key: torch.Tensor | None,
                        pos_query: torch.Tensor | None, pair_to_local: torch.Tensor,
                        mask: torch.Tensor, num_heads: int, head_dim: int) -> torch.Tensor:
    """``hidden [B, L, hidden]`` -> context ``[B, L, H*d]``.

    ``pos_key/pos_query`` are ``[H, S, d]`` (None when that mode is off);
    ``pair_to_local`` is the ``[L, L]`` int64 slot map; ``mask`` is ``[B, L]``.
    """

    batch, length = hidden.shape[:2]
    width = num_heads * head_dim
    factor = 1 + int(pos_key is not None) + int(pos_query is not None)
    scale = math.sqrt(head_dim * factor)
    fused = torch.nn.functional.linear(hidden, qkv_weight, qkv_bias)

    def heads(t: torch.Tensor) -> torch.Tensor:
        return t.view(batch, length, num_heads, head_dim).permute(0, 2, 1, 3).contiguous()

    q, k, v = (heads(t) for t in fused.split(width, dim=-1))
    return optimized_core(q, k, v, pos_key, pos_query, pair_to_local, mask, scale)


def optimized_core(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   pos_key: torch.Tensor | None, pos_query: torch.Tensor | None,
                   pair_to_local: torch.Tensor, mask: torch.Tensor, scale: float) -> torch.Tensor:
    """Attention part of ``_torch.py:339-387`` from head-major ``q/k/v [B, H, L, d]``."""

    batch, num_heads, length, head_dim = q.shape
    width = num_heads * head_dim
    scores = torch.matmul(q, k.transpose(-1, -2) / scale)
    index = pair_to_local.expand(batch, num_heads, length, length)
    if pos_key is not None:
        raw = torch.matmul(q, pos_key.transpose(-1, -2)) / scale
        scores = scores + torch.gather(raw, -1, index)
    if pos_query is not None:
        raw = torch.matmul(k, pos_query.transpose(-1, -2)) / scale
        scores = scores + torch.gather(raw.transpose(-1, -2), -2, index)
    m = mask.bool()
    pair = m[:, None, None, :] & m[:, None, :, None]
    scores = scores.masked_fill(~pair, torch.finfo(q.dtype).min)
    context = torch.matmul(torch.softmax(scores, dim=-1), v)
    return context.permute(0, 2, 1, 3).reshape(batch, length, width)
