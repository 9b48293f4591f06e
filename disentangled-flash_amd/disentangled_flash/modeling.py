"""DeBERTa-v2/v3 attention configuration and the unfused ("original") equation.

This module holds the pieces every backend shares:

* ``DebertaAttentionConfig`` - the subset of ``DebertaV2Config`` the attention
  path reads (reference ``_reference.py:37-59``).
* ``make_log_bucket_position`` / ``build_relative_position`` - DeBERTa's
  log-bucketed relative distance (reference ``_reference.py:115-158``).
* ``DisentangledSelfAttention`` - the unfused eager equation with the same
  parameter names as Hugging Face's module (``query_proj``, ``key_proj``,
  ``value_proj``, ``pos_key_proj``, ``pos_query_proj``), so checkpoints load with
  a strict ``load_state_dict`` (reference ``_reference.py:199-422``).

The eager equation is kept bit-compatible with the Hugging Face one: the
``sqrt(d * factor)`` scale is evaluated in float32 and cast to the activation
dtype before dividing (``_reference.py:161-162,285,401,421``), and masked scores
are filled with ``finfo(dtype).min`` before the softmax (``_reference.py:307-311``).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Callable

import torch
from torch import nn
from torch.nn import functional as F


@dataclass(frozen=True)
class DebertaAttentionConfig:
    """Attention-relevant subset of ``DebertaV2Config`` (``_reference.py:37-59``)."""

    hidden_size: int = 768
    num_attention_heads: int = 12
    attention_head_size: int | None = None
    num_hidden_layers: int = 12
    intermediate_size: int = 3072
    hidden_act: str | Callable[[torch.Tensor], torch.Tensor] = "gelu"
    attention_probs_dropout_prob: float = 0.1
    hidden_dropout_prob: float = 0.1
    layer_norm_eps: float = 1e-7
    relative_attention: bool = True
    max_relative_positions: int = -1
    max_position_embeddings: int = 512
    position_buckets: int = 256
    share_att_key: bool = True
    pos_att_type: Any = ("p2c", "c2p")
    norm_rel_ebd: str = "layer_norm"
    conv_kernel_size: int = 0
    conv_groups: int = 1
    conv_act: str = "tanh"


@dataclass
class BaseModelOutput:
    """Encoder output record with tuple-style indexing (``_reference.py:62-76``)."""

    last_hidden_state: torch.Tensor
    hidden_states: tuple[torch.Tensor, ...] | None = None
    attentions: tuple[torch.Tensor, ...] | None = None

    def __getitem__(self, index: int) -> Any:
        present = [
            item
            for item in (self.last_hidden_state, self.hidden_states, self.attentions)
            if item is not None
        ]
        return present[index]


def make_log_bucket_position(
    relative_pos: torch.Tensor,
    bucket_size: int,
    max_position: int,
) -> torch.Tensor:
    """Map signed distances to DeBERTa's log buckets (``_reference.py:115-136``).

    Distances with ``|d| <= bucket_size // 2`` are kept; larger ones become
    ``sign(d) * (ceil(log(|d| / mid) / log((max_position - 1) / mid) * (mid - 1)) + mid)``.
    The logarithm is evaluated in float32, as in the reference.
    """

    mid = bucket_size // 2
    sign = torch.sign(relative_pos)
    inside = (relative_pos < mid) & (relative_pos > -mid)
    magnitude = torch.where(inside, torch.full_like(relative_pos, mid - 1), relative_pos.abs())
    ratio = magnitude / mid
    log_ratio = torch.log(ratio) / torch.log(torch.tensor((max_position - 1) / mid))
    bucketed = torch.ceil(log_ratio * (mid - 1)) + mid
    return torch.where(magnitude <= mid, relative_pos.type_as(bucketed), bucketed * sign)


def build_relative_position(
    query_layer: torch.Tensor,
    key_layer: torch.Tensor,
    bucket_size: int = -1,
    max_position: int = -1,
) -> torch.Tensor:
    """``[1, Lq, Lk]`` long tensor of (bucketed) ``i - j`` (``_reference.py:139-158``)."""

    query_size = query_layer.size(-2)
    key_size = key_layer.size(-2)
    rows = torch.arange(query_size, dtype=torch.long, device=query_layer.device)
    cols = torch.arange(key_size, dtype=torch.long, device=key_layer.device)
    relative = rows[:, None] - cols[None, :]
    if bucket_size > 0 and max_position > 0:
        relative = make_log_bucket_position(relative, bucket_size, max_position)
    return relative.to(torch.long)[:query_size, :].unsqueeze(0)


def scaled_size_sqrt(layer: torch.Tensor, scale_factor: int) -> torch.Tensor:
    """float32 ``sqrt(head_dim * factor)`` as a 0-d tensor (``_reference.py:161-162``)."""

    return torch.sqrt(torch.tensor(layer.size(-1), dtype=torch.float) * scale_factor)


def build_rpos(
    query_layer: torch.Tensor,
    key_layer: torch.Tensor,
    relative_pos: torch.Tensor,
    position_buckets: int,
    max_relative_positions: int,
) -> torch.Tensor:
    """Key-side relative positions for p2c (``_reference.py:165-179``)."""

    if key_layer.size(-2) != query_layer.size(-2):
        return build_relative_position(
            key_layer,
            key_layer,
            bucket_size=position_buckets,
            max_position=max_relative_positions,
        )
    return relative_pos


def _prepare_attention_mask(
    attention_mask: torch.Tensor,
    query_length: int,
    key_length: int,
) -> torch.Tensor:
    """Expand a ``[B, L]`` padding mask to the pairwise ``[B, 1, L, L]`` product.

    Equivalent of ``DebertaV2Encoder.get_attention_mask`` (``_reference.py:182-196``).
    """

    if attention_mask.dim() <= 2:
        expanded = attention_mask.unsqueeze(1).unsqueeze(2)
        return expanded * expanded.squeeze(-2).unsqueeze(-1)
    if attention_mask.dim() == 3:
        return attention_mask.unsqueeze(1)
    if attention_mask.dim() == 4:
        return attention_mask
    raise ValueError("attention_mask must have 2, 3, or 4 dimensions")


def normalize_pos_att_type(value: Any) -> tuple[str, ...]:
    """Accept ``"c2p|p2c"`` strings as well as sequences (``_torch.py:63-66``)."""

    if value is None:
        return ()
    if isinstance(value, str):
        return tuple(part.strip().lower() for part in value.split("|") if part.strip())
    return tuple(value)


class DisentangledSelfAttention(nn.Module):
    """Unfused DeBERTa-v2/v3 disentangled self-attention ("original" backend).

    The forward follows ``_reference.py:252-422``: three projections, the
    content-to-content score, content-to-position (c2p) and position-to-content
    (p2c) scores gathered through clamped relative positions, the factor-scaled
    sum, a ``finfo.min`` mask fill, softmax and the value product.
    """

    def __init__(self, config: Any) -> None:
        super().__init__()
        if config.hidden_size % config.num_attention_heads != 0:
            raise ValueError(
                f"The hidden size ({config.hidden_size}) is not a multiple of the number "
                f"of attention heads ({config.num_attention_heads})"
            )
        self.num_attention_heads = config.num_attention_heads
        fallback_head = config.hidden_size // config.num_attention_heads
        self.attention_head_size = getattr(config, "attention_head_size", None) or fallback_head
        self.all_head_size = self.num_attention_heads * self.attention_head_size
        self.query_proj = nn.Linear(config.hidden_size, self.all_head_size, bias=True)
        self.key_proj = nn.Linear(config.hidden_size, self.all_head_size, bias=True)
        self.value_proj = nn.Linear(config.hidden_size, self.all_head_size, bias=True)

        self.share_att_key = getattr(config, "share_att_key", False)
        self.pos_att_type = (
            config.pos_att_type if config.pos_att_type is not None else []
        )
        self.relative_attention = getattr(config, "relative_attention", False)
        if self.relative_attention:
            self.position_buckets = getattr(config, "position_buckets", -1)
            self.max_relative_positions = getattr(config, "max_relative_positions", -1)
            if self.max_relative_positions < 1:
                self.max_relative_positions = config.max_position_embeddings
            self.pos_ebd_size = self.max_relative_positions
            if self.position_buckets > 0:
                self.pos_ebd_size = self.position_buckets
            self.pos_dropout = nn.Dropout(config.hidden_dropout_prob)
            if not self.share_att_key:
                if "c2p" in self.pos_att_type:
                    self.pos_key_proj = nn.Linear(
                        config.hidden_size, self.all_head_size, bias=True
                    )
                if "p2c" in self.pos_att_type:
                    self.pos_query_proj = nn.Linear(config.hidden_size, self.all_head_size)
        else:
            self.position_buckets = -1
            self.max_relative_positions = -1
            self.pos_ebd_size = 0
        self.dropout = nn.Dropout(config.attention_probs_dropout_prob)

    def transpose_for_scores(self, tensor: torch.Tensor, attention_heads: int) -> torch.Tensor:
        """``[B, L, H*d]`` -> ``[B*H, L, d]`` contiguous (``_reference.py:243-250``)."""

        shaped = tensor.view(tensor.size()[:-1] + (attention_heads, -1))
        return shaped.permute(0, 2, 1, 3).contiguous().view(-1, shaped.size(1), shaped.size(-1))

    def forward(
        self,
        hidden_states: torch.Tensor,
        attention_mask: torch.Tensor,
        output_attentions: bool = False,
        query_states: torch.Tensor | None = None,
        relative_pos: torch.Tensor | None = None,
        rel_embeddings: torch.Tensor | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor | None]:
        if query_states is None:
            query_states = hidden_states
        heads = self.num_attention_heads
        query_layer = self.transpose_for_scores(self.query_proj(query_states), heads)
        key_layer = self.transpose_for_scores(self.key_proj(hidden_states), heads)
        value_layer = self.transpose_for_scores(self.value_proj(hidden_states), heads)

        factor = 1 + int("c2p" in self.pos_att_type) + int("p2c" in self.pos_att_type)
        scale = scaled_size_sqrt(query_layer, factor)
        scores = torch.bmm(
            query_layer, key_layer.transpose(-1, -2) / scale.to(dtype=query_layer.dtype)
        )
        if self.relative_attention:
            if rel_embeddings is None:
                raise ValueError("rel_embeddings is required when relative_attention=True")
            bias = self.disentangled_attention_bias(
                query_layer,
                key_layer,
                relative_pos,
                self.pos_dropout(rel_embeddings),
                factor,
            )
            scores = scores + bias
        scores = scores.view(-1, heads, scores.size(-2), scores.size(-1))
        scores = scores.masked_fill(~attention_mask.bool(), torch.finfo(query_layer.dtype).min)
        probs = self.dropout(F.softmax(scores, dim=-1))
        context = torch.bmm(probs.view(-1, probs.size(-2), probs.size(-1)), value_layer)
        context = (
            context.view(-1, heads, context.size(-2), context.size(-1))
            .permute(0, 2, 1, 3)
            .contiguous()
        )
        context = context.view(context.size()[:-2] + (-1,))
        return (context, probs) if output_attentions else (context, None)

    def _relative_layers(
        self,
        rel_embeddings: torch.Tensor,
        repeat: int,
    ) -> tuple[torch.Tensor | None, torch.Tensor | None]:
        heads = self.num_attention_heads
        pos_key = pos_query = None
        if self.share_att_key:
            pos_query = self.transpose_for_scores(self.query_proj(rel_embeddings), heads)
            pos_key = self.transpose_for_scores(self.key_proj(rel_embeddings), heads)
        else:
            if "c2p" in self.pos_att_type:
                pos_key = self.transpose_for_scores(self.pos_key_proj(rel_embeddings), heads)
            if "p2c" in self.pos_att_type:
                pos_query = self.transpose_for_scores(self.pos_query_proj(rel_embeddings), heads)
        if pos_key is not None:
            pos_key = pos_key.repeat(repeat, 1, 1)
        if pos_query is not None:
            pos_query = pos_query.repeat(repeat, 1, 1)
        return pos_key, pos_query

    def disentangled_attention_bias(
        self,
        query_layer: torch.Tensor,
        key_layer: torch.Tensor,
        relative_pos: torch.Tensor | None,
        rel_embeddings: torch.Tensor,
        scale_factor: int,
    ) -> torch.Tensor:
        """c2p + p2c score bias, each divided by the dtype-cast scale (``_reference.py:337-422``)."""

        if relative_pos is None:
            relative_pos = build_relative_position(
                query_layer,
                key_layer,
                bucket_size=self.position_buckets,
                max_position=self.max_relative_positions,
            )
        if relative_pos.dim() == 2:
            relative_pos = relative_pos.unsqueeze(0).unsqueeze(0)
        elif relative_pos.dim() == 3:
            relative_pos = relative_pos.unsqueeze(1)
        elif relative_pos.dim() != 4:
            raise ValueError(
                f"Relative position ids must be of dim 2 or 3 or 4. {relative_pos.dim()}"
            )
        span = self.pos_ebd_size
        relative_pos = relative_pos.to(device=query_layer.device, dtype=torch.long)
        table = rel_embeddings[0 : span * 2, :].unsqueeze(0)
        batch = query_layer.size(0) // self.num_attention_heads
        pos_key, pos_query = self._relative_layers(table, batch)

        bias: torch.Tensor | int = 0
        if "c2p" in self.pos_att_type:
            scale = scaled_size_sqrt(pos_key, scale_factor)
            raw = torch.bmm(query_layer, pos_key.transpose(-1, -2))
            index = torch.clamp(relative_pos + span, 0, span * 2 - 1).squeeze(0)
            index = index.expand([query_layer.size(0), query_layer.size(1), relative_pos.size(-1)])
            picked = torch.gather(raw, dim=-1, index=index)
            bias = bias + picked / scale.to(dtype=picked.dtype)
        if "p2c" in self.pos_att_type:
            scale = scaled_size_sqrt(pos_query, scale_factor)
            key_relative = build_rpos(
                query_layer,
                key_layer,
                relative_pos,
                self.max_relative_positions,
                self.position_buckets,
            )
            index = torch.clamp(-key_relative + span, 0, span * 2 - 1).squeeze(0)
            keys = key_layer.size(-2)
            index = index.expand([query_layer.size(0), keys, keys])
            raw = torch.bmm(key_layer, pos_query.transpose(-1, -2))
            picked = torch.gather(raw, dim=-1, index=index).transpose(-1, -2)
            bias = bias + picked / scale.to(dtype=picked.dtype)
        return bias


OriginalDisentangledSelfAttention = DisentangledSelfAttention

__all__ = [
    "BaseModelOutput",
    "DebertaAttentionConfig",
    "DisentangledSelfAttention",
    "OriginalDisentangledSelfAttention",
    "_prepare_attention_mask",
    "build_relative_position",
    "build_rpos",
    "make_log_bucket_position",
    "normalize_pos_att_type",
    "scaled_size_sqrt",
]
