"""Inference-only PyTorch DeBERTa attention ("torch" / "optimized" backend).

Mirror of the reference's prepared PyTorch path (``_torch.py:47-429``): a fused
QKV weight, relative projections computed once per layer, active-slot pruning,
and one dense gather map shared by all layers.  It materialises the full
``[B, H, L, L]`` score tensor, so on the GPU it is the comparator the fused HIP
kernel must beat, and its class is the base of the HIP attention module.
"""

from __future__ import annotations

import math
from typing import Any, NamedTuple

import torch
from torch.nn import functional as F

from .modeling import (
    DebertaAttentionConfig,
    OriginalDisentangledSelfAttention,
    _prepare_attention_mask,
    build_rpos,
    normalize_pos_att_type,
)
from .position import SharedPositionPlanCache, canonical_device


class TorchPositionPlan(NamedTuple):
    """Layer projections plus shared gather indices for one length (``_torch.py:29-37``)."""

    sequence_length: int
    active_slots: torch.Tensor
    c2p_local: torch.Tensor
    p2c_local: torch.Tensor
    pos_key: torch.Tensor | None
    pos_query: torch.Tensor | None


def _invalidate_attention_cache_after_load(module: torch.nn.Module, _keys: Any) -> None:
    module.clear_inference_cache()


class TorchInferenceDisentangledSelfAttention(OriginalDisentangledSelfAttention):
    """Cached, active-slot-pruned DeBERTa attention for inference only.

    ``forward_prepared`` does no cache lookup or mutation.  Derived tensors are
    dropped whenever parameters may have changed: after ``load_state_dict``,
    ``.to()`` / ``_apply`` and ``train(True)`` (``_torch.py:81,102-110``).
    """

    def __init__(
        self,
        config: DebertaAttentionConfig | Any,
        *,
        position_plan_cache: SharedPositionPlanCache | None = None,
    ) -> None:
        super().__init__(config)
        self.pos_att_type = normalize_pos_att_type(self.pos_att_type)
        uses_bias = self.relative_attention and bool({"c2p", "p2c"} & set(self.pos_att_type))
        self.position_plan_cache = position_plan_cache or SharedPositionPlanCache(
            position_buckets=self.position_buckets,
            max_relative_positions=self.max_relative_positions,
            position_embedding_size=self.pos_ebd_size,
            uses_position_bias=uses_bias,
        )
        self.register_buffer("_cached_pos_key", None, persistent=False)
        self.register_buffer("_cached_pos_query", None, persistent=False)
        self.register_buffer("_cached_qkv_weight", None, persistent=False)
        self.register_buffer("_cached_qkv_bias", None, persistent=False)
        self._position_projection_cache: dict[tuple[int, str], TorchPositionPlan] = {}
        self.register_load_state_dict_post_hook(_invalidate_attention_cache_after_load)

    @property
    def has_c2p(self) -> bool:
        return self.relative_attention and "c2p" in self.pos_att_type

    @property
    def has_p2c(self) -> bool:
        return self.relative_attention and "p2c" in self.pos_att_type

    def set_position_plan_cache(
        self, cache: SharedPositionPlanCache
    ) -> TorchInferenceDisentangledSelfAttention:
        self.position_plan_cache = cache
        self._position_projection_cache.clear()
        return self

    def clear_inference_cache(self) -> None:
        self._cached_pos_key = None
        self._cached_pos_query = None
        self._cached_qkv_weight = None
        self._cached_qkv_bias = None
        self._position_projection_cache.clear()

    def train(self, mode: bool = True) -> TorchInferenceDisentangledSelfAttention:
        if mode:
            self.clear_inference_cache()
        return super().train(mode)

    def _apply(self, fn: Any, recurse: bool = True) -> TorchInferenceDisentangledSelfAttention:
        result = super()._apply(fn, recurse=recurse)
        self.clear_inference_cache()
        return result

    @torch.no_grad()
    def _prepare_fused_qkv(self) -> None:
        """Concatenate Wq, Wk, Wv (and biases) into one ``[3*H*d, hidden]`` weight."""

        projections = (self.query_proj, self.key_proj, self.value_proj)
        self._cached_qkv_weight = torch.cat([p.weight for p in projections], dim=0).contiguous()
        biases = [p.bias for p in projections]
        self._cached_qkv_bias = (
            torch.cat(biases, dim=0).contiguous() if all(b is not None for b in biases) else None
        )

    @torch.no_grad()
    def prepare_for_inference(
        self, rel_embeddings: torch.Tensor | None
    ) -> TorchInferenceDisentangledSelfAttention:
        """Cache the fused QKV weight and the projected relative table ``[H, 2*span, d]``."""

        if self.training:
            raise RuntimeError("prepare_for_inference() requires module.eval()")
        self.clear_inference_cache()
        self._prepare_fused_qkv()
        if not self.relative_attention:
            return self
        if rel_embeddings is None:
            raise ValueError("rel_embeddings is required for relative attention")
        table = self.pos_dropout(rel_embeddings[: self.pos_ebd_size * 2]).unsqueeze(0)
        heads = self.num_attention_heads
        if self.has_c2p:
            projection = self.key_proj if self.share_att_key else self.pos_key_proj
            self._cached_pos_key = self.transpose_for_scores(projection(table), heads)
        if self.has_p2c:
            projection = self.query_proj if self.share_att_key else self.pos_query_proj
            self._cached_pos_query = self.transpose_for_scores(projection(table), heads)
        return self

    def _plan_device(self) -> torch.device:
        for cached in (self._cached_pos_key, self._cached_pos_query):
            if cached is not None:
                return cached.device
        return self.query_proj.weight.device

    def _scale(self, scale_factor: int) -> float:
        return math.sqrt(self.attention_head_size * scale_factor)

    @property
    def scale_factor(self) -> int:
        return 1 + int(self.has_c2p) + int(self.has_p2c)

    def _project_active_positions(
        self, active_slots: torch.Tensor
    ) -> tuple[torch.Tensor | None, torch.Tensor | None]:
        """Rows of the projected relative table that a length can reach, ``[H, S, d]``."""

        pos_key = pos_query = None
        if self.has_c2p:
            if self._cached_pos_key is None:
                raise RuntimeError("call prepare_for_inference() before prepare_shape()")
            pos_key = self._cached_pos_key.index_select(1, active_slots).contiguous()
        if self.has_p2c:
            if self._cached_pos_query is None:
                raise RuntimeError("call prepare_for_inference() before prepare_shape()")
            pos_query = self._cached_pos_query.index_select(1, active_slots).contiguous()
        return pos_key, pos_query

    @torch.no_grad()
    def prepare_shape(
        self, sequence_length: int, device: torch.device | str | None = None
    ) -> TorchPositionPlan:
        if self.training:
            raise RuntimeError("prepare_shape() requires module.eval()")
        resolved = canonical_device(device, self._plan_device())
        key = (sequence_length, str(resolved))
        hit = self._position_projection_cache.get(key)
        if hit is not None:
            return hit
        indices = self.position_plan_cache.dense(sequence_length, resolved)
        pos_key, pos_query = self._project_active_positions(indices.active_slots)
        # For square self-attention the transposed p2c lookup uses the same
        # delta map as c2p (the bucket function is odd), so one tensor serves both.
        plan = TorchPositionPlan(
            sequence_length=sequence_length,
            active_slots=indices.active_slots,
            c2p_local=indices.pair_to_local,
            p2c_local=indices.pair_to_local,
            pos_key=pos_key,
            pos_query=pos_query,
        )
        self._position_projection_cache[key] = plan
        return plan

    def _dynamic_position_plan(
        self,
        query_layer: torch.Tensor,
        key_layer: torch.Tensor,
        relative_pos: torch.Tensor,
    ) -> TorchPositionPlan:
        """Plan for a caller-provided ``relative_pos`` tensor (``_torch.py:221-273``)."""

        if relative_pos.dim() == 2:
            relative_pos = relative_pos[None, None]
        elif relative_pos.dim() == 3:
            relative_pos = relative_pos.unsqueeze(1)
        elif relative_pos.dim() != 4:
            raise ValueError(
                f"relative_pos must have 2, 3, or 4 dimensions, got {relative_pos.dim()}"
            )
        relative_pos = relative_pos.to(device=query_layer.device, dtype=torch.long)
        span = self.pos_ebd_size
        c2p_slots = torch.clamp(relative_pos + span, 0, 2 * span - 1)
        key_relative = build_rpos(
            query_layer,
            key_layer,
            relative_pos,
            self.max_relative_positions,
            self.position_buckets,
        )
        p2c_slots = torch.clamp(-key_relative + span, 0, 2 * span - 1).transpose(-1, -2)
        used = []
        if self.has_c2p:
            used.append(c2p_slots.reshape(-1))
        if self.has_p2c:
            used.append(p2c_slots.reshape(-1))
        if used:
            active = torch.unique(torch.cat(used), sorted=True)
            c2p_local = torch.searchsorted(active, c2p_slots)
            p2c_local = torch.searchsorted(active, p2c_slots.contiguous())
        else:
            active = torch.empty(0, dtype=torch.long, device=query_layer.device)
            c2p_local, p2c_local = c2p_slots, p2c_slots
        pos_key, pos_query = self._project_active_positions(active)
        return TorchPositionPlan(
            sequence_length=query_layer.size(-2),
            active_slots=active,
            c2p_local=c2p_local,
            p2c_local=p2c_local,
            pos_key=pos_key,
            pos_query=pos_query,
        )

    def _validate_inference_call(self) -> None:
        name = type(self).__name__
        if self.training:
            raise RuntimeError(f"{name} requires module.eval()")
        if torch.is_grad_enabled():
            raise RuntimeError(f"{name} requires torch.no_grad() or torch.inference_mode()")

    def _project_qkv(
        self, hidden_states: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        if self._cached_qkv_weight is None:
            raise RuntimeError(
                "fused QKV projection is not prepared; call prepare_for_inference() first"
            )
        fused = F.linear(hidden_states, self._cached_qkv_weight, self._cached_qkv_bias)
        return fused.split(self.all_head_size, dim=-1)

    def _reshape_heads(
        self, tensor: torch.Tensor, batch_size: int, sequence_length: int
    ) -> torch.Tensor:
        shaped = tensor.view(
            batch_size, sequence_length, self.num_attention_heads, self.attention_head_size
        )
        return shaped.permute(0, 2, 1, 3).contiguous()

    def forward_prepared(
        self,
        hidden_states: torch.Tensor,
        attention_mask: torch.Tensor,
        plan: TorchPositionPlan,
    ) -> tuple[torch.Tensor, None]:
        """Dense eager forward with a plan built outside the hot path (``_torch.py:316-387``)."""

        self._validate_inference_call()
        batch, length = hidden_states.shape[:2]
        if length != plan.sequence_length:
            raise ValueError(
                f"prepared length {plan.sequence_length} does not match input length {length}"
            )
        query, key, value = self._project_qkv(hidden_states)
        q = self._reshape_heads(query, batch, length)
        k = self._reshape_heads(key, batch, length)
        v = self._reshape_heads(value, batch, length)
        scale = self._scale(self.scale_factor)
        heads = self.num_attention_heads
        scores = torch.matmul(q, k.transpose(-1, -2) / scale)
        if self.has_c2p:
            if plan.pos_key is None:
                raise ValueError("prepared plan has no content-to-position keys")
            raw = torch.matmul(q, plan.pos_key.transpose(-1, -2)) / scale
            index = plan.c2p_local.expand(batch, heads, length, length)
            scores = scores + torch.gather(raw, dim=-1, index=index)
        if self.has_p2c:
            if plan.pos_query is None:
                raise ValueError("prepared plan has no position-to-content queries")
            raw = torch.matmul(k, plan.pos_query.transpose(-1, -2)) / scale
            index = plan.p2c_local.expand(batch, heads, length, length)
            scores = scores + torch.gather(raw.transpose(-1, -2), dim=-2, index=index)
        mask = _prepare_attention_mask(attention_mask, length, length).bool()
        scores = scores.masked_fill(~mask, torch.finfo(q.dtype).min)
        context = torch.matmul(torch.softmax(scores, dim=-1), v)
        context = context.permute(0, 2, 1, 3).contiguous().view(batch, length, self.all_head_size)
        return context, None

    def _lazy_prepare(self, rel_embeddings: torch.Tensor | None) -> None:
        stale = (
            (self.has_c2p and self._cached_pos_key is None)
            or (self.has_p2c and self._cached_pos_query is None)
            or self._cached_qkv_weight is None
        )
        if stale:
            self.prepare_for_inference(rel_embeddings)

    def forward(
        self,
        hidden_states: torch.Tensor,
        attention_mask: torch.Tensor,
        output_attentions: bool = False,
        query_states: torch.Tensor | None = None,
        relative_pos: torch.Tensor | None = None,
        rel_embeddings: torch.Tensor | None = None,
    ) -> tuple[torch.Tensor, None]:
        """HF-signature wrapper; preparation stays outside ``forward_prepared``."""

        self._validate_inference_call()
        if output_attentions:
            raise ValueError("output_attentions=True is not supported by the inference path")
        if query_states is not None:
            raise ValueError("the torch inference path supports self-attention only")
        self._lazy_prepare(rel_embeddings)
        length = hidden_states.size(1)
        if relative_pos is None:
            plan = self.prepare_shape(length, hidden_states.device)
        else:
            probe = hidden_states.view(hidden_states.size(0), 1, length, hidden_states.size(-1))
            plan = self._dynamic_position_plan(probe, probe, relative_pos)
        return self.forward_prepared(hidden_states, attention_mask, plan)


__all__ = ["TorchInferenceDisentangledSelfAttention", "TorchPositionPlan"]
