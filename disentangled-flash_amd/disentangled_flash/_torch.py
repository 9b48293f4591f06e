"""Inference-only PyTorch DeBERTa attention ("torch" / "optimized" backend).

Counterpart of the reference's prepared PyTorch path
(``/root/reference/src/disentangled_flash/_torch.py:47-429``), organised
around one idea: everything derived from a layer's parameters lives in a
single :class:`LayerPreparation` record (fused QKV weight and bias, the
projected relative tables) that exists only while the parameters are
unchanged.  Per-length plans are cut from that record and cached beside it.

The forward materialises the full ``[B, H, L, L]`` score tensor, so on the GPU
it is the comparator the fused HIP kernel must beat, and its class is the base
of the HIP attention module.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
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


@dataclass(frozen=True)
class LayerPreparation:
    """Tensors derived from one attention layer's parameters.

    ``rel_key`` / ``rel_query`` are the projected relative tables ``[H, 2*span, d]``
    (bias included), present only for the modes the layer uses.
    """

    qkv_weight: torch.Tensor
    qkv_bias: torch.Tensor | None
    rel_key: torch.Tensor | None
    rel_query: torch.Tensor | None


def forget_prepared_after_load(module: torch.nn.Module, _incompatible_keys: Any) -> None:
    """``load_state_dict`` post-hook: new parameters make derived tensors stale."""

    module.clear_inference_cache()


class ParameterDerivedState:
    """Mixin for modules that cache tensors computed from their parameters.

    The cache is dropped on every event that may change parameters: a move or
    cast (``_apply``, behind ``.to()``/``.half()``/...), switching to training
    mode, and ``load_state_dict`` (the subclass registers
    :func:`forget_prepared_after_load`).  Subclasses implement
    ``clear_inference_cache``, which must tolerate being called before their
    ``__init__`` has finished.
    """

    def clear_inference_cache(self) -> None:  # pragma: no cover - abstract
        raise NotImplementedError

    def train(self, mode: bool = True):
        if mode:
            self.clear_inference_cache()
        return super().train(mode)

    def _apply(self, fn: Any, recurse: bool = True):
        moved = super()._apply(fn, recurse=recurse)
        self.clear_inference_cache()
        return moved


class TorchInferenceDisentangledSelfAttention(ParameterDerivedState, OriginalDisentangledSelfAttention):
    """Cached, active-slot-pruned DeBERTa attention for inference only.

    ``prepare_for_inference(rel_embeddings)`` builds the layer's
    :class:`LayerPreparation`; ``prepare_shape(L)`` cuts a per-length plan from
    it; ``forward_prepared`` then runs with no cache lookup or mutation.
    """

    def __init__(
        self,
        config: DebertaAttentionConfig | Any,
        *,
        position_plan_cache: SharedPositionPlanCache | None = None,
    ) -> None:
        super().__init__(config)
        self.pos_att_type = normalize_pos_att_type(self.pos_att_type)
        if position_plan_cache is None:
            position_plan_cache = SharedPositionPlanCache(
                position_buckets=self.position_buckets,
                max_relative_positions=self.max_relative_positions,
                position_embedding_size=self.pos_ebd_size,
                uses_position_bias=self.has_c2p or self.has_p2c,
            )
        self.position_plan_cache = position_plan_cache
        self._prepared: LayerPreparation | None = None
        self._length_plans: dict[tuple[int, str], Any] = {}
        self.register_load_state_dict_post_hook(forget_prepared_after_load)

    # ---- modes ----
    @property
    def has_c2p(self) -> bool:
        return self.relative_attention and "c2p" in self.pos_att_type

    @property
    def has_p2c(self) -> bool:
        return self.relative_attention and "p2c" in self.pos_att_type

    @property
    def scale_factor(self) -> int:
        return 1 + int(self.has_c2p) + int(self.has_p2c)

    def _scale(self, scale_factor: int) -> float:
        return math.sqrt(self.attention_head_size * scale_factor)

    # ---- derived state ----
    @property
    def prepared(self) -> LayerPreparation | None:
        """The layer's derived tensors, or None until ``prepare_for_inference``."""

        return self._prepared

    def clear_inference_cache(self) -> None:
        self._prepared = None
        plans = self.__dict__.get("_length_plans")
        if plans is not None:
            plans.clear()

    def set_position_plan_cache(
        self, cache: SharedPositionPlanCache
    ) -> TorchInferenceDisentangledSelfAttention:
        """Share a model-wide index cache; plans cut with the old one are dropped."""

        self.position_plan_cache = cache
        self._length_plans.clear()
        return self

    def _relative_table(self, rows: torch.Tensor, projection: torch.nn.Linear) -> torch.Tensor:
        """``[2*span, hidden]`` relative rows -> projected ``[H, 2*span, d]`` (bias included)."""

        projected = projection(rows)
        heads, dim = self.num_attention_heads, self.attention_head_size
        return projected.view(rows.size(0), heads, dim).transpose(0, 1).contiguous()

    @torch.no_grad()
    def prepare_for_inference(
        self, rel_embeddings: torch.Tensor | None
    ) -> TorchInferenceDisentangledSelfAttention:
        """Build the fused QKV weight and the projected relative tables (``_torch.py:125-159``)."""

        if self.training:
            raise RuntimeError("prepare_for_inference() requires module.eval()")
        self.clear_inference_cache()
        parts = (self.query_proj, self.key_proj, self.value_proj)
        weight = torch.cat([part.weight for part in parts], dim=0).contiguous()
        bias = None
        if all(part.bias is not None for part in parts):
            bias = torch.cat([part.bias for part in parts], dim=0).contiguous()
        rel_key = rel_query = None
        if self.relative_attention:
            if rel_embeddings is None:
                raise ValueError("rel_embeddings is required for relative attention")
            # Dropout is the identity in eval mode; kept for the module's semantics.
            rows = self.pos_dropout(rel_embeddings[: 2 * self.pos_ebd_size])
            if self.has_c2p:
                rel_key = self._relative_table(
                    rows, self.key_proj if self.share_att_key else self.pos_key_proj)
            if self.has_p2c:
                rel_query = self._relative_table(
                    rows, self.query_proj if self.share_att_key else self.pos_query_proj)
        self._prepared = LayerPreparation(weight, bias, rel_key, rel_query)
        return self

    def _require_prepared(self, what: str) -> LayerPreparation:
        if self._prepared is None:
            raise RuntimeError(f"call prepare_for_inference() before {what}")
        return self._prepared

    def _plan_device(self) -> torch.device:
        if self._prepared is not None:
            return self._prepared.qkv_weight.device
        return self.query_proj.weight.device

    def _project_active_positions(
        self, active_slots: torch.Tensor
    ) -> tuple[torch.Tensor | None, torch.Tensor | None]:
        """Rows of the projected relative tables a plan can reach, ``[H, S, d]`` each."""

        if not (self.has_c2p or self.has_p2c):
            return None, None
        prep = self._require_prepared("prepare_shape()")

        def rows(table: torch.Tensor | None) -> torch.Tensor | None:
            return None if table is None else table.index_select(1, active_slots).contiguous()

        return (rows(prep.rel_key) if self.has_c2p else None,
                rows(prep.rel_query) if self.has_p2c else None)

    def _cached_plan(self, sequence_length: int, device: torch.device | str | None, build):
        if self.training:
            raise RuntimeError("prepare_shape() requires module.eval()")
        resolved = canonical_device(device, self._plan_device())
        key = (sequence_length, str(resolved))
        plan = self._length_plans.get(key)
        if plan is None:
            plan = build(sequence_length, resolved)
            self._length_plans[key] = plan
        return plan

    @torch.no_grad()
    def prepare_shape(
        self, sequence_length: int, device: torch.device | str | None = None
    ) -> TorchPositionPlan:
        """Plan for one length: active rows plus the shared ``[1, 1, L, L]`` slot map."""

        def build(length: int, resolved: torch.device) -> TorchPositionPlan:
            indices = self.position_plan_cache.dense(length, resolved)
            pos_key, pos_query = self._project_active_positions(indices.active_slots)
            # The bucket function is odd, so for self-attention the transposed
            # p2c lookup is the c2p map itself: one tensor serves both fields.
            return TorchPositionPlan(length, indices.active_slots, indices.pair_to_local,
                                     indices.pair_to_local, pos_key, pos_query)

        return self._cached_plan(sequence_length, device, build)

    def _dynamic_position_plan(
        self,
        query_layer: torch.Tensor,
        key_layer: torch.Tensor,
        relative_pos: torch.Tensor,
    ) -> TorchPositionPlan:
        """Plan for a caller-provided ``relative_pos`` (``_torch.py:221-273``).

        The slots both modes touch are compacted with one ``torch.unique``; its
        inverse indices are the local slots, split back into the c2p and p2c maps.
        """

        if relative_pos.dim() not in (2, 3, 4):
            raise ValueError(
                f"relative_pos must have 2, 3, or 4 dimensions, got {relative_pos.dim()}"
            )
        while relative_pos.dim() < 4:  # [L, L] -> [1, 1, L, L]; [B, L, L] -> [B, 1, L, L]
            relative_pos = relative_pos.unsqueeze(-3)
        relative_pos = relative_pos.to(device=query_layer.device, dtype=torch.long)
        top = 2 * self.pos_ebd_size - 1
        c2p_slots = (relative_pos + self.pos_ebd_size).clamp(0, top)
        key_rel = build_rpos(query_layer, key_layer, relative_pos, self.max_relative_positions,
                             self.position_buckets)
        p2c_slots = (self.pos_ebd_size - key_rel).clamp(0, top).transpose(-1, -2).contiguous()
        used = [slots for slots, on in ((c2p_slots, self.has_c2p), (p2c_slots, self.has_p2c))
                if on]
        if used:
            flat = torch.cat([slots.reshape(-1) for slots in used])
            active, inverse = torch.unique(flat, sorted=True, return_inverse=True)
            pieces = iter(inverse.split([slots.numel() for slots in used]))
            c2p_local = next(pieces).view_as(c2p_slots) if self.has_c2p else c2p_slots
            p2c_local = next(pieces).view_as(p2c_slots) if self.has_p2c else p2c_slots
        else:
            active = torch.empty(0, dtype=torch.long, device=query_layer.device)
            c2p_local, p2c_local = c2p_slots, p2c_slots
        pos_key, pos_query = self._project_active_positions(active)
        return TorchPositionPlan(query_layer.size(-2), active, c2p_local, p2c_local,
                                 pos_key, pos_query)

    # ---- forward ----
    def _validate_inference_call(self) -> None:
        name = type(self).__name__
        if self.training:
            raise RuntimeError(f"{name} requires module.eval()")
        if torch.is_grad_enabled():
            raise RuntimeError(f"{name} requires torch.no_grad() or torch.inference_mode()")

    def _fused_projection(self, hidden_states: torch.Tensor) -> torch.Tensor:
        """``[B, L, hidden]`` -> ``[B, L, 3*H*d]`` with the fused weight (``_torch.py:284-297``)."""

        if self._prepared is None:
            raise RuntimeError(
                "fused QKV projection is not prepared; call prepare_for_inference() first"
            )
        return F.linear(hidden_states, self._prepared.qkv_weight, self._prepared.qkv_bias)

    def _project_qkv(
        self, hidden_states: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        return self._fused_projection(hidden_states).split(self.all_head_size, dim=-1)

    def _reshape_heads(self, tensor: torch.Tensor, batch_size: int,
                       sequence_length: int) -> torch.Tensor:
        """``[B, L, H*d]`` -> head-major ``[B, H, L, d]`` contiguous."""

        heads = tensor.unflatten(-1, (self.num_attention_heads, self.attention_head_size))
        return heads.transpose(1, 2).contiguous()

    def _check_plan_length(self, plan: Any, length: int) -> None:
        if plan.sequence_length != length:
            raise ValueError(
                f"prepared length {plan.sequence_length} does not match input length {length}"
            )

    def _relative_scores(self, q: torch.Tensor, k: torch.Tensor, plan: TorchPositionPlan,
                         scale: float) -> list[torch.Tensor]:
        """Gathered c2p and p2c score terms ``[B, H, L, L]``, each already divided by ``scale``."""

        full = (q.size(0), q.size(1), q.size(2), q.size(2))
        terms = []
        if self.has_c2p:
            if plan.pos_key is None:
                raise ValueError("prepared plan has no content-to-position keys")
            # c2p[i, j] = (q_i . Kr[slot(i - j)]) / scale
            per_slot = q @ plan.pos_key.transpose(-1, -2) / scale
            terms.append(per_slot.gather(-1, plan.c2p_local.expand(full)))
        if self.has_p2c:
            if plan.pos_query is None:
                raise ValueError("prepared plan has no position-to-content queries")
            # p2c[i, j] = (k_j . Qr[slot(i - j)]) / scale, gathered along the key axis
            per_slot = k @ plan.pos_query.transpose(-1, -2) / scale
            terms.append(per_slot.transpose(-1, -2).gather(-2, plan.p2c_local.expand(full)))
        return terms

    def forward_prepared(
        self,
        hidden_states: torch.Tensor,
        attention_mask: torch.Tensor,
        plan: TorchPositionPlan,
    ) -> tuple[torch.Tensor, None]:
        """Dense eager forward with a plan built outside the hot path (``_torch.py:316-387``)."""

        self._validate_inference_call()
        batch, length = hidden_states.shape[:2]
        self._check_plan_length(plan, length)
        q, k, v = (self._reshape_heads(part, batch, length)
                   for part in self._project_qkv(hidden_states))
        scale = self._scale(self.scale_factor)
        scores = q @ (k.transpose(-1, -2) / scale)
        for term in self._relative_scores(q, k, plan, scale):
            scores = scores + term
        keep = _prepare_attention_mask(attention_mask, length, length).bool()
        probs = scores.masked_fill(~keep, torch.finfo(q.dtype).min).softmax(dim=-1)
        context = (probs @ v).transpose(1, 2).reshape(batch, length, self.all_head_size)
        return context, None

    def _ensure_prepared(self, rel_embeddings: torch.Tensor | None) -> None:
        """Lazy preparation for the HF-signature ``forward``."""

        prep = self._prepared
        if (prep is None or (self.has_c2p and prep.rel_key is None)
                or (self.has_p2c and prep.rel_query is None)):
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
        self._ensure_prepared(rel_embeddings)
        length = hidden_states.size(1)
        if relative_pos is None:
            plan = self.prepare_shape(length, hidden_states.device)
        else:
            probe = hidden_states.view(hidden_states.size(0), 1, length, hidden_states.size(-1))
            plan = self._dynamic_position_plan(probe, probe, relative_pos)
        return self.forward_prepared(hidden_states, attention_mask, plan)


__all__ = [
    "LayerPreparation",
    "ParameterDerivedState",
    "TorchInferenceDisentangledSelfAttention",
    "TorchPositionPlan",
]
