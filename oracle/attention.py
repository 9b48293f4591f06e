"""float64 numpy restatements of DeBERTa disentangled attention (test infrastructure only).

* ``original_attention`` - the unfused Hugging Face equation
  (``/root/reference/src/disentangled_flash/_reference.py:252-422``), starting
  from hidden states and projection weights.
* ``fused_attention`` - the contract of the fused kernel
  (``kernel.py:196-345``): head-major Q/K/V, projected active relative rows,
  the compact delta LUT and the factorized mask with Hugging Face padded-row
  semantics (``kernel.py:250-261``).
* ``brute_force_attention`` - the same contract as plain Python loops, for
  tiny shapes.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from .positions import compact_plan, log_bucket_scalar, relative_positions


@dataclass(frozen=True)
class AttentionSpec:
    """The configuration fields the attention equation reads (``_reference.py:37-59``)."""

    hidden_size: int
    num_heads: int
    head_dim: int
    position_buckets: int = 256
    max_relative_positions: int = 512
    pos_att_type: tuple[str, ...] = ("c2p", "p2c")
    share_att_key: bool = True

    @property
    def span(self) -> int:
        """``pos_ebd_size`` (``_reference.py:221-228``)."""

        return self.position_buckets if self.position_buckets > 0 else self.max_relative_positions

    @property
    def scale_factor(self) -> int:
        return 1 + int("c2p" in self.pos_att_type) + int("p2c" in self.pos_att_type)


def _linear(x: np.ndarray, weight: np.ndarray, bias: np.ndarray | None) -> np.ndarray:
    y = x @ weight.T
    return y if bias is None else y + bias


def _heads(x: np.ndarray, heads: int) -> np.ndarray:
    """``[B, L, H*d]`` -> ``[B, H, L, d]``."""

    b, length, width = x.shape
    return x.reshape(b, length, heads, width // heads).transpose(0, 2, 1, 3)


def _softmax(x: np.ndarray) -> np.ndarray:
    shifted = x - x.max(axis=-1, keepdims=True)
    e = np.exp(shifted)
    return e / e.sum(axis=-1, keepdims=True)


def project_relative(spec: AttentionSpec, params: dict, rel_embeddings: np.ndarray):
    """Projected relative tables ``[H, 2*span, d]`` for c2p keys and p2c queries.

    ``_reference.py:363-387``: share_att_key reuses key_proj / query_proj,
    otherwise pos_key_proj / pos_query_proj.
    """

    table = np.asarray(rel_embeddings, np.float64)[: 2 * spec.span][None]
    pos_key = pos_query = None
    if "c2p" in spec.pos_att_type:
        name = "key" if spec.share_att_key else "pos_key"
        pos_key = _heads(_linear(table, params[f"{name}_weight"], params.get(f"{name}_bias")),
                         spec.num_heads)[0]
    if "p2c" in spec.pos_att_type:
        name = "query" if spec.share_att_key else "pos_query"
        pos_query = _heads(_linear(table, params[f"{name}_weight"], params.get(f"{name}_bias")),
                           spec.num_heads)[0]
    return pos_key, pos_query


def original_attention(spec: AttentionSpec, params: dict, hidden: np.ndarray,
                       rel_embeddings: np.ndarray, mask: np.ndarray,
                       scale: float | None = None, fill: float = -3.4028234663852886e38):
    """Unfused HF attention in float64 (``_reference.py:252-335`` and ``:337-422``).

    ``scale`` defaults to ``sqrt(d * factor)`` evaluated in float32, as
    ``scaled_size_sqrt`` does (``_reference.py:161-162``); the reference then
    casts it to the activation dtype (pass that rounded value to reproduce
    fp16/bf16 runs).  ``fill`` is the ``finfo(dtype).min`` used by
    ``masked_fill``.  Returns ``[B, L, H*d]``.
    """

    h = np.asarray(hidden, np.float64)
    heads = spec.num_heads
    q = _heads(_linear(h, params["query_weight"], params["query_bias"]), heads)
    k = _heads(_linear(h, params["key_weight"], params["key_bias"]), heads)
    v = _heads(_linear(h, params["value_weight"], params["value_bias"]), heads)
    if scale is None:
        scale = reference_scale(spec.head_dim, spec.scale_factor)
    length = h.shape[1]
    scores = q @ (k / scale).transpose(0, 1, 3, 2)

    span = spec.span
    rel = relative_positions(length, spec.position_buckets, spec.max_relative_positions)
    pos_key, pos_query = project_relative(spec, params, rel_embeddings)
    if "c2p" in spec.pos_att_type:
        raw = q @ pos_key.transpose(0, 2, 1)[None]            # [B, H, L, 2span]
        index = np.clip(rel + span, 0, 2 * span - 1)           # [L, L]
        picked = np.take_along_axis(raw, np.broadcast_to(index, raw.shape[:2] + index.shape), -1)
        scores = scores + picked / scale
    if "p2c" in spec.pos_att_type:
        raw = k @ pos_query.transpose(0, 2, 1)[None]          # [B, H, L(key), 2span]
        index = np.clip(-rel + span, 0, 2 * span - 1)          # [L(key row), L]
        picked = np.take_along_axis(raw, np.broadcast_to(index, raw.shape[:2] + index.shape), -1)
        scores = scores + picked.transpose(0, 1, 3, 2) / scale

    m = np.asarray(mask).astype(bool)
    pair = m[:, None, None, :] & m[:, None, :, None]
    scores = np.where(pair, scores, fill)
    out = _softmax(scores) @ v
    b = h.shape[0]
    return out.transpose(0, 2, 1, 3).reshape(b, length, heads * spec.head_dim)


def reference_scale(head_dim: int, factor: int, dtype=np.float32) -> float:
    """``scaled_size_sqrt`` (float32 sqrt) cast to ``dtype`` (``_reference.py:161-162,285``)."""

    value = np.sqrt(np.float32(head_dim) * np.float32(factor), dtype=np.float32)
    return float(np.asarray(value).astype(dtype))


def qkv_heads(spec: AttentionSpec, params: dict, hidden: np.ndarray):
    """Head-major float64 ``(q, k, v)`` ``[B, H, L, d]`` from hidden states."""

    h = np.asarray(hidden, np.float64)
    return tuple(
        _heads(_linear(h, params[f"{n}_weight"], params[f"{n}_bias"]), spec.num_heads)
        for n in ("query", "key", "value")
    )


def fused_attention(q, k, v, pos_key, pos_query, delta_to_local, mask, scale: float,
                    has_c2p: bool, has_p2c: bool):
    """Fused-kernel contract in float64 (``kernel.py:196-345``).

    ``q, k, v``: ``[B, H, L, d]``; ``pos_key, pos_query``: ``[H, S, d]`` active
    rows; ``delta_to_local``: ``[2L-1]``; ``mask``: ``[B, L]``.  Score
    ``(q_i.k_j + q_i.Kr[slot] + k_j.Qr[slot]) / scale`` with
    ``slot = delta_to_local[i - j + L - 1]``.  Kept rows attend to kept keys;
    a padded row (in range) is uniform over all keys.  Returns ``[B, L, H*d]``.
    """

    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    b, heads, length, d = q.shape
    scores = q @ k.transpose(0, 1, 3, 2)
    idx = np.arange(length)
    slot = np.asarray(delta_to_local)[idx[:, None] - idx[None, :] + length - 1]
    if has_c2p:
        raw = q @ np.asarray(pos_key, np.float64).transpose(0, 2, 1)[None]  # [B,H,L,S]
        scores = scores + np.take_along_axis(raw, np.broadcast_to(slot, (b, heads, length, length)), -1)
    if has_p2c:
        raw = k @ np.asarray(pos_query, np.float64).transpose(0, 2, 1)[None]  # [B,H,L(key),S]
        # p2c[i, j] = raw[j, slot(i - j)]
        gathered = np.take_along_axis(
            raw, np.broadcast_to(slot.T, (b, heads, length, length)), -1
        )  # [.., j, i] = raw[j, slot[i, j]]
        scores = scores + gathered.transpose(0, 1, 3, 2)
    scores = scores / scale
    m = np.asarray(mask).astype(bool)
    kept = m[:, None, :, None] & m[:, None, None, :]
    padded_row = ~m[:, None, :, None] & np.ones((1, 1, 1, length), bool)
    scores = np.where(kept, scores, -np.inf)
    scores = np.where(padded_row, 0.0, scores)
    out = _softmax(scores) @ v
    return out.transpose(0, 2, 1, 3).reshape(b, length, heads * d)


def brute_force_attention(q, k, v, pos_key, pos_query, mask, scale: float, span: int,
                          bucket_size: int, max_position: int, has_c2p: bool, has_p2c: bool):
    """Pure-Python loop version of the HF equation for tiny shapes.

    Uses ``pos_key/pos_query`` of the full ``[H, 2*span, d]`` relative tables
    (not the compact rows) and the float64 scalar bucket function, so it checks
    the compact plan and the p2c index identity independently.
    """

    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    b_count, heads, length, d = q.shape
    out = np.zeros((b_count, length, heads * d))

    def bucket(delta: int) -> int:
        return log_bucket_scalar(delta, bucket_size, max_position) if bucket_size > 0 else delta

    for b in range(b_count):
        for h in range(heads):
            for i in range(length):
                row = []
                for j in range(length):
                    s = float(np.dot(q[b, h, i], k[b, h, j]))
                    if has_c2p:
                        c_slot = min(max(bucket(i - j) + span, 0), 2 * span - 1)
                        s += float(np.dot(q[b, h, i], pos_key[h, c_slot]))
                    if has_p2c:
                        # HF: p2c_pos[j, i] = clamp(-bucket(j - i) + span), read at key row j.
                        p_slot = min(max(-bucket(j - i) + span, 0), 2 * span - 1)
                        s += float(np.dot(k[b, h, j], pos_query[h, p_slot]))
                    row.append(s / scale)
                if mask[b][i]:
                    row = [x if mask[b][j] else -math.inf for j, x in enumerate(row)]
                else:
                    row = [0.0] * length
                top = max(row)
                weights = [math.exp(x - top) for x in row]
                total = sum(weights)
                for j in range(length):
                    out[b, i, h * d:(h + 1) * d] += weights[j] / total * v[b, h, j]
    return out


def plan_for(spec: AttentionSpec, length: int):
    """Compact plan of ``spec`` at ``length`` (``position.py:89-128``)."""

    uses = bool({"c2p", "p2c"} & set(spec.pos_att_type))
    return compact_plan(length, position_buckets=spec.position_buckets,
                        max_relative_positions=spec.max_relative_positions,
                        position_embedding_size=spec.span, uses_position_bias=uses)
