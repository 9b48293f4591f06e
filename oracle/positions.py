"""Relative-position planning restated in numpy (test infrastructure only).

Follows ``/root/reference/src/disentangled_flash/_reference.py:115-158`` (bucket
function, relative positions) and ``position.py:89-156`` (compact and dense plans).
"""

from __future__ import annotations

import math

import numpy as np


def log_bucket(delta: np.ndarray, bucket_size: int, max_position: int,
               dtype=np.float32) -> np.ndarray:
    """``make_log_bucket_position`` (``_reference.py:115-136``), returned as int64.

    ``dtype`` is the float type of the logarithm; the reference uses float32.
    """

    delta = np.asarray(delta, dtype=np.int64)
    mid = bucket_size // 2
    inside = (delta < mid) & (delta > -mid)
    magnitude = np.where(inside, mid - 1, np.abs(delta)).astype(dtype)
    denom = np.log(dtype((max_position - 1) / mid))
    logged = np.ceil(np.log(magnitude / dtype(mid)) / denom * dtype(mid - 1)) + dtype(mid)
    bucketed = np.where(np.abs(delta) <= mid, delta.astype(dtype), logged * np.sign(delta))
    return bucketed.astype(np.int64)


def log_bucket_scalar(delta: int, bucket_size: int, max_position: int) -> int:
    """Pure-Python float64 bucket of one distance (for brute-force checks)."""

    mid = bucket_size // 2
    if abs(delta) <= mid:
        return delta
    value = math.ceil(math.log(abs(delta) / mid) / math.log((max_position - 1) / mid) * (mid - 1))
    return int(math.copysign(value + mid, delta))


def relative_positions(length: int, bucket_size: int, max_position: int) -> np.ndarray:
    """``build_relative_position`` for square self-attention: ``[L, L]`` of bucket(i - j)."""

    idx = np.arange(length)
    rel = idx[:, None] - idx[None, :]
    if bucket_size > 0 and max_position > 0:
        rel = log_bucket(rel, bucket_size, max_position)
    return rel.astype(np.int64)


def compact_plan(length: int, *, position_buckets: int, max_relative_positions: int,
                 position_embedding_size: int, uses_position_bias: bool = True):
    """``(active_slots int64 [S], delta_to_local int32 [2L-1])`` (``position.py:89-128``)."""

    if length < 1:
        raise ValueError("sequence_length must be positive")
    if not uses_position_bias:
        return np.zeros(0, np.int64), np.zeros(2 * length - 1, np.int32)
    deltas = np.arange(-(length - 1), length, dtype=np.int64)
    if position_buckets > 0:
        deltas = log_bucket(deltas, position_buckets, max_relative_positions)
    span = position_embedding_size
    slots = np.clip(deltas + span, 0, 2 * span - 1)
    active = np.unique(slots)
    lookup = np.searchsorted(active, slots).astype(np.int32)
    return active, lookup


def dense_map(lookup: np.ndarray, length: int) -> np.ndarray:
    """``pair_to_local[i, j] = delta_to_local[i - j + L - 1]`` (``position.py:130-156``)."""

    idx = np.arange(length)
    return lookup[idx[:, None] - idx[None, :] + length - 1].astype(np.int64)
