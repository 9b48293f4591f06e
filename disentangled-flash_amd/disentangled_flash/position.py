"""Model-wide relative-position index plans (reference ``position.py:17-156``).

A plan depends only on the bucketing configuration, the sequence length and
the device, never on layer weights, so one cache serves every encoder layer.

``compact(L)`` returns the sorted set of relative-embedding rows ("active
slots") that an ``L``-token sequence can touch and an int32 lookup table
``delta_to_local[i - j + L - 1]`` giving the position of ``slot(i - j)`` inside
that set.  The fused HIP kernel reads this table for every delta of a tile's
window and gathers the projected position row of each delta, so it accepts any
table (monotone or not); the log-bucket tables built here happen to be monotone
in ``i - j``.

``dense(L)`` adds the ``[1, 1, L, L]`` int64 gather map that the unfused
PyTorch path uses.
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from .modeling import make_log_bucket_position


class SharedPositionIndexPlan(NamedTuple):
    """Compact ``O(L)`` plan: active slots and the delta lookup table."""

    sequence_length: int
    active_slots: torch.Tensor
    delta_to_local: torch.Tensor


class SharedDensePositionIndexPlan(NamedTuple):
    """Compact plan plus the shared dense ``[1, 1, L, L]`` gather map."""

    compact: SharedPositionIndexPlan
    pair_to_local: torch.Tensor

    @property
    def sequence_length(self) -> int:
        return self.compact.sequence_length

    @property
    def active_slots(self) -> torch.Tensor:
        return self.compact.active_slots


def canonical_device(
    requested: torch.device | str | None,
    resident: torch.device,
) -> torch.device:
    """Resolve an index-less device name (``"cuda"``) to the resident device."""

    resolved = torch.device(requested) if requested is not None else resident
    if resolved.type == resident.type and resolved.index is None:
        return resident
    return resolved


def compact_position_plan(
    sequence_length: int,
    *,
    position_buckets: int,
    max_relative_positions: int,
    position_embedding_size: int,
    uses_position_bias: bool = True,
) -> tuple[torch.Tensor, torch.Tensor]:
    """CPU ``(active_slots int64 [S], delta_to_local int32 [2L-1])`` (``position.py:89-128``)."""

    if sequence_length < 1:
        raise ValueError("sequence_length must be positive")
    if not uses_position_bias:
        return (
            torch.empty(0, dtype=torch.long),
            torch.zeros(2 * sequence_length - 1, dtype=torch.int32),
        )
    deltas = torch.arange(-(sequence_length - 1), sequence_length, dtype=torch.long)
    if position_buckets > 0:
        deltas = make_log_bucket_position(deltas, position_buckets, max_relative_positions).to(
            torch.long
        )
    slots = torch.clamp(deltas + position_embedding_size, 0, 2 * position_embedding_size - 1)
    active = torch.unique(slots, sorted=True)
    lookup = torch.searchsorted(active, slots).to(torch.int32)
    return active, lookup


class SharedPositionPlanCache:
    """Per-(length, device) cache of immutable position index tensors."""

    def __init__(
        self,
        *,
        position_buckets: int,
        max_relative_positions: int,
        position_embedding_size: int,
        uses_position_bias: bool = True,
    ) -> None:
        self.position_buckets = position_buckets
        self.max_relative_positions = max_relative_positions
        self.position_embedding_size = position_embedding_size
        self.uses_position_bias = uses_position_bias
        self._compact: dict[tuple[int, str], SharedPositionIndexPlan] = {}
        self._dense: dict[tuple[int, str], SharedDensePositionIndexPlan] = {}

    def clear(self) -> None:
        self._compact.clear()
        self._dense.clear()

    @staticmethod
    def _key(sequence_length: int, device: torch.device | str) -> tuple[int, str, torch.device]:
        if sequence_length < 1:
            raise ValueError("sequence_length must be positive")
        resolved = torch.device(device)
        return sequence_length, str(resolved), resolved

    @torch.no_grad()
    def compact(self, sequence_length: int, device: torch.device | str) -> SharedPositionIndexPlan:
        length, name, resolved = self._key(sequence_length, device)
        hit = self._compact.get((length, name))
        if hit is not None:
            return hit
        active, lookup = compact_position_plan(
            length,
            position_buckets=self.position_buckets,
            max_relative_positions=self.max_relative_positions,
            position_embedding_size=self.position_embedding_size,
            uses_position_bias=self.uses_position_bias,
        )
        plan = SharedPositionIndexPlan(
            sequence_length=length,
            active_slots=active.to(device=resolved),
            delta_to_local=lookup.to(device=resolved),
        )
        self._compact[(length, name)] = plan
        return plan

    @torch.no_grad()
    def dense(
        self, sequence_length: int, device: torch.device | str
    ) -> SharedDensePositionIndexPlan:
        length, name, resolved = self._key(sequence_length, device)
        hit = self._dense.get((length, name))
        if hit is not None:
            return hit
        compact = self.compact(length, resolved)
        positions = torch.arange(length, dtype=torch.long)
        delta_index = positions[:, None] - positions[None, :] + (length - 1)
        pair = compact.delta_to_local.cpu()[delta_index].to(device=resolved, dtype=torch.long)
        plan = SharedDensePositionIndexPlan(compact=compact, pair_to_local=pair[None, None])
        self._dense[(length, name)] = plan
        return plan


__all__ = [
    "SharedDensePositionIndexPlan",
    "SharedPositionIndexPlan",
    "SharedPositionPlanCache",
    "canonical_device",
    "compact_position_plan",
]
