"""Pins ``tests/gpu_reference.fused_reference`` (the GPU tests' large-shape checker).

The GPU parity tests at full size compare the kernel with ``fused_reference``,
a torch float64 statement of the fused contract.  Here, on the CPU, it is held
to the golden vectors (transformers' original attention in float64) and to the
oracle's ``fused_attention`` over every relative mode, ragged and fully masked
rows, L = 1, a non-monotone lookup table and split chunking, at 1e-12.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import ATTENTION_CASES, load_case
from gpu_reference import fused_reference
from oracle.attention import (
    fused_attention,
    plan_for,
    project_relative,
    qkv_heads,
    reference_scale,
)
from oracle.positions import compact_plan

MODES = {"both": (True, True), "c2p": (True, False), "p2c": (False, True), "none": (False, False)}


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float64))


def _run_reference(q, k, v, pk, pq, lut, mask, scale, has_c2p, has_p2c, chunk=4):
    heads, d = q.shape[1], q.shape[3]
    dummy = np.zeros((heads, 1, d))
    got = fused_reference(_t(q), _t(k), _t(v), _t(pk if pk is not None else dummy),
                          _t(pq if pq is not None else dummy), torch.from_numpy(lut),
                          torch.from_numpy(np.asarray(mask, bool)), scale, has_c2p, has_p2c,
                          chunk=chunk)
    return got.numpy()


@pytest.mark.parametrize("name", ATTENTION_CASES)
def test_fused_reference_matches_golden(name):
    spec, params, hidden, rel, mask, expected = load_case(name)
    q, k, v = qkv_heads(spec, params, hidden)
    pos_key, pos_query = project_relative(spec, params, rel)
    active, lookup = plan_for(spec, hidden.shape[1])
    pk = pos_key[:, active] if pos_key is not None else None
    pq = pos_query[:, active] if pos_query is not None else None
    has_c2p, has_p2c = "c2p" in spec.pos_att_type, "p2c" in spec.pos_att_type
    got = _run_reference(q, k, v, pk, pq, lookup, mask,
                         reference_scale(spec.head_dim, spec.scale_factor), has_c2p, has_p2c)
    np.testing.assert_allclose(got, expected, rtol=0, atol=1e-10)


def _random_case(seed, batch, heads, length, dim, lengths, lut_kind="plan"):
    rng = np.random.default_rng(seed)
    active, lut = compact_plan(length, position_buckets=256, max_relative_positions=512,
                               position_embedding_size=256)
    slots = active.size
    if lut_kind == "shuffled":
        # Non-monotone table: every delta gets an arbitrary slot.
        lut = rng.integers(0, slots, size=2 * length - 1).astype(np.int32)
    q, k, v = (rng.standard_normal((batch, heads, length, dim)) for _ in range(3))
    pk, pq = (rng.standard_normal((heads, slots, dim)) for _ in range(2))
    mask = np.arange(length)[None] < np.asarray(lengths)[:, None]
    return q, k, v, pk, pq, lut, mask


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("lut_kind", ["plan", "shuffled"])
def test_fused_reference_matches_oracle(mode, lut_kind):
    has_c2p, has_p2c = MODES[mode]
    # Ragged rows, a fully masked sequence and a full one; batch 5 with chunk 2
    # exercises the chunk loop and its ragged last chunk.
    q, k, v, pk, pq, lut, mask = _random_case(11, 5, 3, 37, 16, [37, 20, 0, 1, 36], lut_kind)
    scale = float(np.sqrt(16 * (1 + has_c2p + has_p2c)))
    want = fused_attention(q, k, v, pk, pq, lut, mask, scale, has_c2p, has_p2c)
    got = _run_reference(q, k, v, pk, pq, lut, mask, scale, has_c2p, has_p2c, chunk=2)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-12)


@pytest.mark.parametrize("mode", ["both", "p2c"])
def test_fused_reference_length_one_and_long_plan(mode):
    has_c2p, has_p2c = MODES[mode]
    for length, lengths in ((1, [1, 0]), (300, [300, 129])):
        q, k, v, pk, pq, lut, mask = _random_case(3 + length, 2, 2, length, 8, lengths)
        scale = float(np.sqrt(8 * (1 + has_c2p + has_p2c)))
        want = fused_attention(q, k, v, pk, pq, lut, mask, scale, has_c2p, has_p2c)
        got = _run_reference(q, k, v, pk, pq, lut, mask, scale, has_c2p, has_p2c)
        np.testing.assert_allclose(got, want, rtol=0, atol=1e-12)
        if length == 1:
            # One key: every row's output is V itself.
            np.testing.assert_allclose(got, v.transpose(0, 2, 1, 3).reshape(2, 1, -1),
                                       rtol=0, atol=1e-12)


def test_fused_reference_rounds_tables_like_the_score_gemms():
    # round_tables_to rounds the unscaled c2p/p2c tables to the dtype; with
    # tables whose products are exact in fp16 it equals the unrounded result.
    q, k, v, pk, pq, lut, mask = _random_case(5, 2, 2, 24, 8, [24, 10])
    q, k, pk, pq = (np.round(a * 4) / 4 for a in (q, k, pk, pq))
    scale = float(np.sqrt(24))
    exact = _run_reference(q, k, v, pk, pq, lut, mask, scale, True, True)
    rounded = fused_reference(_t(q), _t(k), _t(v), _t(pk), _t(pq), torch.from_numpy(lut),
                              torch.from_numpy(mask), scale, True, True,
                              round_tables_to=torch.float16).numpy()
    np.testing.assert_allclose(rounded, exact, rtol=0, atol=1e-12)
