"""The CPU oracle, pinned against golden vectors, closed forms and brute force."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import ATTENTION_CASES, GOLDEN, load_case
from oracle.attention import (
    AttentionSpec,
    brute_force_attention,
    fused_attention,
    original_attention,
    plan_for,
    project_relative,
    qkv_heads,
    reference_scale,
)
from oracle.optimized import optimized_attention
from oracle.positions import compact_plan, dense_map, log_bucket, log_bucket_scalar

# Closed-form active-slot counts for buckets=256, max_rel=512 (log-bucket formula).
ACTIVE_SLOTS = {16: 31, 32: 63, 64: 127, 65: 129, 128: 255, 129: 257, 256: 385, 384: 459,
                512: 511, 513: 512, 1024: 512}


def test_bucket_matches_huggingface_vectors():
    data = np.load(GOLDEN / "buckets.npz")
    deltas = data["deltas"].astype(np.int64)
    for key in data.files:
        if key == "deltas":
            continue
        size, maximum = (int(part[1:]) for part in key.split("_"))
        np.testing.assert_array_equal(log_bucket(deltas, size, maximum), data[key])


@pytest.mark.parametrize("size,maximum", [(256, 512), (16, 64), (64, 512), (8, 32), (256, 2048)])
def test_bucket_closed_form_properties(size, maximum):
    deltas = np.arange(-4000, 4001)
    b32 = log_bucket(deltas, size, maximum)
    b64 = log_bucket(deltas, size, maximum, dtype=np.float64)
    np.testing.assert_array_equal(b32, b64)                  # float32 == float64 log
    np.testing.assert_array_equal(b32, -b32[::-1])           # odd symmetry
    mid = size // 2
    band = np.abs(deltas) <= mid
    np.testing.assert_array_equal(b32[band], deltas[band])   # identity inside the band
    assert np.all(np.diff(b32) >= 0)                         # monotone
    scalar = [log_bucket_scalar(int(d), size, maximum) for d in deltas[::37]]
    np.testing.assert_array_equal(b32[::37], scalar)


def test_bucket_known_values():
    assert log_bucket(np.array([256]), 256, 512)[0] == 192
    assert log_bucket(np.array([511]), 256, 512)[0] == 255
    assert log_bucket(np.array([129]), 256, 512)[0] == 129
    assert log_bucket(np.array([-511]), 256, 512)[0] == -255


@pytest.mark.parametrize("length,expected", sorted(ACTIVE_SLOTS.items()))
def test_active_slot_counts(length, expected):
    active, lookup = compact_plan(length, position_buckets=256, max_relative_positions=512,
                                  position_embedding_size=256)
    assert active.size == expected
    assert lookup.shape == (2 * length - 1,)


def test_reference_position_test_case():
    # tests/test_position.py:6-16 of the reference: L=65 -> 129-entry LUT, <=129 slots.
    active, lookup = compact_plan(65, position_buckets=256, max_relative_positions=512,
                                  position_embedding_size=256)
    assert lookup.shape == (129,)
    assert active.ndim == 1 and active.size <= 129


@pytest.mark.parametrize("length,buckets,maximum,span", [(65, 256, 512, 256), (300, 16, 64, 16),
                                                         (40, -1, 16, 16), (700, 256, 512, 256)])
def test_compact_plan_brute_force(length, buckets, maximum, span):
    active, lookup = compact_plan(length, position_buckets=buckets, max_relative_positions=maximum,
                                  position_embedding_size=span)
    slots = {}
    for delta in range(-(length - 1), length):
        rel = log_bucket_scalar(delta, buckets, maximum) if buckets > 0 else delta
        slots[delta] = min(max(rel + span, 0), 2 * span - 1)
    assert list(active) == sorted(set(slots.values()))
    for delta, slot in slots.items():
        assert active[lookup[delta + length - 1]] == slot
    assert np.all(np.diff(lookup) >= 0)   # monotone: contiguous windows per tile


def test_dense_map_matches_lookup():
    _, lookup = compact_plan(20, position_buckets=8, max_relative_positions=32,
                             position_embedding_size=8)
    pair = dense_map(lookup, 20)
    for i in range(20):
        for j in range(20):
            assert pair[i, j] == lookup[i - j + 19]


@pytest.mark.parametrize("name", ATTENTION_CASES)
def test_original_matches_golden(name):
    spec, params, hidden, rel, mask, expected = load_case(name)
    got = original_attention(spec, params, hidden, rel, mask)
    np.testing.assert_allclose(got, expected, rtol=0, atol=1e-10)


@pytest.mark.parametrize("name", ATTENTION_CASES)
def test_fused_contract_matches_golden(name):
    spec, params, hidden, rel, mask, expected = load_case(name)
    length = hidden.shape[1]
    q, k, v = qkv_heads(spec, params, hidden)
    pos_key, pos_query = project_relative(spec, params, rel)
    active, lookup = plan_for(spec, length)
    pk = pos_key[:, active] if pos_key is not None else None
    pq = pos_query[:, active] if pos_query is not None else None
    got = fused_attention(q, k, v, pk, pq, lookup, mask, reference_scale(spec.head_dim, spec.scale_factor),
                          "c2p" in spec.pos_att_type, "p2c" in spec.pos_att_type)
    np.testing.assert_allclose(got, expected, rtol=0, atol=1e-10)


@pytest.mark.parametrize("name", ["v3_small", "c2p_separate_buckets16", "p2c_d128_unbucketed"])
def test_brute_force_matches_golden(name):
    spec, params, hidden, rel, mask, expected = load_case(name)
    hidden = hidden[:, :12]
    mask = mask[:, :12]
    q, k, v = qkv_heads(spec, params, hidden)
    pos_key, pos_query = project_relative(spec, params, rel)
    got = brute_force_attention(q, k, v, pos_key, pos_query, mask,
                                reference_scale(spec.head_dim, spec.scale_factor), spec.span,
                                spec.position_buckets, spec.max_relative_positions,
                                "c2p" in spec.pos_att_type, "p2c" in spec.pos_att_type)
    ref = original_attention(spec, params, hidden, rel, mask)
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-10)


def _random_heads(rng, b, h, length, d):
    return [rng.normal(0, 1, (b, h, length, d)) / math.sqrt(d) for _ in range(3)]


def test_no_relative_terms_is_textbook_sdpa():
    rng = np.random.default_rng(3)
    q, k, v = _random_heads(rng, 2, 3, 17, 32)
    mask = np.ones((2, 17), bool)
    got = fused_attention(q, k, v, None, None, np.zeros(33, np.int32), mask, math.sqrt(32),
                          False, False)
    ref = torch.nn.functional.scaled_dot_product_attention(
        *(torch.from_numpy(t) for t in (q, k, v)))
    ref = ref.permute(0, 2, 1, 3).reshape(2, 17, 96).numpy()
    np.testing.assert_allclose(got, ref, atol=1e-12)


def test_padded_rows_are_mean_of_values_and_length_one_is_identity():
    rng = np.random.default_rng(5)
    q, k, v = _random_heads(rng, 2, 2, 9, 32)
    active, lookup = compact_plan(9, position_buckets=256, max_relative_positions=512,
                                  position_embedding_size=256)
    rows = rng.normal(0, 1, (2, active.size, 32))
    mask = np.array([[1] * 5 + [0] * 4, [0] * 9], bool)
    out = fused_attention(q, k, v, rows, rows, lookup, mask, math.sqrt(96), True, True)
    out = out.reshape(2, 9, 2, 32)
    mean_v = v.mean(axis=2)                       # [B, H, d]
    for i in range(5, 9):
        np.testing.assert_allclose(out[0, i], mean_v[0], atol=1e-12)
    for i in range(9):
        np.testing.assert_allclose(out[1, i], mean_v[1], atol=1e-12)
    single = fused_attention(q[:, :, :1], k[:, :, :1], v[:, :, :1], rows, rows,
                             np.zeros(1, np.int32), np.ones((2, 1), bool), 1.0, True, True)
    np.testing.assert_allclose(single.reshape(2, 1, 2, 32), v[:, :, :1].transpose(0, 2, 1, 3),
                               atol=1e-12)


@pytest.mark.parametrize("name", ["v3_small", "c2p_separate_buckets16", "fully_masked_row"])
def test_optimized_restatement_matches_original(name):
    spec, params, hidden, rel, mask, expected = load_case(name)
    length = hidden.shape[1]
    pos_key, pos_query = project_relative(spec, params, rel)
    active, lookup = plan_for(spec, length)
    weight = np.concatenate([params["query_weight"], params["key_weight"], params["value_weight"]])
    bias = np.concatenate([params["query_bias"], params["key_bias"], params["value_bias"]])
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).double()  # noqa: E731
    got = optimized_attention(
        t(hidden), t(weight), t(bias),
        t(pos_key[:, active]) if pos_key is not None else None,
        t(pos_query[:, active]) if pos_query is not None else None,
        torch.from_numpy(dense_map(lookup, length)), torch.from_numpy(mask),
        spec.num_heads, spec.head_dim)
    # The prepared path divides by the exact math.sqrt scale (_torch.py:168-169);
    # the original path by its float32 rounding, hence the looser golden check.
    exact = original_attention(spec, params, hidden, rel, mask,
                               scale=math.sqrt(spec.head_dim * spec.scale_factor))
    np.testing.assert_allclose(got.numpy(), exact, atol=1e-10)
    np.testing.assert_allclose(got.numpy(), expected, atol=1e-6)


def test_spec_defaults():
    spec = AttentionSpec(hidden_size=768, num_heads=12, head_dim=64)
    assert spec.span == 256 and spec.scale_factor == 3


def test_float64_buckets_differ_from_float32_somewhere():
    """Why the position plan stays on the host, as in the reference (``position.py:104-110``).

    The reference buckets deltas with a float32 log on the CPU.  A float64 (or
    device) log gives another bucket where ``log(|d| / mid) / log((max - 1) / mid) * (mid - 1)``
    lies within float32 rounding of an integer: at buckets 256 / max_position 256,
    |d| = 1292 is bucket 555 in exact arithmetic and 554 in the reference's float32.
    For the encoder configurations here (256 buckets, max_position 512) the two agree.
    """

    from disentangled_flash.modeling import make_log_bucket_position

    deltas = np.array([-1292, 1292], dtype=np.int64)
    exact = np.array([log_bucket_scalar(int(d), 256, 256) for d in deltas])
    assert list(exact) == [-555, 555]
    assert list(log_bucket(deltas, 256, 256, dtype=np.float64)) == [-555, 555]
    ref = make_log_bucket_position(torch.from_numpy(deltas), 256, 256).to(torch.long).numpy()
    assert list(ref) == [-554, 554]
    assert list(log_bucket(deltas, 256, 256)) == [-554, 554]  # the float32 restatement agrees

    span = np.arange(-8191, 8192)
    ref = make_log_bucket_position(torch.from_numpy(span), 256, 512).to(torch.long).numpy()
    assert np.array_equal(ref, log_bucket(span, 256, 512, dtype=np.float64))


def test_reference_scale_casts_like_the_original_path():
    """Known answers for the original path's scale quirk: sqrt(float32(d) * f) cast to
    the activation dtype before dividing (``_reference.py:161-162,285``).  For d = 64,
    f = 3 the exact value 13.8564... becomes 13.859375 in fp16 and 13.875 in bf16."""

    import torch

    assert reference_scale(64, 3) == np.float32(np.sqrt(np.float32(192.0)))
    assert reference_scale(64, 3, np.float16) == 13.859375
    bf16 = float(torch.tensor(reference_scale(64, 3), dtype=torch.float32).to(torch.bfloat16))
    assert bf16 == 13.875
    assert reference_scale(64, 1, np.float16) == 8.0  # exact: no rounding at f = 1
