"""Shared pytest setup: import paths, the ``gpu`` marker and golden-vector loading."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]
PACKAGE_DIR = REPO / "disentangled-flash_amd"
GOLDEN = REPO / "tests" / "golden"
for entry in (str(PACKAGE_DIR), str(REPO)):
    if entry not in sys.path:
        sys.path.insert(0, entry)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


ATTENTION_CASES = sorted(p.stem[len("attention_"):] for p in GOLDEN.glob("attention_*.npz"))


def load_case(name: str):
    """Golden case -> (spec, params, hidden, rel, mask, expected)."""

    from oracle.attention import AttentionSpec

    data = np.load(GOLDEN / f"attention_{name}.npz")
    hidden, heads, head_dim, _batch, _length, share, buckets, max_rel = (int(x) for x in data["meta"])
    modes = tuple(m for m in str(data["modes"]).split(",") if m)
    spec = AttentionSpec(hidden_size=hidden, num_heads=heads, head_dim=head_dim,
                         position_buckets=buckets, max_relative_positions=max_rel,
                         pos_att_type=modes, share_att_key=bool(share))
    params = {}
    for key in data.files:
        if key.startswith("param."):
            name_ = key[len("param."):].replace("_proj.", "_")
            params[name_] = data[key].astype(np.float64)
    return spec, params, data["hidden"], data["rel"], data["mask"].astype(bool), data["out"]


@pytest.fixture(scope="session")
def golden_dir() -> Path:
    return GOLDEN
