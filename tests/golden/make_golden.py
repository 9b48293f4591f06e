"""Write the golden vectors in ``tests/golden/`` (run in a container with transformers).

The reference's ``original`` backend is a verbatim copy of Hugging Face
Transformers' ``DisentangledSelfAttention`` (reference ``_reference.py:14-22``,
``THIRD_PARTY_NOTICES.md``).  The installed ``transformers`` (5.15.0) carries
the same equation (``models/deberta_v2/modeling_deberta_v2.py``), so the
vectors come from that library, run in float64 on the CPU.  Inputs are drawn
from numpy ``default_rng`` seeds and stored with the outputs.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import types
from pathlib import Path

import numpy as np
import torch
import transformers
from transformers.models.deberta_v2 import modeling_deberta_v2 as hf

HERE = Path(__file__).resolve().parent

CASES = {
    # name: (hidden, heads, head_dim, batch, length, modes, share, buckets, max_rel, lengths)
    "v3_small": (128, 2, 64, 2, 65, ("c2p", "p2c"), True, 256, 512, (65, 37)),
    "c2p_separate_buckets16": (128, 4, 32, 2, 40, ("c2p",), False, 16, 64, (40, 1)),
    "p2c_d128_unbucketed": (128, 1, 128, 1, 24, ("p2c",), False, -1, 16, (20,)),
    "length1": (64, 2, 32, 2, 1, ("c2p", "p2c"), True, 256, 512, (1, 0)),
    "fully_masked_row": (64, 1, 64, 2, 33, ("p2c", "c2p"), True, 8, 32, (0, 33)),
    "no_relative": (64, 2, 32, 1, 17, (), True, 256, 512, (11,)),
}

BUCKET_CONFIGS = [(256, 512), (16, 64), (64, 512), (256, 2048), (8, 32)]


def make_case(name, hidden, heads, head_dim, batch, length, modes, share, buckets, max_rel,
              lengths, seed):
    rng = np.random.default_rng(seed)
    cfg = types.SimpleNamespace(
        hidden_size=hidden, num_attention_heads=heads, attention_head_size=head_dim,
        share_att_key=share, pos_att_type=list(modes), relative_attention=True,
        position_buckets=buckets, max_relative_positions=max_rel,
        max_position_embeddings=512, hidden_dropout_prob=0.0,
        attention_probs_dropout_prob=0.0,
    )
    module = hf.DisentangledSelfAttention(cfg).double().eval()
    arrays = {}
    with torch.no_grad():
        for pname, param in module.named_parameters():
            std = 0.2 if pname.endswith("weight") else 0.1
            value = rng.normal(0.0, std, size=tuple(param.shape)).astype(np.float32)
            param.copy_(torch.from_numpy(value))
            arrays["param." + pname] = value
    span = buckets if buckets > 0 else max_rel
    rel = rng.normal(0.0, 1.0, size=(2 * span, hidden)).astype(np.float32)
    states = rng.normal(0.0, 1.0, size=(batch, length, hidden)).astype(np.float32)
    mask = (np.arange(length)[None, :] < np.asarray(lengths)[:, None])
    pair = torch.from_numpy(mask)[:, None, None, :] & torch.from_numpy(mask)[:, None, :, None]
    with torch.no_grad():
        out, _ = module(
            torch.from_numpy(states).double(),
            pair,
            rel_embeddings=torch.from_numpy(rel).double(),
        )
    arrays.update(hidden=states, rel=rel, mask=mask.astype(np.uint8), out=out.numpy())
    meta = np.array([hidden, heads, head_dim, batch, length, int(share), buckets, max_rel])
    arrays["meta"] = meta
    arrays["modes"] = np.array(",".join(modes))
    np.savez_compressed(HERE / f"attention_{name}.npz", **arrays)


def make_buckets():
    arrays = {}
    deltas = torch.arange(-2047, 2048, dtype=torch.long)
    for size, maximum in BUCKET_CONFIGS:
        value = hf.make_log_bucket_position(deltas, size, maximum).to(torch.long)
        arrays[f"b{size}_m{maximum}"] = value.numpy().astype(np.int16)
    arrays["deltas"] = deltas.numpy().astype(np.int16)
    np.savez_compressed(HERE / "buckets.npz", **arrays)


def main():
    print("transformers", transformers.__version__)
    make_buckets()
    for seed, (name, spec) in enumerate(CASES.items()):
        make_case(name, *spec, seed=1000 + seed)
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
