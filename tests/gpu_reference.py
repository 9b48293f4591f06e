"""Float64 torch statement of the fused-kernel contract, for large GPU checks.

Same equation as ``oracle.attention.fused_attention``, written with torch so
that shapes like B=32, L=512 run on the GPU in float64 in well under a second.
``tests/test_gpu_reference_pin.py`` holds it to the golden vectors and to the
oracle (every mode, masked rows, L=1, non-monotone tables) on the CPU.  Tests
only.
"""

from __future__ import annotations

import torch


def fused_reference(q, k, v, pos_key, pos_query, lut, mask, scale, has_c2p, has_p2c,
                    chunk: int = 4, round_tables_to=None):
    """``q/k/v [B, H, L, d]``, ``pos_* [H, S, d]``, ``lut [2L-1]``, ``mask [B, L]`` -> ``[B, L, H*d]``.

    ``round_tables_to`` rounds the unscaled c2p/p2c score tables to that dtype
    before use, as the reference does when its separate score GEMMs run in
    fp16/bf16 (``kernel.py:577,583``).
    """

    b, h, length, d = q.shape
    out = torch.empty((b, length, h * d), dtype=torch.float64, device=q.device)
    idx = torch.arange(length, device=q.device)
    slot = lut.long()[idx[:, None] - idx[None, :] + length - 1]          # [L, L]
    m = mask.bool()
    for start in range(0, b, chunk):
        sl = slice(start, min(b, start + chunk))
        qd, kd, vd = (t[sl].double() for t in (q, k, v))
        scores = qd @ kd.transpose(-1, -2)
        nb = qd.shape[0]
        if has_c2p:
            raw = qd @ pos_key.double().transpose(-1, -2)                # [nb, H, L, S]
            if round_tables_to is not None:
                raw = raw.to(round_tables_to).double()
            scores += torch.gather(raw, -1, slot.expand(nb, h, length, length))
        if has_p2c:
            raw = kd @ pos_query.double().transpose(-1, -2)              # [nb, H, L(key), S]
            if round_tables_to is not None:
                raw = raw.to(round_tables_to).double()
            scores += torch.gather(raw, -1, slot.t().expand(nb, h, length, length)).transpose(-1, -2)
        scores = scores / scale
        mk = m[sl]
        kept = mk[:, None, :, None] & mk[:, None, None, :]
        scores = scores.masked_fill(~kept, float("-inf"))
        scores = scores.masked_fill(~mk[:, None, :, None], 0.0)
        probs = torch.softmax(scores, dim=-1)
        out[sl] = (probs @ vd).permute(0, 2, 1, 3).reshape(nb, length, h * d)
    return out
