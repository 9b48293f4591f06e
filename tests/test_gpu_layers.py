"""Parity of the fused residual add + LayerNorm kernel (through the C ABI).

Reference: the float64 LayerNorm of the dtype-rounded sum ``T(x + r)``, which is
what ``LayerNorm(dense(x) + input_tensor)`` computes in the reference's
``DebertaV2SelfOutput``/``DebertaV2Output`` (``_reference.py:108-112, 482-485``):
the add rounds to the activation dtype, torch's LayerNorm normalises in fp32.
Tolerance: half an output ulp plus fp32 statistics error, written per dtype.
"""

from __future__ import annotations

import pytest
import torch
from torch.nn import functional as F

pytestmark = pytest.mark.gpu

DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
# |out - ref| <= REL * |ref| + ABS
TOLS = {torch.float16: (2.0 ** -10, 1e-3), torch.bfloat16: (2.0 ** -7, 8e-3),
        torch.float32: (1e-6, 1e-5)}


def _case(rows, hidden, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, hidden, generator=gen) * 0.7
    r = torch.randn(rows, hidden, generator=gen) * 1.3 + 0.25
    w = 1.0 + 0.1 * torch.randn(hidden, generator=gen)
    b = 0.1 * torch.randn(hidden, generator=gen)
    return [t.to("cuda", dtype) for t in (x, r, w, b)]


def _reference(x, r, w, b, eps):
    s = (x.float() + r.float()).to(x.dtype).double()
    return F.layer_norm(s, (s.shape[-1],), w.double(), b.double(), eps)


@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize("rows,hidden", [(1, 768), (37, 768), (4096, 768), (3, 1024),
                                         (65, 1536), (2, 36), (5, 4096), (9, 260)])
def test_add_layernorm_matches_float64(dtype, rows, hidden):
    from disentangled_flash.layers import add_layernorm

    x, r, w, b = _case(rows, hidden, DTYPES[dtype], rows * 7 + hidden)
    eps = 1e-7
    out = add_layernorm(x, r, w, b, eps)
    torch.cuda.synchronize()
    ref = _reference(x, r, w, b, eps)
    rel, abs_tol = TOLS[x.dtype]
    err = (out.double() - ref).abs()
    bound = rel * ref.abs() + abs_tol
    assert torch.isfinite(out).all()
    assert bool((err <= bound).all()), f"max err {err.max().item():.3e}"
    # torch's own fp-dtype pipeline (add, then LayerNorm) agrees to an output ulp.
    torch_out = F.layer_norm(x + r, (hidden,), w, b, eps)
    assert (out.double() - torch_out.double()).abs().max().item() <= 2 * bound.max().item()


def test_add_layernorm_zero_rows_and_errors():
    from disentangled_flash import _lib
    from disentangled_flash.layers import add_layernorm

    x = torch.empty(0, 768, device="cuda", dtype=torch.float16)
    w = torch.ones(768, device="cuda", dtype=torch.float16)
    assert add_layernorm(x, x, w, w, 1e-5).shape == (0, 768)
    lib = _lib.load()
    y = torch.zeros(8, 6, device="cuda", dtype=torch.float16)
    rc = lib.dflash_add_layernorm_fwd(y.data_ptr(), y.data_ptr(), y.data_ptr(), y.data_ptr(),
                                      y.data_ptr(), 8, 6, 1e-5, 0, None)
    assert rc == -2  # hidden not a multiple of 4


def test_output_block_matches_huggingface_modules():
    from transformers import DebertaV2Config
    from transformers.models.deberta_v2.modeling_deberta_v2 import (
        DebertaV2Output,
        DebertaV2SelfOutput,
    )

    from disentangled_flash.layers import fusable_output_block, output_block

    cfg = DebertaV2Config(hidden_size=768, intermediate_size=3072, hidden_dropout_prob=0.0,
                          layer_norm_eps=1e-7)
    torch.manual_seed(3)
    for cls, width in ((DebertaV2SelfOutput, 768), (DebertaV2Output, 3072)):
        module = cls(cfg).to("cuda", torch.float16).eval()
        with torch.no_grad():
            module.LayerNorm.weight.normal_(1.0, 0.1)
            module.LayerNorm.bias.normal_(0.0, 0.1)
        assert fusable_output_block(module)
        h = torch.randn(4, 33, width, device="cuda", dtype=torch.float16)
        res = torch.randn(4, 33, 768, device="cuda", dtype=torch.float16)
        with torch.inference_mode():
            expected = module(h, res)
            got = output_block(module, h, res)
        assert (got.float() - expected.float()).abs().max().item() <= 8e-3
