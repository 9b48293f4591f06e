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


@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize("rows,hidden", [(1, 768), (4096, 768), (65, 1536), (2, 36), (9, 260)])
def test_layernorm_without_residual_matches_float64(dtype, rows, hidden):
    """The NULL-residual form (the attention-output block after the GEMM's add)."""

    from disentangled_flash.layers import layernorm

    x, _, w, b = _case(rows, hidden, DTYPES[dtype], rows * 11 + hidden)
    eps = 1e-7
    out = layernorm(x, w, b, eps)
    torch.cuda.synchronize()
    ref = F.layer_norm(x.double(), (hidden,), w.double(), b.double(), eps)
    rel, abs_tol = TOLS[x.dtype]
    err = (out.double() - ref).abs()
    assert bool((err <= rel * ref.abs() + abs_tol).all()), f"max err {err.max().item():.3e}"


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


# ConvLayer tail (reference _reference.py:519-566).  Reference: the module's
# steps in float64 from the exact convolution, rounding to the dtype wherever the
# module produces a tensor (convolution output, activation, residual sum,
# LayerNorm output, masked output).  The fused path rounds the fp32 sum of the
# three taps, so it may differ from the exactly rounded convolution by an ulp at
# a rounding boundary, which the later steps carry to about two output ulps:
# |out - ref| <= REL * |ref| + ABS.  The Hugging Face module itself (MIOpen
# convolution, bias added in the dtype) lands up to about three output ulps from
# the float64 steps, so the fused output is held to three times the band from it.
CONV_TOLS = {torch.float16: (2.0 ** -9, 2e-3), torch.bfloat16: (2.0 ** -6, 1.6e-2),
             torch.float32: (1e-5, 5e-5)}


def _conv_emulated(module, x, res, mask):
    dt = x.dtype
    conv = module.conv
    full = F.conv1d(x.double().transpose(1, 2), conv.weight.double(), conv.bias.double(),
                    padding=1).transpose(1, 2)
    c = full.to(dt).double() * (mask == 1)[..., None]
    act = {"gelu": F.gelu, "tanh": torch.tanh, "relu": torch.relu}[module.conv_act]
    a = act(c).to(dt).double()
    s = (res.double() + a).to(dt).double()
    norm = module.LayerNorm
    y = F.layer_norm(s, (s.shape[-1],), norm.weight.double(), norm.bias.double(), norm.eps)
    return (y.to(dt).double() * mask.to(dt).double()[..., None]).to(dt)


def _conv_module(hidden, act, dtype, seed):
    from transformers import DebertaV2Config
    from transformers.models.deberta_v2.modeling_deberta_v2 import ConvLayer

    cfg = DebertaV2Config(hidden_size=hidden, conv_kernel_size=3, conv_act=act,
                          hidden_dropout_prob=0.0, layer_norm_eps=1e-7)
    torch.manual_seed(seed)
    module = ConvLayer(cfg).eval()
    with torch.no_grad():
        module.conv.weight.normal_(0.0, 0.02)
        module.conv.bias.normal_(0.0, 0.05)
        module.LayerNorm.weight.normal_(1.0, 0.1)
        module.LayerNorm.bias.normal_(0.0, 0.1)
    return module.to("cuda", dtype)


@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize("act", ["gelu", "tanh", "relu"])
@pytest.mark.parametrize("batch,length,hidden", [(3, 37, 768), (2, 1, 64), (2, 130, 1536)])
def test_conv_layer_block_matches_huggingface(dtype, act, batch, length, hidden):
    from disentangled_flash.layers import conv_layer_block, conv_taps, fusable_conv_layer

    dt = DTYPES[dtype]
    module = _conv_module(hidden, act, dt, seed=batch * 100 + length)
    assert fusable_conv_layer(module)
    gen = torch.Generator().manual_seed(length)
    x = (torch.randn(batch, length, hidden, generator=gen) * 0.5).to("cuda", dt)
    res = torch.randn(batch, length, hidden, generator=gen).to("cuda", dt)
    lengths = torch.randint(1, length + 1, (batch,), generator=gen)
    mask = (torch.arange(length)[None] < lengths[:, None]).long().cuda()
    with torch.inference_mode():
        expected = module(x, res, mask)
        got = conv_layer_block(module, conv_taps(module), x, res, mask)
        got_bool = conv_layer_block(module, conv_taps(module), x, res, mask.bool())
    torch.cuda.synchronize()
    ref = _conv_emulated(module, x, res, mask).double()
    rel, abs_tol = CONV_TOLS[dt]
    bound = rel * ref.abs() + abs_tol
    err = (got.double() - ref).abs()
    assert torch.isfinite(got).all()
    assert bool((err <= bound).all()), f"max err vs float64 steps {err.max().item():.3e}"
    module_err = (got.double() - expected.double()).abs()
    assert bool((module_err <= 3 * bound).all()), f"max err vs module {module_err.max().item():.3e}"
    assert torch.equal(got, got_bool)  # a bool mask means the same as its 0/1 form
    # padded positions are exactly zero, as output * mask makes them
    assert bool((got[mask == 0] == 0).all())


def test_conv_layer_block_numeric_mask_values():
    """A numeric mask keeps the convolution only where it equals 1 and scales by it."""

    from disentangled_flash.layers import conv_layer_block, conv_taps

    module = _conv_module(256, "tanh", torch.float32, seed=5)
    x = torch.randn(2, 9, 256, device="cuda")
    res = torch.randn(2, 9, 256, device="cuda")
    mask = torch.tensor([[1, 1, 2, 0, 1, 1, 1, 0, 0], [1] * 9], device="cuda")
    with torch.inference_mode():
        expected = module(x, res, mask)
        got = conv_layer_block(module, conv_taps(module), x, res, mask)
    assert (got - expected).abs().max().item() <= 5e-5


def test_conv_layer_tail_rejects_bad_arguments():
    from disentangled_flash import _lib

    lib = _lib.load()
    y = torch.zeros(64, device="cuda")
    m = torch.ones(4, dtype=torch.int64, device="cuda")

    def call(z_dtype=2, batch=1, hidden=8, act=0):
        return lib.dflash_conv_layer_tail_fwd(y.data_ptr(), z_dtype, y.data_ptr(), y.data_ptr(),
                                              y.data_ptr(), y.data_ptr(), m.data_ptr(),
                                              y.data_ptr(), batch, 4, hidden, 1e-5, act, 2, None)

    assert call(act=7) == -2        # unknown activation
    assert call(hidden=6) == -2     # hidden not a multiple of 4
    assert call(z_dtype=1) == -4    # taps neither fp32 nor the dtype
    assert call(batch=0) == 0       # empty batch is a no-op


def test_hip_ops_run_their_fakes_under_fake_tensor_mode():
    """Under FakeTensorMode (as in non-strict export or opcheck) the HIP ops go
    through their registered fake implementations, not the C ABI."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    from disentangled_flash import layers

    with FakeTensorMode():
        x = torch.empty(4, 256, 768, device="cuda", dtype=torch.float16)
        w = torch.empty(2304, 768, device="cuda", dtype=torch.float16)
        b = torch.empty(2304, device="cuda", dtype=torch.float16)
        y = layers.linear_epilogue(x, w, b, None, layers.GEMM_BIAS)
        assert y.shape == (4, 256, 2304) and y.dtype == torch.float16


def test_linear_epilogue_checks_the_residual():
    from disentangled_flash import layers

    x = torch.randn(64, 256, device="cuda", dtype=torch.float16)
    w = torch.randn(128, 256, device="cuda", dtype=torch.float16) / 16
    b = torch.randn(128, device="cuda", dtype=torch.float16)
    good = torch.randn(64, 128, device="cuda", dtype=torch.float16)
    with pytest.raises(ValueError, match="needs a residual"):
        layers.linear_epilogue(x, w, b, None, layers.GEMM_BIAS_ADD)
    with pytest.raises(ValueError, match="shape"):
        layers.linear_epilogue(x, w, b, good[:32], layers.GEMM_BIAS_ADD)
    with pytest.raises(ValueError, match="dtype"):
        layers.linear_epilogue(x, w, b, good.float(), layers.GEMM_BIAS_ADD)
    with pytest.raises(ValueError, match="contiguous"):
        layers.linear_epilogue(x, w, b, good.t().contiguous().t(), layers.GEMM_BIAS_ADD)
    y = layers.linear_epilogue(x, w, b, good, layers.GEMM_BIAS_ADD)
    ref = (F.linear(x.double(), w.double(), b.double()).half().double() + good.double())
    assert (y.double() - ref).abs().max().item() < 2e-2
