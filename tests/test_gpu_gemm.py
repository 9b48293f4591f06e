"""Parity of the hand-written gfx950 GEMM (``dflash_linear_fwd``) with a float64 matmul.

``y = epilogue(x @ W.T + b)`` for the three epilogues the encoder uses:
plain bias (fused QKV projection), exact-erf GELU of the dtype-rounded linear
output (FFN intermediate) and residual add of the dtype-rounded linear output
(attention output dense).  The reference is computed in float64 from the same
inputs with the same roundings in place; the GEMM accumulates in fp32, so it
may land one rounding step away at a tie and the bound is two units in the
last place of the output dtype at the reference's magnitude, plus the fp32
accumulation error (16 u * sum_k |x_k w_k|, which matters only for outputs near
zero), plus 2e-6 absolute for the GELU's erf approximation (Abramowitz &
Stegun 7.1.26, |error| <= 1.5e-7).
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

MANTISSA = {torch.float16: 10, torch.bfloat16: 7}
CONFIGS = {"auto": 0, "wide": 1, "pair": 2, "eight": 3, "small": 4, "tiny": 5}


def _ulp(ref: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    tiny = torch.finfo(dtype).tiny
    mag = ref.abs().clamp_min(tiny)
    return torch.exp2(torch.floor(torch.log2(mag)) - MANTISSA[dtype])


def _inputs(m, k, n, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=gen)
    w = torch.randn(n, k, generator=gen) / math.sqrt(k)
    b = torch.randn(n, generator=gen) * 0.1
    r = torch.randn(m, n, generator=gen)
    return tuple(t.to("cuda", dtype) for t in (x, w, b, r))


def _reference(x, w, b, r, epilogue, dtype):
    lin = (x.double() @ w.double().t() + b.double()).to(dtype).double()
    # Elementwise fp32 accumulation allowance: 16 u * (|x| @ |w|^T + |b|).
    acc = (x.double().abs() @ w.double().abs().t() + b.double().abs()) * 2.0 ** -20
    if epilogue == 1:
        return F.gelu(lin), lin, acc
    if epilogue == 2:
        return lin + r.double(), lin, acc
    return lin, lin, acc


def _run(x, w, b, r, epilogue, config=0):
    from disentangled_flash import _lib

    lib = _lib.load()
    y = torch.empty(x.shape[0], w.shape[0], device="cuda", dtype=x.dtype)
    code = lib.dflash_linear_fwd(x.data_ptr(), w.data_ptr(), b.data_ptr(),
                                 r.data_ptr() if r is not None else None, y.data_ptr(),
                                 x.shape[0], w.shape[0], x.shape[1], epilogue | (config << 8),
                                 _lib.DTYPE_CODES[x.dtype], torch.cuda.current_stream().cuda_stream)
    return code, y


def _check(y, ref, lin, acc, dtype, epilogue):
    tol = 2 * _ulp(ref, dtype) + acc
    if epilogue == 1:
        # One step of the rounded linear output moves GELU by at most 1.13 of
        # its ulp; the erf approximation adds < 1e-6 absolute.
        tol = tol + 1.2 * _ulp(lin, dtype) + 2e-6
    if epilogue == 2:
        tol = tol + _ulp(lin, dtype)
    excess = ((y.double() - ref).abs() - tol).max().item()
    err = (y.double() - ref).abs().max().item()
    return err, excess


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("epilogue", [0, 1, 2], ids=["bias", "gelu", "add"])
@pytest.mark.parametrize("shape", [(16384, 768, 2304), (16384, 768, 3072), (4096, 3072, 768),
                                   (300, 64, 384), (1, 32, 192), (257, 1536, 4608),
                                   (513, 96, 640), (16384, 64, 320)],
                         ids=lambda s: "x".join(map(str, s)))
def test_linear_matches_float64(dtype, epilogue, shape):
    m, k, n = shape
    x, w, b, r = _inputs(m, k, n, dtype, seed=m + k + n)
    ref, lin, acc = _reference(x, w, b, r, epilogue, dtype)
    for name, config in CONFIGS.items():
        if config in (1, 3) and n % 192 or config in (2, 4) and n % 128:
            continue
        # Widths that fit neither 128 nor 192 run the 64 x 64 tiles, forced or
        # automatic (at any row count).
        if config not in (0, 5) and n % 128 and n % 192:
            continue
        code, y = _run(x, w, b, r if epilogue == 2 else None, epilogue, config)
        assert code == 0, (name, code)
        torch.cuda.synchronize()
        err, excess = _check(y, ref, lin, acc, dtype, epilogue)
        print(f"{dtype} {shape} epi {epilogue} {name}: max|err| {err:.3e}")
        assert excess <= 0, f"{name}: error exceeds the bound by {excess:.3e}"


def test_linear_ops_and_errors():
    from disentangled_flash import _lib
    from disentangled_flash.layers import GEMM_BIAS_GELU, gemm_fits, linear_epilogue

    x, w, b, _ = _inputs(96, 64, 384, torch.float16, 1)
    y = linear_epilogue(x.view(2, 48, 64), w, b, None, GEMM_BIAS_GELU)
    ref, _, _ = _reference(x, w, b, None, 1, torch.float16)
    assert y.shape == (2, 48, 384)
    assert (y.view(96, 384).double() - ref).abs().max().item() < 5e-3
    assert gemm_fits(w, b) and not gemm_fits(w.float(), b.float()) and not gemm_fits(w, None)
    lib = _lib.load()
    # N not a multiple of 64, fp32, a missing residual: refused, nothing launched.
    code, _ = _run(x, w[:100], b[:100], None, 0)
    assert code == -2
    xf, wf, bf = x.float(), w.float(), b.float()
    assert _run(xf, wf, bf, None, 0)[0] == -4
    assert _run(x, w, b, None, 2)[0] == -1
    assert lib.dflash_linear_fwd(None, None, None, None, None, 0, 192, 32, 0, 0, None) == 0


def test_encoder_gemm_tails_match_modules(monkeypatch):
    """The fused tails against the HF module pieces they replace, in fp16."""

    from disentangled_flash import layers
    from disentangled_flash.layers import (
        fusable_intermediate,
        intermediate_block,
        output_block_gemm,
    )
    from transformers import DebertaV2Config
    from transformers.models.deberta_v2.modeling_deberta_v2 import (
        DebertaV2Intermediate,
        DebertaV2SelfOutput,
    )

    monkeypatch.setattr(layers, "HIP_GEMM_MIN_ROWS", 0)  # the hand-written GEMM at 520 rows
    cfg = DebertaV2Config(hidden_size=768, intermediate_size=3072, hidden_act="gelu",
                          hidden_dropout_prob=0.0, layer_norm_eps=1e-7)
    torch.manual_seed(3)
    inter = DebertaV2Intermediate(cfg).to("cuda", torch.float16).eval()
    out = DebertaV2SelfOutput(cfg).to("cuda", torch.float16).eval()
    assert fusable_intermediate(inter)
    h = torch.randn(4, 130, 768, device="cuda", dtype=torch.float16)
    res = torch.randn(4, 130, 768, device="cuda", dtype=torch.float16)
    with torch.inference_mode():
        got_i = intermediate_block(inter, h)
        want_i = inter.double()(h.double())
        got_o = output_block_gemm(out, h, res)
        want_o = out.double()(h.double(), res.double())
    err_i = (got_i.double() - want_i).abs().max().item()
    err_o = (got_o.double() - want_o).abs().max().item()
    print(f"intermediate {err_i:.3e}, self-output {err_o:.3e}")
    assert err_i <= 4e-3
    assert err_o <= 2e-2  # LayerNorm output of O(1) rows in fp16 (rstd ~ 1, two roundings)


def test_projection_dispatch_rules():
    """Which GEMM an encoder projection runs on, by rows, width and launch mode: the
    hand-written GEMM from HIP_GEMM_MIN_ROWS rows and in launch-bound eager forwards at
    base width; hipBLASLt otherwise, in particular while a HIP graph is captured."""

    from disentangled_flash import layers

    base = torch.zeros(1, 512, 768, device="cuda", dtype=torch.float16)      # 512 rows, K 768
    xlarge = torch.zeros(1, 512, 1536, device="cuda", dtype=torch.float16)   # K 1536
    big = torch.zeros(32, 512, 768, device="cuda", dtype=torch.float16)      # 16384 rows
    mid = torch.zeros(8, 512, 768, device="cuda", dtype=torch.float16)       # 4096 rows
    assert layers.hip_gemm_rows(base) and layers.hip_gemm_rows(base, 2304)
    assert layers.eager_small_gemm(torch.zeros(1, 512, 3072, device="cuda", dtype=torch.float16), 768)
    assert not layers.hip_gemm_rows(xlarge) and not layers.hip_gemm_rows(xlarge, 4608)
    assert layers.hip_gemm_rows(big) and not layers.eager_small_gemm(big, 768)
    assert not layers.hip_gemm_rows(mid)
    assert not layers.hip_gemm_rows(base.cpu())
    with layers.graph_gemm_choice():
        assert not layers.hip_gemm_rows(base) and layers.hip_gemm_rows(big)
    assert layers.hip_gemm_rows(base)
    graph = torch.cuda.CUDAGraph()
    seen = []
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side), torch.cuda.graph(graph, stream=side):
        seen.append((layers.hip_gemm_rows(base), layers.hip_gemm_rows(big)))
    torch.cuda.current_stream().wait_stream(side)
    assert seen == [(False, True)]
