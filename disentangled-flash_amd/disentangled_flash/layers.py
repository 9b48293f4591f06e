"""Fused encoder-layer tails for the HIP backend.

``DebertaV2SelfOutput`` and ``DebertaV2Output`` (reference ``_reference.py:101-112``
and ``474-485``) both end in ``LayerNorm(dense(x) + input_tensor)``.  The HIP
encoder keeps the dense projection on hipBLASLt (``F.linear`` with its bias
epilogue) and replaces the separate residual add and LayerNorm with one
kernel, ``disentangled_flash::add_layernorm``, which reads the projection and
the residual once and writes the normalised row.

The ``ConvLayer`` run after the first encoder layer (reference
``_reference.py:519-566``, called at ``deberta.py:272-273``) is fused the same
way: its Conv1d (kernel 3, padding 1) becomes one library GEMM of the layer
input with the three taps side by side, and one kernel,
``disentangled_flash::conv_layer_tail``, sums the taps of neighbouring rows and
applies the mask, activation, residual add, LayerNorm and output mask.

The ops have fake implementations so that ``torch.compile(fullgraph=True)``
traces through them, like the attention ops.
"""

from __future__ import annotations

import contextlib
import threading

import torch
from torch import nn
from torch.nn import functional as F

from . import _lib


@_lib.hip_op("disentangled_flash::add_layernorm")
def add_layernorm(
    x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float
) -> torch.Tensor:
    """``LayerNorm(x + residual)`` over the last dimension; the sum is rounded to the dtype first."""

    lib = _lib.load()
    hidden = x.shape[-1]
    rows = x.numel() // hidden if hidden else 0
    out = torch.empty_like(x)
    code = lib.dflash_add_layernorm_fwd(
        x.data_ptr(),
        residual.data_ptr(),
        weight.data_ptr(),
        bias.data_ptr(),
        out.data_ptr(),
        rows,
        hidden,
        float(eps),
        _lib.DTYPE_CODES[x.dtype],
        _lib.current_stream_handle(x.device),
    )
    _lib.check(code, "dflash_add_layernorm_fwd")
    return out


@add_layernorm.register_fake
def _add_layernorm_fake(x, residual, weight, bias, eps):
    return torch.empty_like(x)


@_lib.hip_op("disentangled_flash::layernorm")
def layernorm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float) -> torch.Tensor:
    """``LayerNorm(x)`` over the last dimension (statistics in fp32)."""

    lib = _lib.load()
    hidden = x.shape[-1]
    rows = x.numel() // hidden if hidden else 0
    out = torch.empty_like(x)
    code = lib.dflash_add_layernorm_fwd(
        x.data_ptr(), None, weight.data_ptr(), bias.data_ptr(), out.data_ptr(), rows, hidden,
        float(eps), _lib.DTYPE_CODES[x.dtype], _lib.current_stream_handle(x.device))
    _lib.check(code, "dflash_add_layernorm_fwd")
    return out


@layernorm.register_fake
def _layernorm_fake(x, weight, bias, eps):
    return torch.empty_like(x)


# Whether the encoder runs its projections on the hand-written GEMM
# (dflash_linear_fwd) where it fits, or on hipBLASLt through F.linear; read when
# an encoder is prepared and on every QKV projection.  A switch for A/B timing.
USE_HIP_GEMM = True

# Which GEMM runs an encoder projection, by rows (tokens, M = B*L), width and
# launch mode.  Measured on whole encoders (12-layer base fp16, 24-layer xlarge
# bf16) and per GEMM in HIP graphs:
#   * HIP-graph replay: below HIP_GEMM_MIN_ROWS rows hipBLASLt (plus a separate
#     GELU) is faster on the device, up to 1.5x at 512 rows; at 16384 rows the
#     two tie;
#   * eager, up to HIP_GEMM_EAGER_MAX_ROWS rows: the forward is bound by launch
#     time, and an F.linear call costs about 19 us of hipBLASLt host time against
#     a few for the hand-written GEMM.  For base-width projections (N or K at
#     most HIP_GEMM_EAGER_MAX_WIDTH) that wins (1.85 -> 1.37 ms per forward at
#     B*L <= 2048; 0.8-1.0 ms with the library's 64-row tiles at these rows);
#     for the xlarge widths (N, K >= 1536) the hand-written kernel's device time
#     outweighs it (3.47 -> 3.82 ms), and from about 4096 rows eager forwards are
#     device-bound again.
# So: the hand-written GEMM from HIP_GEMM_MIN_ROWS rows (QKV, attention-output
# dense, FFN intermediate; the FFN output dense, K = 4 x hidden, stays on
# hipBLASLt there), and in eager forwards up to HIP_GEMM_EAGER_MAX_ROWS rows at
# base width; hipBLASLt otherwise, and always while a HIP graph is being captured
# or torch.compile traces.  Checked on every call: the layer program binds the
# fused steps once per bucket, while B varies per call.
HIP_GEMM_MIN_ROWS = 16384
HIP_GEMM_EAGER_MAX_ROWS = 2048
HIP_GEMM_EAGER_MAX_WIDTH = 768

_GRAPH_CHOICE = threading.local()


@contextlib.contextmanager
def graph_gemm_choice():
    """Eager forwards inside this block (on this thread) pick their GEMMs as HIP-graph
    capture does (hipBLASLt below :data:`HIP_GEMM_MIN_ROWS` rows), so they reproduce a
    captured bucket's replays bit for bit."""

    saved = getattr(_GRAPH_CHOICE, "on", False)
    _GRAPH_CHOICE.on = True
    try:
        yield
    finally:
        _GRAPH_CHOICE.on = saved


def eager_small_gemm(x: torch.Tensor, n: int) -> bool:
    """True for an eager ``[..., K] x [N, K]^T`` projection small enough to be
    launch-bound, at base width (see the rules above)."""

    k = x.shape[-1]
    if k <= 0 or x.device.type != "cuda" or torch.compiler.is_compiling():
        return False
    if x.numel() // k > HIP_GEMM_EAGER_MAX_ROWS or min(k, n) > HIP_GEMM_EAGER_MAX_WIDTH:
        return False
    if getattr(_GRAPH_CHOICE, "on", False):
        return False
    return not torch.cuda.is_current_stream_capturing()


def hip_gemm_rows(x: torch.Tensor, n: int | None = None) -> bool:
    """True if the projection of ``x`` (``[..., K]``) to ``n`` columns (default K)
    runs on the hand-written GEMM."""

    k = x.shape[-1]
    if k <= 0 or x.device.type != "cuda":
        return False
    if x.numel() // k >= HIP_GEMM_MIN_ROWS:
        return True
    return eager_small_gemm(x, k if n is None else n)


# Tile configuration the encoder asks dflash_linear_fwd for (bits 8.. of its
# epilogue argument; 0 = the library's choice by shape).  A switch for A/B timing.
GEMM_CONFIG = 0

# dflash_linear_fwd epilogues.
GEMM_BIAS = 0
GEMM_BIAS_GELU = 1
GEMM_BIAS_ADD = 2
GEMM_DTYPES = (torch.float16, torch.bfloat16)


@_lib.hip_op("disentangled_flash::linear_epilogue")
def linear_epilogue(
    x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, residual: torch.Tensor | None,
    epilogue: int
) -> torch.Tensor:
    """``epilogue(x @ weight.T + bias)`` on the hand-written gfx950 GEMM.

    ``x`` is ``[..., K]`` with dense rows, ``weight`` the ``[N, K]`` nn.Linear
    weight; epilogue ``GEMM_BIAS`` (plain linear), ``GEMM_BIAS_GELU`` (exact-erf
    GELU of the dtype-rounded linear output) or ``GEMM_BIAS_ADD`` (plus
    ``residual`` ``[..., N]``, after rounding the linear output).
    """

    lib = _lib.load()
    k = x.shape[-1]
    n = weight.shape[0]
    rows = x.numel() // k if k else 0
    out = x.new_empty(x.shape[:-1] + (n,))
    if int(epilogue) == GEMM_BIAS_ADD:
        # The kernel reads rows * n elements of the residual in the output dtype.
        if residual is None:
            raise ValueError("linear_epilogue: GEMM_BIAS_ADD needs a residual")
        if residual.shape != out.shape:
            raise ValueError(f"linear_epilogue: residual shape {tuple(residual.shape)} "
                             f"!= output shape {tuple(out.shape)}")
        if residual.dtype != x.dtype or residual.device != x.device:
            raise ValueError("linear_epilogue: residual must have the input's dtype and device")
        if not residual.is_contiguous():
            raise ValueError("linear_epilogue: residual must be contiguous")
    code = lib.dflash_linear_fwd(
        x.data_ptr(), weight.data_ptr(), bias.data_ptr(),
        residual.data_ptr() if residual is not None else None, out.data_ptr(), rows, n, k,
        int(epilogue) | (int(GEMM_CONFIG) << 8), _lib.DTYPE_CODES[x.dtype],
        _lib.current_stream_handle(x.device))
    _lib.check(code, "dflash_linear_fwd")
    return out


@linear_epilogue.register_fake
def _linear_epilogue_fake(x, weight, bias, residual, epilogue):
    return x.new_empty(x.shape[:-1] + (weight.shape[0],))


def gemm_fits(weight: torch.Tensor, bias: torch.Tensor | None) -> bool:
    """True if ``F.linear(x, weight, bias)`` can run on :func:`linear_epilogue`.

    That is: a bias, fp16 or bf16 weight and bias on a GPU, N a multiple of 128
    or 192 (the tile widths) and K a multiple of 32 (the k-step) - every
    projection of DeBERTa base, large and xlarge.
    """

    if bias is None or weight.dim() != 2:
        return False
    n, k = weight.shape
    if weight.dtype not in GEMM_DTYPES or bias.dtype != weight.dtype:
        return False
    if not weight.is_contiguous() or weight.device.type != "cuda":
        return False
    return (n % 128 == 0 or n % 192 == 0) and k % 32 == 0


def linear_fits(linear: nn.Module) -> bool:
    return USE_HIP_GEMM and isinstance(linear, nn.Linear) and gemm_fits(linear.weight, linear.bias)


def gemm_rows(x: torch.Tensor) -> torch.Tensor:
    """``x`` with dense rows (last dimension contiguous, rows packed)."""

    return x if x.is_contiguous() else x.contiguous()


def fusable_intermediate(module: nn.Module) -> bool:
    """True for a Hugging Face ``DebertaV2Intermediate`` whose activation is the erf GELU.

    ``dense`` must fit :func:`gemm_fits` and ``intermediate_act_fn`` must be
    transformers' ``GELUActivation`` (``ACT2FN["gelu"]``) computing the erf form,
    or ``torch.nn.functional.gelu`` itself.
    """

    if not linear_fits(getattr(module, "dense", None)):
        return False
    act = getattr(module, "intermediate_act_fn", None)
    if act is F.gelu:
        return True
    if type(act).__name__ != "GELUActivation":
        return False
    inner = getattr(act, "act", None)
    return inner is F.gelu or getattr(inner, "__name__", "") == "_gelu_python"


def intermediate_block(module: nn.Module, hidden_states: torch.Tensor) -> torch.Tensor:
    """``module(hidden_states)`` as one GEMM with the GELU in its epilogue, or the
    module itself where :func:`hip_gemm_rows` says so."""

    if not hip_gemm_rows(hidden_states, module.dense.out_features):
        return module(hidden_states)
    return linear_epilogue(gemm_rows(hidden_states), module.dense.weight, module.dense.bias,
                           None, GEMM_BIAS_GELU)


def output_block_gemm(module: nn.Module, hidden_states: torch.Tensor,
                      input_tensor: torch.Tensor) -> torch.Tensor:
    """``module(hidden_states, input_tensor)``: GEMM with the residual added in its
    epilogue, then LayerNorm over the sum (one read of it instead of two); where
    :func:`hip_gemm_rows` says so, hipBLASLt and the fused add + LayerNorm."""

    if not hip_gemm_rows(hidden_states, module.dense.out_features):
        return output_block(module, hidden_states, input_tensor)
    summed = linear_epilogue(gemm_rows(hidden_states), module.dense.weight, module.dense.bias,
                             gemm_rows(input_tensor), GEMM_BIAS_ADD)
    norm = module.LayerNorm
    return layernorm(summed, norm.weight, norm.bias, norm.eps)


def fusable_output_block(module: nn.Module) -> bool:
    """True for a Hugging Face ``SelfOutput``/``Output`` block the fused tail can run.

    That is: a ``dense`` ``nn.Linear`` with bias, an affine ``nn.LayerNorm``
    over the last dimension and a ``dropout`` (the identity in inference), with
    parameters in one dtype the kernel supports.
    """

    dense = getattr(module, "dense", None)
    norm = getattr(module, "LayerNorm", None)
    if not isinstance(dense, nn.Linear) or dense.bias is None:
        return False
    if not isinstance(norm, nn.LayerNorm) or not norm.elementwise_affine or norm.bias is None:
        return False
    if len(norm.normalized_shape) != 1 or norm.normalized_shape[0] != dense.out_features:
        return False
    hidden = dense.out_features
    if hidden % 4 != 0 or hidden > 4096:
        return False
    dtype = dense.weight.dtype
    if dtype not in _lib.DTYPE_CODES or norm.weight.dtype != dtype or norm.bias.dtype != dtype:
        return False
    return hasattr(module, "dropout")


def output_block(module: nn.Module, hidden_states: torch.Tensor,
                 input_tensor: torch.Tensor) -> torch.Tensor:
    """``module(hidden_states, input_tensor)`` with the residual add and LayerNorm fused.

    The dense runs on hipBLASLt, or in launch-bound eager forwards at base width
    (:func:`eager_small_gemm`) on the hand-written GEMM with the residual in its
    epilogue.  The caller checks :func:`fusable_output_block` once when the
    encoder is prepared; this function is the hot path.
    """

    dense = module.dense
    residual = input_tensor if input_tensor.is_contiguous() else input_tensor.contiguous()
    norm = module.LayerNorm
    if USE_HIP_GEMM and eager_small_gemm(hidden_states, dense.out_features) \
            and gemm_fits(dense.weight, dense.bias) and hidden_states.dtype == dense.weight.dtype:
        summed = linear_epilogue(gemm_rows(hidden_states), dense.weight, dense.bias, residual,
                                 GEMM_BIAS_ADD)
        return layernorm(summed, norm.weight, norm.bias, norm.eps)
    projected = F.linear(hidden_states, dense.weight, dense.bias)
    return add_layernorm(projected, residual, norm.weight, norm.bias, norm.eps)


# ConvLayer.conv_act values the fused tail implements (DFLASH_ACT_* codes);
# "gelu" is the exact erf form of Hugging Face's ACT2FN["gelu"].
CONV_ACTIVATIONS = {"gelu": 0, "tanh": 1, "relu": 2}


@_lib.hip_op("disentangled_flash::conv_layer_tail")
def conv_layer_tail(
    taps: torch.Tensor, residual: torch.Tensor, conv_bias: torch.Tensor, weight: torch.Tensor,
    bias: torch.Tensor, mask: torch.Tensor, eps: float, act: int
) -> torch.Tensor:
    """ConvLayer output from the tap products ``taps`` ``[B*L, 3*hidden]``.

    ``residual`` is ``[B, L, hidden]``; ``mask`` the caller's ``[B, L]`` mask
    as int64 (a bool mask as 0/1).
    """

    lib = _lib.load()
    batch, length, hidden = residual.shape
    out = torch.empty_like(residual)
    code = lib.dflash_conv_layer_tail_fwd(
        taps.data_ptr(),
        _lib.DTYPE_CODES[taps.dtype],
        residual.data_ptr(),
        conv_bias.data_ptr(),
        weight.data_ptr(),
        bias.data_ptr(),
        mask.data_ptr(),
        out.data_ptr(),
        batch,
        length,
        hidden,
        float(eps),
        int(act),
        _lib.DTYPE_CODES[residual.dtype],
        _lib.current_stream_handle(residual.device),
    )
    _lib.check(code, "dflash_conv_layer_tail_fwd")
    return out


@conv_layer_tail.register_fake
def _conv_layer_tail_fake(taps, residual, conv_bias, weight, bias, mask, eps, act):
    return torch.empty_like(residual)


def fusable_conv_layer(module: nn.Module | None) -> bool:
    """True for a Hugging Face ``ConvLayer`` the fused tail can run.

    That is: ``conv`` an ``nn.Conv1d(hidden, hidden, 3, padding=1)`` with bias,
    one group, unit stride and dilation and zero padding; ``conv_act`` one of
    :data:`CONV_ACTIVATIONS`; an affine ``nn.LayerNorm`` over ``hidden``; a
    ``dropout`` (the identity in inference); one dtype the kernel supports.
    """

    if module is None:
        return False
    conv = getattr(module, "conv", None)
    norm = getattr(module, "LayerNorm", None)
    if not isinstance(conv, nn.Conv1d) or conv.bias is None:
        return False
    if (conv.kernel_size != (3,) or conv.padding != (1,) or conv.stride != (1,)
            or conv.dilation != (1,) or conv.groups != 1 or conv.padding_mode != "zeros"):
        return False
    hidden = conv.out_channels
    if conv.in_channels != hidden or hidden % 4 != 0 or hidden > 4096:
        return False
    if getattr(module, "conv_act", None) not in CONV_ACTIVATIONS:
        return False
    if not isinstance(norm, nn.LayerNorm) or not norm.elementwise_affine or norm.bias is None:
        return False
    if tuple(norm.normalized_shape) != (hidden,):
        return False
    dtype = conv.weight.dtype
    params = (conv.bias, norm.weight, norm.bias)
    if dtype not in _lib.DTYPE_CODES or any(p.dtype != dtype for p in params):
        return False
    return hasattr(module, "dropout")


def conv_taps(module: nn.Module) -> torch.Tensor:
    """Conv1d weight ``[hidden, hidden, 3]`` as ``[3*hidden, hidden]``, tap-major."""

    weight = module.conv.weight
    hidden = weight.shape[0]
    return weight.detach().permute(2, 0, 1).reshape(3 * hidden, hidden).contiguous()


def conv_layer_block(module: nn.Module, taps: torch.Tensor, hidden_states: torch.Tensor,
                     residual_states: torch.Tensor, input_mask: torch.Tensor) -> torch.Tensor:
    """``module(hidden_states, residual_states, input_mask)`` for a 2-D mask.

    The tap products are one GEMM with fp32 output for 16-bit inputs, so the
    convolution is rounded once, in the tail kernel.
    """

    batch, length, hidden = hidden_states.shape
    rows = hidden_states.reshape(batch * length, hidden)
    if hidden_states.dtype == torch.float32:
        products = torch.mm(rows, taps.t())
    else:
        products = torch.ops.aten.mm.dtype(rows, taps.t(), torch.float32)
    mask = input_mask if input_mask.dtype == torch.int64 else input_mask.to(torch.int64)
    residual = residual_states if residual_states.is_contiguous() else residual_states.contiguous()
    norm = module.LayerNorm
    return conv_layer_tail(products, residual, module.conv.bias, norm.weight, norm.bias,
                           mask.contiguous(), norm.eps, CONV_ACTIVATIONS[module.conv_act])


__all__ = [
    "CONV_ACTIVATIONS",
    "add_layernorm",
    "conv_layer_block",
    "conv_layer_tail",
    "conv_taps",
    "fusable_conv_layer",
    "fusable_output_block",
    "output_block",
]
