"""Fused encoder-layer tails for the HIP backend.

``DebertaV2SelfOutput`` and ``DebertaV2Output`` (reference ``_reference.py:101-112``
and ``474-485``) both end in ``LayerNorm(dense(x) + input_tensor)``.  The HIP
encoder keeps the dense projection on hipBLASLt (``F.linear`` with its bias
epilogue) and replaces the separate residual add and LayerNorm with one
kernel, ``disentangled_flash::add_layernorm``, which reads the projection and
the residual once and writes the normalised row.

The op has a fake implementation so that ``torch.compile(fullgraph=True)``
traces through it, like the attention ops.
"""

from __future__ import annotations

import torch
from torch import nn
from torch.nn import functional as F

from . import _lib


@torch.library.custom_op("disentangled_flash::add_layernorm", mutates_args=())
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

    The caller checks :func:`fusable_output_block` once when the encoder is
    prepared; this function is the hot path.
    """

    projected = F.linear(hidden_states, module.dense.weight, module.dense.bias)
    residual = input_tensor if input_tensor.is_contiguous() else input_tensor.contiguous()
    norm = module.LayerNorm
    return add_layernorm(projected, residual, norm.weight, norm.bias, norm.eps)


__all__ = ["add_layernorm", "fusable_output_block", "output_block"]
