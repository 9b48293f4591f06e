"""HIP (gfx950) fused DeBERTa attention: op boundary and attention module.

Two custom ops wrap the C ABI of ``libdflash.so``:

* ``disentangled_flash::deberta_attention`` - same arguments and semantics as the
  reference's ``gliner2_attention::deberta_attention`` (``kernel.py:368-438``):
  head-major Q/K/V plus precomputed ``[B, H, L, S]`` c2p/p2c tables.
* ``disentangled_flash::deberta_attention_rel`` - the MI355X design: the kernel
  reads Q/K/V straight out of the fused QKV projection output ``[B, L, 3*H*d]``
  and computes the relative scores from the ``[H, S, d]`` projected position
  rows inside each tile, so neither the head reshape copies nor the two
  ``[B, H, L, S]`` tables exist.

Both ops register a fake (meta) implementation, so ``torch.compile(fullgraph=True)``
traces through them the way the reference relies on ``triton_op``.

``HipInferenceDisentangledSelfAttention`` mirrors ``TritonInferenceDisentangledSelfAttention``
(``kernel.py:471-638``): same plan type, validation and error messages.
"""

from __future__ import annotations

import ctypes
from typing import Any, NamedTuple

import torch

from . import _lib
from ._torch import TorchInferenceDisentangledSelfAttention
from . import layers
from .layers import GEMM_BIAS, gemm_fits, gemm_rows, linear_epilogue
from .modeling import DebertaAttentionConfig
from .position import SharedPositionPlanCache

LOG2E = 1.4426950408889634
SUPPORTED_HEAD_DIMS = (32, 64, 128)
SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
RELATIVE_MODES = ("fused", "table")


@_lib.hip_op("disentangled_flash::deberta_attention")
def deberta_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    c2p: torch.Tensor,
    p2c: torch.Tensor,
    delta_to_local: torch.Tensor,
    attention_mask: torch.Tensor,
    num_heads: int,
    sequence_length: int,
    active_slots: int,
    score_scale_log2: float,
    has_c2p: bool,
    has_p2c: bool,
    is_bf16: bool,
    is_fp32: bool,
    strict_fp32: bool,
) -> torch.Tensor:
    """Fused attention over precomputed c2p/p2c tables (reference op contract).

    ``query/key/value`` are ``[B, H, L, d]`` contiguous, ``c2p/p2c`` are
    ``[B, H, L, S]`` contiguous (ignored when their mode is off) and the
    output is ``[B, L, H*d]`` in the input dtype.
    """

    _check_table_inputs(query, key, value, c2p, p2c, delta_to_local, attention_mask, num_heads,
                        sequence_length, active_slots, has_c2p, has_p2c)
    lib = _lib.load()
    batch, _, length, head_dim = query.shape
    out = torch.empty(
        (batch, sequence_length, num_heads * head_dim), device=query.device, dtype=query.dtype
    )
    code = lib.dflash_attention_fwd(
        query.data_ptr(),
        key.data_ptr(),
        value.data_ptr(),
        c2p.data_ptr() if has_c2p else None,
        p2c.data_ptr() if has_p2c else None,
        delta_to_local.data_ptr(),
        attention_mask.data_ptr(),
        out.data_ptr(),
        batch,
        num_heads,
        sequence_length,
        head_dim,
        active_slots,
        score_scale_log2,
        int(has_c2p),
        int(has_p2c),
        _lib.DTYPE_CODES[query.dtype],
        int(strict_fp32),
        _lib.current_stream_handle(query.device),
    )
    _lib.check(code, "dflash_attention_fwd")
    return out


@deberta_attention.register_fake
def _deberta_attention_fake(query, key, value, c2p, p2c, delta_to_local, attention_mask,
                            num_heads, sequence_length, active_slots, score_scale_log2,
                            has_c2p, has_p2c, is_bf16, is_fp32, strict_fp32):
    batch, _, _, head_dim = query.shape
    return query.new_empty((batch, sequence_length, num_heads * head_dim))


@_lib.hip_op("disentangled_flash::deberta_attention_rel")
def deberta_attention_rel(
    qkv: torch.Tensor,
    pos_key: torch.Tensor,
    pos_query: torch.Tensor,
    delta_to_local: torch.Tensor,
    attention_mask: torch.Tensor,
    num_heads: int,
    head_dim: int,
    score_scale_log2: float,
    has_c2p: bool,
    has_p2c: bool,
    strict_fp32: bool,
    key_splits: int = 0,
) -> torch.Tensor:
    """Fused attention with in-kernel relative scores.

    ``qkv`` is the fused projection output ``[B, L, 3*H*d]`` (Q, K, V column
    blocks); ``pos_key/pos_query`` are ``[H, S, d]``.  When a mode is off its
    position tensor is never read.  Output ``[B, L, H*d]``.

    ``key_splits``: 0 lets the library split the key range of every query block
    over several workgroups when the unsplit grid would leave the GPU underfilled
    (``dflash_attention_rel_split_plan``); 1 never splits; n > 1 forces n splits.
    """

    if key_splits < 0:
        raise ValueError(f"key_splits must be >= 0, got {key_splits}")
    _check_rel_inputs(qkv, pos_key, pos_query, delta_to_local, attention_mask, num_heads,
                      head_dim, has_c2p, has_p2c)
    lib = _lib.load()
    batch, length, width = qkv.shape
    hd = num_heads * head_dim
    out = torch.empty((batch, length, hd), device=qkv.device, dtype=qkv.dtype)
    stride_b, stride_l = qkv.stride(0), qkv.stride(1)
    base = qkv.data_ptr()
    esize = qkv.element_size()
    active = pos_key.size(1) if has_c2p else (pos_query.size(1) if has_p2c else 0)
    splits, workspace_bytes = _split_plan(lib, qkv.device, qkv.dtype, batch, num_heads, length,
                                          head_dim, key_splits)
    workspace = None
    if workspace_bytes:
        workspace = torch.empty(workspace_bytes // 4, device=qkv.device, dtype=torch.float32)
    code = lib.dflash_attention_rel_fwd_split(
        base,
        base + hd * esize,
        base + 2 * hd * esize,
        stride_b,
        head_dim,
        stride_l,
        pos_key.data_ptr() if has_c2p else None,
        pos_query.data_ptr() if has_p2c else None,
        delta_to_local.data_ptr(),
        attention_mask.data_ptr(),
        out.data_ptr(),
        batch,
        num_heads,
        length,
        head_dim,
        active,
        score_scale_log2,
        int(has_c2p),
        int(has_p2c),
        _lib.DTYPE_CODES[qkv.dtype],
        int(strict_fp32),
        splits,
        workspace.data_ptr() if workspace is not None else None,
        workspace_bytes,
        _lib.current_stream_handle(qkv.device),
    )
    _lib.check(code, "dflash_attention_rel_fwd_split")
    return out


_SPLIT_PLANS: dict[tuple, tuple[int, int]] = {}


def _check_table_inputs(query, key, value, c2p, p2c, delta_to_local, attention_mask, num_heads,
                        sequence_length, active_slots, has_c2p, has_p2c) -> None:
    """Host checks of ``deberta_attention``'s tensors before anything is launched.

    The kernel addresses Q/K/V as ``[B, H, L, d]`` and each table as
    ``[B, H, L, S]`` from the integers given here, so a tensor of another shape,
    layout or dtype would be read out of bounds or as garbage.
    """

    if query.dim() != 4:
        raise ValueError(f"query must be [B, H, L, d], got shape {tuple(query.shape)}")
    batch, heads, length, head_dim = query.shape
    if heads != num_heads or length != sequence_length:
        raise ValueError(f"query shape {tuple(query.shape)} does not match num_heads={num_heads}, "
                         f"sequence_length={sequence_length}")
    if query.dtype not in SUPPORTED_DTYPES:
        raise TypeError(f"query dtype {query.dtype} is not fp16, bf16 or fp32")
    device = query.device
    for name, t in (("query", query), ("key", key), ("value", value)):
        if t.shape != query.shape or t.dtype != query.dtype or t.device != device:
            raise ValueError(f"{name} must match query: [B, H, L, d] {tuple(query.shape)}, "
                             f"{query.dtype}, {device}")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    for name, table, used in (("c2p", c2p, has_c2p), ("p2c", p2c, has_p2c)):
        if not used:
            continue
        if table.shape != (batch, heads, length, active_slots):
            raise ValueError(f"{name} must be [B, H, L, S] = {(batch, heads, length, active_slots)}, "
                             f"got {tuple(table.shape)}")
        if table.dtype != query.dtype or table.device != device or not table.is_contiguous():
            raise ValueError(f"{name} must be a contiguous {query.dtype} tensor on {device}")
    if delta_to_local.dtype != torch.int32 or delta_to_local.dim() != 1:
        raise TypeError("delta_to_local must be a 1-D int32 tensor")
    if length > 0 and delta_to_local.numel() != 2 * length - 1:
        raise ValueError(f"delta_to_local has {delta_to_local.numel()} entries, expected "
                         f"2L-1 = {2 * length - 1}")
    if not delta_to_local.is_contiguous() or delta_to_local.device != device:
        raise ValueError("delta_to_local must be contiguous and on the query device")
    if attention_mask.shape != (batch, length):
        raise ValueError(f"attention_mask shape {tuple(attention_mask.shape)} does not match "
                         f"[{batch}, {length}]")
    if attention_mask.element_size() != 1 or not attention_mask.is_contiguous() or (
            attention_mask.device != device):
        raise ValueError("attention_mask must be a contiguous bool/uint8 tensor on the query device")


def _check_rel_inputs(qkv, pos_key, pos_query, delta_to_local, attention_mask, num_heads,
                      head_dim, has_c2p, has_p2c) -> None:
    """Host checks of ``deberta_attention_rel``'s tensors before anything is launched.

    The kernel bounds every row read by the shapes given here, so a tensor
    that is narrower, strided differently or of another dtype than they say
    would be read out of bounds or as garbage.
    """

    if qkv.dim() != 3:
        raise ValueError(f"qkv must be [B, L, 3*H*d], got shape {tuple(qkv.shape)}")
    batch, length, width = qkv.shape
    if width != 3 * num_heads * head_dim:
        raise ValueError(f"qkv width {width} != 3 * num_heads * head_dim = "
                         f"{3 * num_heads * head_dim}")
    if qkv.stride(-1) != 1 or (length > 1 and qkv.stride(1) < width) or (
            batch > 1 and qkv.stride(0) < length * qkv.stride(1)):
        raise ValueError(f"qkv rows must be dense in the last dimension, strides {qkv.stride()}")
    if qkv.dtype not in SUPPORTED_DTYPES:
        raise TypeError(f"qkv dtype {qkv.dtype} is not fp16, bf16 or fp32")
    device = qkv.device
    for name, table, used in (("pos_key", pos_key, has_c2p), ("pos_query", pos_query, has_p2c)):
        if not used:
            continue
        if table.dtype != qkv.dtype:
            raise TypeError(f"{name} dtype {table.dtype} does not match qkv dtype {qkv.dtype}")
        if table.dim() != 3 or table.size(0) != num_heads or table.size(2) != head_dim:
            raise ValueError(f"{name} must be [H={num_heads}, S, d={head_dim}], got "
                             f"{tuple(table.shape)}")
        if not table.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
        if table.device != device:
            raise ValueError(f"{name} is on {table.device}, qkv on {device}")
    if has_c2p and has_p2c and pos_key.size(1) != pos_query.size(1):
        raise ValueError("pos_key and pos_query must have the same number of active slots")
    if delta_to_local.dtype != torch.int32 or delta_to_local.dim() != 1:
        raise TypeError("delta_to_local must be a 1-D int32 tensor")
    if length > 0 and delta_to_local.numel() != 2 * length - 1:
        raise ValueError(f"delta_to_local has {delta_to_local.numel()} entries, expected "
                         f"2L-1 = {2 * length - 1}")
    if not delta_to_local.is_contiguous() or delta_to_local.device != device:
        raise ValueError("delta_to_local must be contiguous and on the qkv device")
    if attention_mask.shape != (batch, length):
        raise ValueError(f"attention_mask shape {tuple(attention_mask.shape)} does not match "
                         f"[{batch}, {length}]")
    if attention_mask.element_size() != 1 or not attention_mask.is_contiguous() or (
            attention_mask.device != device):
        raise ValueError("attention_mask must be a contiguous bool/uint8 tensor on the qkv device")


def _split_plan(lib, device: torch.device, dtype: torch.dtype, batch: int, heads: int,
                length: int, head_dim: int, key_splits: int) -> tuple[int, int]:
    """(splits, workspace bytes) for one launch; cached per device and shape.

    The fp32 kernel has no split form, so fp32 never gets a workspace.
    """

    if batch == 0 or key_splits == 1 or dtype == torch.float32:
        return 1, 0
    key = (device.index, batch, heads, length, head_dim, key_splits)
    plan = _SPLIT_PLANS.get(key)
    if plan is None:
        splits = ctypes.c_int(key_splits)
        size = ctypes.c_size_t(0)
        with torch.cuda.device(device):
            _lib.check(lib.dflash_attention_rel_split_plan(batch, heads, length, head_dim,
                                                           ctypes.byref(splits),
                                                           ctypes.byref(size)),
                       "dflash_attention_rel_split_plan")
        plan = (splits.value, size.value)
        _SPLIT_PLANS[key] = plan
    return plan


@deberta_attention_rel.register_fake
def _deberta_attention_rel_fake(qkv, pos_key, pos_query, delta_to_local, attention_mask,
                                num_heads, head_dim, score_scale_log2, has_c2p, has_p2c,
                                strict_fp32, key_splits=0):
    batch, length, _ = qkv.shape
    return qkv.new_empty((batch, length, num_heads * head_dim))


def _require_2d_padding_mask(
    attention_mask: torch.Tensor, batch_size: int, sequence_length: int
) -> torch.Tensor:
    """Validate the factorized ``[B, L]`` padding mask (``kernel.py:441-458``)."""

    if attention_mask.dim() != 2:
        raise ValueError(
            "the HIP fast path requires a factorized padding mask with shape "
            "[B, L]; arbitrary pairwise masks are not supported"
        )
    if attention_mask.shape != (batch_size, sequence_length):
        raise ValueError(
            f"attention_mask shape {tuple(attention_mask.shape)} does not match "
            f"[{batch_size}, {sequence_length}]"
        )
    return attention_mask.bool().contiguous()


class HipPreparedPositionPlan(NamedTuple):
    """Layer projections plus one shared compact position LUT (``kernel.py:461-468``)."""

    sequence_length: int
    active_slots: torch.Tensor
    delta_to_local: torch.Tensor
    pos_key: torch.Tensor | None
    pos_query: torch.Tensor | None


class HipInferenceDisentangledSelfAttention(TorchInferenceDisentangledSelfAttention):
    """Forward-only MI355X DeBERTa-v2/v3 self-attention.

    Head dimensions 32, 64 and 128; fp16, bf16 and fp32.  ``fp32_precision``
    follows the reference (``kernel.py:485-493``): ``"strict"`` gives fp32-accurate
    products (IEEE fp32 MFMA at d = 128 with the c2p term; otherwise six bf16
    MFMAs over a three-way bf16 split of each operand, which keeps all 24
    significand bits);
    ``"fast"`` is TF32 there, and gfx950 has no TF32 matrix path, so the fused
    kernel splits each fp32 operand into bf16 hi + lo and runs every product as
    three bf16 MFMAs (relative error about 2^-16 per product, below TF32's
    2^-11).  ``relative_mode="table"`` follows the same two modes for QK and PV.

    ``relative_mode="fused"`` (default) computes the c2p/p2c scores inside the
    attention kernel; ``"table"`` reproduces the reference's data flow (two
    separate score GEMMs, then the fused kernel reading ``[B, H, L, S]`` tables).
    """

    def __init__(
        self,
        config: DebertaAttentionConfig | Any,
        *,
        position_plan_cache: SharedPositionPlanCache | None = None,
        fp32_precision: str = "strict",
        relative_mode: str = "fused",
    ) -> None:
        super().__init__(config, position_plan_cache=position_plan_cache)
        if fp32_precision not in {"strict", "fast"}:
            raise ValueError("fp32_precision must be 'strict' or 'fast'")
        if relative_mode not in RELATIVE_MODES:
            raise ValueError(f"relative_mode must be one of {RELATIVE_MODES}")
        self.fp32_precision = fp32_precision
        self.relative_mode = relative_mode

    @torch.no_grad()
    def prepare_shape(
        self, sequence_length: int, device: torch.device | str | None = None
    ) -> HipPreparedPositionPlan:
        """Prepare the ``O(L)`` plan: LUT plus the active rows of the projected tables."""

        def build(length: int, resolved: torch.device) -> HipPreparedPositionPlan:
            if resolved.type != "cuda":
                raise ValueError("HIP shape plans must be prepared on a GPU device")
            indices = self.position_plan_cache.compact(length, resolved)
            pos_key, pos_query = self._project_active_positions(indices.active_slots)
            lut = indices.delta_to_local.to(dtype=torch.int32).contiguous()
            return HipPreparedPositionPlan(length, indices.active_slots, lut, pos_key, pos_query)

        return self._cached_plan(sequence_length, device, build)

    def _fused_projection(self, hidden_states: torch.Tensor) -> torch.Tensor:
        """Fused QKV projection ``[B, L, 3*H*d]`` (``_torch.py:284-297``).

        fp16/bf16 projections of a supported width run on the hand-written gfx950
        GEMM (``dflash_linear_fwd``) where ``layers.hip_gemm_rows`` says so (by
        row count and launch mode); others on ``F.linear``.
        """

        prep = self._prepared
        if prep is None:
            raise RuntimeError(
                "fused QKV projection is not prepared; call prepare_for_inference() first"
            )
        if layers.USE_HIP_GEMM and hidden_states.device.type == "cuda" \
                and layers.hip_gemm_rows(hidden_states, prep.qkv_weight.shape[0]) \
                and gemm_fits(prep.qkv_weight, prep.qkv_bias) \
                and hidden_states.dtype == prep.qkv_weight.dtype:
            return linear_epilogue(gemm_rows(hidden_states), prep.qkv_weight, prep.qkv_bias, None,
                                   GEMM_BIAS)
        return super()._fused_projection(hidden_states)

    def _validate_hip_call(self, hidden_states: torch.Tensor) -> None:
        if hidden_states.device.type != "cuda":
            raise RuntimeError("HipInferenceDisentangledSelfAttention requires a GPU tensor")
        if hidden_states.dtype not in SUPPORTED_DTYPES:
            raise TypeError("the HIP path supports FP16, BF16, and FP32")
        if self.attention_head_size not in SUPPORTED_HEAD_DIMS:
            raise ValueError("the HIP path supports attention head dimensions 32, 64, and 128")
        self._validate_inference_call()
        _lib.load()

    def score_scale_log2(self) -> float:
        return LOG2E / self._scale(self.scale_factor)

    def forward_prepared(
        self,
        hidden_states: torch.Tensor,
        attention_mask: torch.Tensor,
        plan: HipPreparedPositionPlan,
    ) -> tuple[torch.Tensor, None]:
        """Fused forward using a plan prepared outside the hot path (``kernel.py:545-608``)."""

        self._validate_hip_call(hidden_states)
        batch, length = hidden_states.shape[:2]
        if length != plan.sequence_length:
            raise ValueError(
                f"prepared length {plan.sequence_length} does not match input length {length}"
            )
        mask = _require_2d_padding_mask(attention_mask, batch, length)
        has_c2p, has_p2c = self.has_c2p, self.has_p2c
        if has_c2p and plan.pos_key is None:
            raise ValueError("prepared HIP plan has no content-to-position keys")
        if has_p2c and plan.pos_query is None:
            raise ValueError("prepared HIP plan has no position-to-content queries")
        scale_log2 = self.score_scale_log2()
        strict = self.fp32_precision == "strict"
        fused = self._fused_projection(hidden_states)
        if fused.stride(-1) != 1 or fused.stride(1) != fused.size(-1):
            fused = fused.contiguous()
        if self.relative_mode == "fused":
            placeholder = plan.delta_to_local
            output = deberta_attention_rel(
                fused,
                plan.pos_key if has_c2p else placeholder,
                plan.pos_query if has_p2c else placeholder,
                plan.delta_to_local,
                mask,
                self.num_attention_heads,
                self.attention_head_size,
                scale_log2,
                has_c2p,
                has_p2c,
                strict,
            )
            return output, None

        query, key, value = fused.split(self.all_head_size, dim=-1)
        q = self._reshape_heads(query, batch, length)
        k = self._reshape_heads(key, batch, length)
        v = self._reshape_heads(value, batch, length)
        c2p = torch.matmul(q, plan.pos_key.transpose(-1, -2)) if has_c2p else q
        p2c = torch.matmul(k, plan.pos_query.transpose(-1, -2)) if has_p2c else k
        output = deberta_attention(
            q,
            k,
            v,
            c2p,
            p2c,
            plan.delta_to_local,
            mask,
            self.num_attention_heads,
            length,
            plan.active_slots.numel(),
            scale_log2,
            has_c2p,
            has_p2c,
            hidden_states.dtype == torch.bfloat16,
            hidden_states.dtype == torch.float32,
            strict,
        )
        return output, None

    def forward(
        self,
        hidden_states: torch.Tensor,
        attention_mask: torch.Tensor,
        output_attentions: bool = False,
        query_states: torch.Tensor | None = None,
        relative_pos: torch.Tensor | None = None,
        rel_embeddings: torch.Tensor | None = None,
    ) -> tuple[torch.Tensor, None]:
        """HF-signature wrapper with lazy preparation (``kernel.py:610-638``)."""

        self._validate_hip_call(hidden_states)
        if output_attentions:
            raise ValueError("output_attentions=True is not supported by the HIP path")
        if query_states is not None:
            raise ValueError("the HIP path supports self-attention only")
        if relative_pos is not None:
            raise ValueError("custom relative_pos tensors are not supported by the HIP path")
        self._ensure_prepared(rel_embeddings)
        plan = self.prepare_shape(hidden_states.size(1), hidden_states.device)
        return self.forward_prepared(hidden_states, attention_mask, plan)


DisentangledFlashAttention = HipInferenceDisentangledSelfAttention


def attention_flops(batch: int, heads: int, length: int, head_dim: int) -> int:
    """Headline FLOPs of QK^T + PV over the dense length (FlashAttention convention)."""

    return 4 * batch * heads * length * length * head_dim


def relative_flops(batch: int, heads: int, length: int, head_dim: int, slots: int,
                   modes: int = 2) -> int:
    """FLOPs of the c2p/p2c score products over the active slots."""

    return 2 * modes * batch * heads * length * slots * head_dim


__all__ = [
    "DisentangledFlashAttention",
    "HipInferenceDisentangledSelfAttention",
    "HipPreparedPositionPlan",
    "attention_flops",
    "deberta_attention",
    "deberta_attention_rel",
    "relative_flops",
]
