"""ctypes binding of ``libdflash.so`` (the C ABI declared in ``include/dflash.h``).

The library is a plain HIP shared object built for gfx950 next to this file.
It is loaded after ``torch`` so that it binds to the HIP runtime torch already
loaded (both resolve ``libamdhip64.so.7``), which keeps torch's streams and
device pointers valid inside the library.

There is no fallback: if the library is missing or cannot be loaded, every
HIP-backend call raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import functools
import os
from pathlib import Path

import torch  # noqa: F401  (load torch's HIP runtime first)

LIBRARY_NAME = "libdflash.so"
ABI_VERSION = 7

DTYPE_CODES = {
    torch.float16: 0,
    torch.bfloat16: 1,
    torch.float32: 2,
}

_c_void_p = ctypes.c_void_p
_c_int = ctypes.c_int
_c_int64 = ctypes.c_int64
_c_float = ctypes.c_float

_handle: ctypes.CDLL | None = None
_load_error: str | None = None


def library_path() -> Path:
    override = os.environ.get("DFLASH_LIBRARY")
    return Path(override) if override else Path(__file__).with_name(LIBRARY_NAME)


def _bind(lib: ctypes.CDLL) -> None:
    lib.dflash_attention_fwd.restype = _c_int
    lib.dflash_attention_fwd.argtypes = [
        _c_void_p, _c_void_p, _c_void_p,            # query, key, value
        _c_void_p, _c_void_p,                        # c2p, p2c
        _c_void_p, _c_void_p, _c_void_p,             # delta_to_local, mask, out
        _c_int, _c_int, _c_int, _c_int, _c_int,      # B, H, L, D, S
        _c_float, _c_int, _c_int, _c_int, _c_int,    # scale, has_c2p, has_p2c, dtype, strict
        _c_void_p,                                   # stream
    ]
    lib.dflash_attention_rel_fwd.restype = _c_int
    lib.dflash_attention_rel_fwd.argtypes = [
        _c_void_p, _c_void_p, _c_void_p,             # query, key, value
        _c_int64, _c_int64, _c_int64,                # stride_b, stride_h, stride_l
        _c_void_p, _c_void_p,                        # pos_key, pos_query
        _c_void_p, _c_void_p, _c_void_p,             # delta_to_local, mask, out
        _c_int, _c_int, _c_int, _c_int, _c_int,      # B, H, L, D, S
        _c_float, _c_int, _c_int, _c_int, _c_int,    # scale, has_c2p, has_p2c, dtype, strict
        _c_void_p,                                   # stream
    ]
    lib.dflash_attention_rel_split_plan.restype = _c_int
    lib.dflash_attention_rel_split_plan.argtypes = [
        _c_int, _c_int, _c_int, _c_int,                           # B, H, L, D
        ctypes.POINTER(_c_int), ctypes.POINTER(ctypes.c_size_t),  # splits, workspace_bytes
    ]
    lib.dflash_attention_rel_fwd_split.restype = _c_int
    lib.dflash_attention_rel_fwd_split.argtypes = [
        *lib.dflash_attention_rel_fwd.argtypes[:-1],              # as dflash_attention_rel_fwd
        _c_int, _c_void_p, ctypes.c_size_t,                       # splits, workspace, bytes
        _c_void_p,                                                # stream
    ]
    lib.dflash_attention_rel_fwd_noalloc.restype = _c_int
    lib.dflash_attention_rel_fwd_noalloc.argtypes = [
        *lib.dflash_attention_rel_fwd.argtypes[:-1],              # as dflash_attention_rel_fwd
        _c_int,                                                   # splits (0 = plan)
        _c_void_p,                                                # stream
    ]
    lib.dflash_attention_rel_noalloc_scratch_bytes.restype = ctypes.c_size_t
    lib.dflash_attention_rel_noalloc_scratch_bytes.argtypes = []
    lib.dflash_add_layernorm_fwd.restype = _c_int
    lib.dflash_add_layernorm_fwd.argtypes = [
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # x, residual, gamma, beta, out
        _c_int, _c_int, _c_float, _c_int,                        # rows, hidden, eps, dtype
        _c_void_p,                                               # stream
    ]
    lib.dflash_conv_layer_tail_fwd.restype = _c_int
    lib.dflash_conv_layer_tail_fwd.argtypes = [
        _c_void_p, _c_int,                                       # z, z_dtype
        _c_void_p, _c_void_p, _c_void_p, _c_void_p,              # residual, bias, gamma, beta
        _c_void_p, _c_void_p,                                    # mask, out
        _c_int, _c_int, _c_int, _c_float, _c_int, _c_int,        # B, L, hidden, eps, act, dtype
        _c_void_p,                                               # stream
    ]
    lib.dflash_linear_fwd.restype = _c_int
    lib.dflash_linear_fwd.argtypes = [
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # x, weight, bias, residual, y
        _c_int, _c_int, _c_int, _c_int, _c_int,                  # M, N, K, epilogue, dtype
        _c_void_p,                                               # stream
    ]
    lib.dflash_error_string.restype = ctypes.c_char_p
    lib.dflash_error_string.argtypes = [_c_int]
    lib.dflash_abi_version.restype = _c_int
    lib.dflash_abi_version.argtypes = []


def load() -> ctypes.CDLL:
    """Load and bind the library once; raise ``RuntimeError`` if it is unusable."""

    global _handle, _load_error
    if _handle is not None:
        return _handle
    path = library_path()
    if not path.exists():
        _load_error = (
            f"{path} is missing: build the HIP library first "
            "(python __graft_entry__.py, or python disentangled-flash_amd/csrc/build.py)"
        )
        raise RuntimeError(_load_error)
    try:
        lib = ctypes.CDLL(str(path))
        _bind(lib)
    except (OSError, AttributeError) as error:
        _load_error = f"cannot load {path}: {error}"
        raise RuntimeError(_load_error) from error
    version = lib.dflash_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{path} has ABI version {version}, expected {ABI_VERSION}")
    _handle = lib
    return lib


def is_available() -> bool:
    try:
        load()
    except RuntimeError:
        return False
    return True


def check(code: int, what: str) -> None:
    if code != 0:
        message = load().dflash_error_string(code).decode()
        raise RuntimeError(f"{what} failed with code {code}: {message}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)

_PLAIN_TENSORS = (torch.Tensor, torch.nn.Parameter)

try:
    from torch.utils._python_dispatch import _get_current_dispatch_mode as _get_dispatch_mode
except ImportError:  # pragma: no cover - older torch
    def _get_dispatch_mode():
        return None


def current_stream_handle(device: torch.device) -> int:
    """The HIP stream torch launches on for ``device`` (raw handle)."""

    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def hip_op(name: str):
    """``torch.library.custom_op(name)`` whose eager calls skip the dispatcher.

    Under ``torch.compile`` tracing the function is the custom op (with the fake
    implementation registered on it), so compiled graphs keep the HIP op as one
    node.  Called eagerly - and during HIP-graph capture - it runs the
    implementation directly: the op dispatch adds about 3 us of host time per
    call, which an eager encoder forward of a few thousand tokens (bound by launch
    time) pays on every layer.
    """

    def wrap(impl):
        op = torch.library.custom_op(name, mutates_args=())(impl)

        @functools.wraps(impl)
        def call(*args, **kwargs):
            # Through the custom op when tracing (torch.compile, export,
            # make_fx), under any dispatch mode (FakeTensorMode, opcheck) or
            # with a tensor that is not a plain CUDA tensor, so that the
            # registered fake runs instead of a data_ptr() of a fake tensor.
            if torch.compiler.is_compiling() or _get_dispatch_mode() is not None:
                return op(*args, **kwargs)
            for a in args:
                if isinstance(a, torch.Tensor) and (
                        type(a) not in _PLAIN_TENSORS or a.device.type != "cuda"):
                    return op(*args, **kwargs)
            return impl(*args, **kwargs)

        call.register_fake = op.register_fake
        call.custom_op = op
        return call

    return wrap


__all__ = ["DTYPE_CODES", "check", "current_stream_handle", "hip_op", "is_available",
           "library_path", "load"]
