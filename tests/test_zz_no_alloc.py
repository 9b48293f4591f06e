"""The allocation-free entry point against the workspace entry point, through the C ABI.

``dflash_attention_rel_fwd_noalloc`` runs the same kernels as
``dflash_attention_rel_fwd_split`` but keeps the partial rows of the split-key
form in the library's static per-GPU scratch instead of a caller workspace.
Its outputs must be bit-identical to the workspace entry point's with the
same split count, on consecutive calls (the second smaller, so stale scratch
contents from the first would show), and oversized requests must be refused
before anything is launched.
"""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

pytestmark = pytest.mark.gpu

LOG2E = 1.4426950408889634


def _inputs(batch, heads, length, dim, dtype, seed, lengths=None):
    from disentangled_flash.position import compact_position_plan

    active, lut = compact_position_plan(length, position_buckets=256, max_relative_positions=512,
                                        position_embedding_size=256)
    gen = torch.Generator().manual_seed(seed)
    qkv = torch.randn(batch, length, 3 * heads * dim, generator=gen) / math.sqrt(dim)
    pk, pq = (torch.randn(heads, active.numel(), dim, generator=gen) / math.sqrt(dim)
              for _ in range(2))
    if lengths is None:
        lengths = torch.randint(1, length + 1, (batch,), generator=gen)
    mask = torch.arange(length)[None] < torch.as_tensor(lengths)[:, None]
    dev = "cuda"
    return {"qkv": qkv.to(dev, dtype), "pk": pk.to(dev, dtype), "pq": pq.to(dev, dtype),
            "lut": lut.to(dev).int().contiguous(), "mask": mask.to(dev).contiguous(),
            "B": batch, "H": heads, "L": length, "D": dim, "S": active.numel(), "dtype": dtype}


def _common_args(inp, out):
    from disentangled_flash import _lib

    qkv = inp["qkv"]
    hd = inp["H"] * inp["D"]
    es = qkv.element_size()
    base = qkv.data_ptr()
    return (base, base + hd * es, base + 2 * hd * es, qkv.stride(0), inp["D"], qkv.stride(1),
            inp["pk"].data_ptr(), inp["pq"].data_ptr(), inp["lut"].data_ptr(),
            inp["mask"].data_ptr(), out.data_ptr(), inp["B"], inp["H"], inp["L"], inp["D"],
            inp["S"], LOG2E / math.sqrt(3 * inp["D"]), 1, 1, _lib.DTYPE_CODES[inp["dtype"]], 1)


def _with_workspace(lib, inp, splits):
    from disentangled_flash import _lib

    count = ctypes.c_int(splits)
    size = ctypes.c_size_t(0)
    _lib.check(lib.dflash_attention_rel_split_plan(inp["B"], inp["H"], inp["L"], inp["D"],
                                                   ctypes.byref(count), ctypes.byref(size)),
               "split_plan")
    out = torch.empty(inp["B"], inp["L"], inp["H"] * inp["D"], device="cuda", dtype=inp["dtype"])
    ws = torch.empty(max(1, size.value // 4), device="cuda", dtype=torch.float32)
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.dflash_attention_rel_fwd_split(*_common_args(inp, out), count.value,
                                                  ws.data_ptr(), size.value, stream),
               "rel_fwd_split")
    return out, count.value


def _no_alloc(lib, inp, splits):
    from disentangled_flash import _lib

    out = torch.empty(inp["B"], inp["L"], inp["H"] * inp["D"], device="cuda", dtype=inp["dtype"])
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.dflash_attention_rel_fwd_noalloc(*_common_args(inp, out), splits, stream),
               "rel_fwd_noalloc")
    return out


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_no_alloc_matches_workspace_entry_point(dtype):
    from disentangled_flash import _lib

    lib = _lib.load()
    assert lib.dflash_attention_rel_noalloc_scratch_bytes() == 16 << 20
    # First call: B=1, L=512, H=12, d=64 (the plan splits it); second, smaller:
    # B=1, L=256, H=4, d=32 with ragged masks, then a forced count of 3.
    cases = [(_inputs(1, 12, 512, 64, dtype, 1, lengths=[512]), 0),
             (_inputs(2, 4, 256, 32, dtype, 2, lengths=[200, 1]), 0),
             (_inputs(1, 2, 130, 64, dtype, 3, lengths=[77]), 3)]
    for inp, splits in cases:
        want, count = _with_workspace(lib, inp, splits)
        got = _no_alloc(lib, inp, splits)
        torch.cuda.synchronize()
        print(f"B={inp['B']} H={inp['H']} L={inp['L']} d={inp['D']} splits {splits} -> {count}",
              flush=True)
        if splits == 0 and inp["L"] == 512:
            assert count > 1, "the first case must exercise the split form"
        assert torch.equal(got, want)


def test_no_alloc_without_split_and_refusal():
    from disentangled_flash import _lib

    lib = _lib.load()
    # A full grid does not split: no scratch involved, same kernel as the plain entry point.
    inp = _inputs(16, 12, 256, 64, torch.float16, 4)
    want, count = _with_workspace(lib, inp, 0)
    assert count == 1
    got = _no_alloc(lib, inp, 0)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    # Forcing 8 splits at B=16, L=512, H=12 needs 8*16*512*12*66*4 bytes > 16 MiB: refused.
    big = _inputs(16, 12, 512, 64, torch.float16, 5)
    out = torch.full((16, 512, 768), 7.0, device="cuda", dtype=torch.float16)
    stream = torch.cuda.current_stream().cuda_stream
    code = lib.dflash_attention_rel_fwd_noalloc(*_common_args(big, out), 8, stream)
    assert code == -8
    assert b"scratch" in lib.dflash_error_string(code)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all()), "a refused call must launch nothing"


def test_no_alloc_refuses_overlap_from_another_stream():
    """A split call from a second stream while the first stream's call is pending
    returns DFLASH_ERR_BUSY and launches nothing; once it has completed, or on the
    same stream, calls pass and match the workspace entry point."""
    from disentangled_flash import _lib

    lib = _lib.load()
    inp = _inputs(1, 12, 512, 64, torch.float16, 6, lengths=[512])
    want, count = _with_workspace(lib, inp, 0)
    assert count > 1, "the case must exercise the split form (scratch in use)"
    first = torch.empty_like(want)
    blocked = torch.full_like(want, 7.0)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s1):
        # Keep s1 busy (a bounded spin kernel) so that its split call is still
        # pending when s2 asks for the scratch.
        torch.cuda._sleep(50_000_000)
        assert lib.dflash_attention_rel_fwd_noalloc(*_common_args(inp, first), 0,
                                                    s1.cuda_stream) == 0
        # Same stream: ordered, so it passes.
        again = torch.empty_like(want)
        assert lib.dflash_attention_rel_fwd_noalloc(*_common_args(inp, again), 0,
                                                    s1.cuda_stream) == 0
    code = lib.dflash_attention_rel_fwd_noalloc(*_common_args(inp, blocked), 0, s2.cuda_stream)
    print(f"second stream while the first is pending: code {code}", flush=True)
    assert code == -9
    assert b"another stream" in lib.dflash_error_string(code)
    s1.synchronize()
    torch.cuda.synchronize()
    assert bool((blocked == 7.0).all()), "a refused call must launch nothing"
    assert torch.equal(first, want) and torch.equal(again, want)
    # After s1 has completed, s2 may use the scratch.
    late = torch.empty_like(want)
    assert lib.dflash_attention_rel_fwd_noalloc(*_common_args(inp, late), 0, s2.cuda_stream) == 0
    s2.synchronize()
    assert torch.equal(late, want)
