"""Benchmark of the fused DeBERTa disentangled-attention hot path on one MI355X.

Headline metric: fused attention TFLOP/s and fraction of the
fp16 dense MFMA peak at the attention microbench configuration
(B=32, L=512, H=12, d=64, c2p|p2c, position_buckets=256, max_rel=512), plus the
12-layer encoder latency at B=32, L=512 fp16 for the ``hip`` and the torch
``optimized`` backends on the same GPU.

A step is one launch of the fused attention over the whole batch with Q/K/V,
the projected relative rows, the LUT and the mask already resident in HBM.
``value`` counts F_attn = 4*B*H*L^2*d (QK^T + PV over the dense L) per step.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-encoder] [--skip-cpu]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for entry in (str(REPO / "disentangled-flash_amd"), str(REPO)):
    if entry not in sys.path:
        sys.path.insert(0, entry)

import torch  # noqa: E402

PEAK_TFLOPS = {"fp16": 2500.0, "bf16": 2500.0, "fp32": 157.3}
HBM_PEAK_GBS = 8000.0
LOG2E = 1.4426950408889634
DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
TRAFFIC_FILE = REPO / "profiles" / "attention_c2_fp16_traffic.json"


def log(message: str) -> None:
    print(message, file=sys.stderr, flush=True)


def c2_inputs(dtype: torch.dtype, padded: bool, seed: int = 2024, batch: int = 32,
              heads: int = 12, length: int = 512, dim: int = 64, device: str = "cuda",
              valid_lengths=None):
    """Attention microbenchmark inputs: Q/K/V and Qr/Kr ~ N(0,1)/sqrt(d); lengths U[256, 512] or none."""

    from disentangled_flash.position import compact_position_plan

    active, lut = compact_position_plan(length, position_buckets=256, max_relative_positions=512,
                                        position_embedding_size=256)
    gen = torch.Generator().manual_seed(seed)
    scale = 1.0 / math.sqrt(dim)
    q, k, v = (torch.randn(batch, heads, length, dim, generator=gen) * scale for _ in range(3))
    pos_key, pos_query = (torch.randn(heads, active.numel(), dim, generator=gen) * scale
                          for _ in range(2))
    if valid_lengths is not None:
        choices = torch.tensor(list(valid_lengths))
        lengths = choices[torch.arange(batch) % len(choices)].clamp(max=length)
        mask = torch.arange(length)[None] < lengths[:, None]
    elif padded:
        lengths = torch.randint(length // 2, length + 1, (batch,), generator=gen)
        mask = torch.arange(length)[None] < lengths[:, None]
    else:
        mask = torch.ones(batch, length, dtype=torch.bool)
    qkv = torch.cat([t.permute(0, 2, 1, 3).reshape(batch, length, heads * dim) for t in (q, k, v)],
                    dim=-1)
    to = lambda t: t.to(device, dtype).contiguous()  # noqa: E731
    return {
        "qkv": to(qkv), "q": to(q), "k": to(k), "v": to(v),
        "pos_key": to(pos_key), "pos_query": to(pos_query),
        "lut": lut.to(device), "mask": mask.to(device),
        "batch": batch, "heads": heads, "length": length, "dim": dim,
        "slots": active.numel(), "valid_fraction": float(mask.float().mean()),
    }


RAMP_SECONDS = 0.3


def ramp_clocks(fn, seconds: float = RAMP_SECONDS) -> None:
    """Run ``fn`` back to back for ``seconds`` (untimed) before a measurement.

    The MI355X runs a short burst of launches after an idle period below its
    sustained clock: the C2 kernel times about 112-118 us in the first few
    milliseconds of load and about 93 us once the load has lasted ~20 ms, and
    drops back after ~0.2 s idle.  Every timing below therefore starts from a
    ramp of this length, so the numbers are the steady-state rates.
    """

    fn()  # first-call set-up (library load, op registration) is not load
    torch.cuda.synchronize()
    deadline = time.perf_counter() + seconds
    launches = 0
    while time.perf_counter() < deadline or launches < 20:
        for _ in range(10):
            fn()
        launches += 10
        torch.cuda.synchronize()


def time_launches(fn, steps: int, warmup: int) -> float:
    """Average milliseconds per call over ``steps`` back-to-back calls (HIP events)."""

    ramp_clocks(fn)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def time_p50(fn, steps: int, warmup: int) -> float:
    """Median milliseconds of individually event-timed calls."""

    ramp_clocks(fn)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    samples = []
    for _ in range(steps):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        fn()
        end.record()
        end.synchronize()
        samples.append(start.elapsed_time(end))
    return statistics.median(samples)


def fused_call(inp, has_c2p: bool = True, has_p2c: bool = True, key_splits: int = 0,
               strict_fp32: bool = True):
    from disentangled_flash.kernel import deberta_attention_rel

    scale_log2 = LOG2E / math.sqrt((1 + int(has_c2p) + int(has_p2c)) * inp["dim"])
    return lambda: deberta_attention_rel(inp["qkv"], inp["pos_key"], inp["pos_query"], inp["lut"],
                                         inp["mask"], inp["heads"], inp["dim"], scale_log2,
                                         has_c2p, has_p2c, strict_fp32, key_splits)


# Kernel dtypes of the edge sweep and the profiling target: "fp32-fast" is fp32
# data with fp32_precision="fast" (bf16x3 products).
KERNEL_DTYPES = {**{name: (dtype, True) for name, dtype in DTYPES.items()},
                 "fp32-fast": (torch.float32, False)}


def table_call(inp, precomputed: bool = False):
    """Reference data flow: two separate score GEMMs, then the table-reading kernel
    (the reference op's contract).  With ``precomputed`` the tables are computed once
    and only the kernel runs."""

    from disentangled_flash.kernel import deberta_attention

    scale_log2 = LOG2E / math.sqrt(3 * inp["dim"])

    def tables():
        return (torch.matmul(inp["q"], inp["pos_key"].transpose(-1, -2)),
                torch.matmul(inp["k"], inp["pos_query"].transpose(-1, -2)))

    fixed = tables() if precomputed else None

    def run():
        c2p, p2c = fixed if fixed is not None else tables()
        return deberta_attention(inp["q"], inp["k"], inp["v"], c2p, p2c, inp["lut"], inp["mask"],
                                 inp["heads"], inp["length"], inp["slots"], scale_log2,
                                 True, True, inp["q"].dtype == torch.bfloat16,
                                 inp["q"].dtype == torch.float32, True)

    return run


def torch_optimized_call(inp):
    """The prepared torch equation (``_torch.py:339-387``) on the GPU from resident Q/K/V."""

    from disentangled_flash.position import SharedPositionPlanCache

    cache = SharedPositionPlanCache(position_buckets=256, max_relative_positions=512,
                                    position_embedding_size=256)
    pair = cache.dense(inp["length"], inp["q"].device).pair_to_local
    b, h, length = inp["batch"], inp["heads"], inp["length"]
    scale = math.sqrt(3 * inp["dim"])
    q, k, v = inp["q"], inp["k"], inp["v"]
    mask = inp["mask"]

    def run():
        index = pair.expand(b, h, length, length)
        scores = torch.matmul(q, k.transpose(-1, -2) / scale)
        scores = scores + torch.gather(torch.matmul(q, inp["pos_key"].transpose(-1, -2)) / scale,
                                       -1, index)
        raw = torch.matmul(k, inp["pos_query"].transpose(-1, -2)) / scale
        scores = scores + torch.gather(raw.transpose(-1, -2), -2, index)
        pairm = mask[:, None, None, :] & mask[:, None, :, None]
        scores = scores.masked_fill(~pairm, torch.finfo(q.dtype).min)
        ctx = torch.matmul(torch.softmax(scores, dim=-1), v)
        return ctx.permute(0, 2, 1, 3).reshape(b, length, h * inp["dim"])

    return run


def attention_flops(inp) -> float:
    return 4.0 * inp["batch"] * inp["heads"] * inp["length"] ** 2 * inp["dim"]


def relative_flops(inp) -> float:
    return 4.0 * inp["batch"] * inp["heads"] * inp["length"] * inp["slots"] * inp["dim"]


def algorithmic_bytes(inp) -> float:
    """HBM bytes a fused launch must move: Q, K, V, O, the relative rows, LUT and mask."""

    esize = inp["qkv"].element_size()
    per_tensor = inp["batch"] * inp["heads"] * inp["length"] * inp["dim"] * esize
    rel = 2 * inp["heads"] * inp["slots"] * inp["dim"] * esize
    return 4 * per_tensor + rel + inp["lut"].numel() * 4 + inp["mask"].numel()


def encoder_config():
    from transformers import DebertaV2Config

    return DebertaV2Config(
        vocab_size=128100, hidden_size=768, num_hidden_layers=12, num_attention_heads=12,
        intermediate_size=3072, hidden_act="gelu", hidden_dropout_prob=0.0,
        attention_probs_dropout_prob=0.0, max_position_embeddings=512, type_vocab_size=0,
        initializer_range=0.02, layer_norm_eps=1e-7, relative_attention=True,
        max_relative_positions=-1, position_buckets=256, pos_att_type=["p2c", "c2p"],
        norm_rel_ebd="layer_norm", share_att_key=True, conv_kernel_size=3, conv_act="gelu",
        position_biased_input=False,
    )


def encoder_inputs(batch: int, length: int, dtype, device, seed: int = 19):
    """Embedding-table hidden states and U[L/2, L] right-padded masks (C3)."""

    gen = torch.Generator().manual_seed(seed)
    table = torch.randn(128100, 768, generator=gen) * 0.02
    table[0].zero_()
    tokens = torch.randint(1, 128100, (batch, length), generator=gen)
    lengths = torch.randint(length // 2, length + 1, (batch,), generator=gen)
    mask = torch.arange(length)[None] < lengths[:, None]
    tokens = tokens.masked_fill(~mask, 0)
    hidden = table[tokens].to(device=device, dtype=dtype).contiguous()
    # Integer mask, as a tokenizer produces it (Hugging Face's ConvLayer computes 1 - mask).
    return hidden, mask.to(device=device, dtype=torch.long)


def _sig(v, digits: int = 4):
    """Floats to ``digits`` significant digits for the JSON line (errors are ~1e-6)."""

    return float(f"{v:.{digits}g}") if isinstance(v, float) else v


def forward_peak_bytes(run) -> int:
    """Peak bytes a forward allocates on top of what is resident before it."""

    torch.cuda.synchronize()
    resident = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    run()
    torch.cuda.synchronize()
    return torch.cuda.max_memory_allocated() - resident


def bench_encoder(batch: int, length: int, steps: int, warmup: int,
                  backends=("original", "optimized", "hip"), dtype=torch.float16,
                  fp32_precision: str = "strict"):
    """12-layer encoder latency: HF original vs torch ``optimized`` vs ``hip``.

    ``<backend>_peak_gb`` is the reference's peak-memory figure for one model
    (``benchmark_cuda.py:548-551`` resets the peak counter before its measured
    calls): the encoder's parameters, the inputs and the forward's peak
    allocation on top of them.
    """

    import copy

    from transformers import DebertaV2Model

    from disentangled_flash import enable_deberta_inference

    torch.manual_seed(17)
    base = DebertaV2Model(encoder_config()).to("cuda", dtype).eval()
    hidden, mask = encoder_inputs(batch, length, dtype, "cuda")
    weights = sum(t.numel() * t.element_size()
                  for t in list(base.encoder.parameters()) + list(base.encoder.buffers()))
    resident = weights + hidden.numel() * hidden.element_size() + mask.numel() * mask.element_size()
    results = {}
    with torch.inference_mode():
        original = base.encoder
        original_run = lambda: original(hidden, mask, output_hidden_states=False)  # noqa: E731
        if "original" in backends:
            results["original_ms"] = time_p50(original_run, steps, warmup)
            results["original_peak_gb"] = round(
                (resident + forward_peak_bytes(original_run)) / 1e9, 3)
        reference_out = original_run().last_hidden_state
        for backend in (b for b in ("optimized", "hip") if b in backends):
            model = copy.deepcopy(base)
            enable_deberta_inference(model, backend=backend, sequence_lengths=[length],
                                     fp32_precision=fp32_precision)
            encoder = model.encoder
            plans = encoder.active_plans
            run = lambda: encoder.forward_prepared(hidden, mask, plans,  # noqa: E731
                                                   output_hidden_states=False)
            results[f"{backend}_ms"] = time_p50(run, steps, warmup)
            results[f"{backend}_peak_gb"] = round((resident + forward_peak_bytes(run)) / 1e9, 3)
            out = run().last_hidden_state
            results[f"{backend}_max_abs_err_vs_original"] = float(
                (out.float() - reference_out.float()).abs().max())
            del model, encoder
            torch.cuda.empty_cache()
    if "optimized_ms" in results and "hip_ms" in results:
        results["speedup_vs_optimized"] = results["optimized_ms"] / results["hip_ms"]
    if "original_ms" in results and "hip_ms" in results:
        results["speedup_vs_original"] = results["original_ms"] / results["hip_ms"]
    return results


def bench_sweep(steps: int, warmup: int, batches=(1, 8, 16, 32),
                lengths=(16, 32, 64, 128, 256, 384, 512)):
    """C3 sweep: 12-layer fp16 encoder latency over B x L for original / optimized / hip.

    ``hip_graph_ms`` replays the hip encoder from a HIP graph captured for that (B, L).

    One random-init model; the ``optimized`` and ``hip`` copies are prepared for every
    bucket once, then each (B, L) is timed with the bucket activated (median of
    individually event-timed forwards, launch gaps included).
    """

    import copy

    from transformers import DebertaV2Model

    from disentangled_flash import enable_deberta_inference

    torch.manual_seed(17)
    base = DebertaV2Model(encoder_config()).to("cuda", torch.float16).eval()
    from disentangled_flash import capture_deberta_buckets

    prepared = {}
    for backend in ("optimized", "hip"):
        model = copy.deepcopy(base)
        enable_deberta_inference(model, backend=backend, sequence_lengths=list(lengths))
        prepared[backend] = model.encoder
    rows = []
    with torch.inference_mode():
        for length in lengths:
            for batch in batches:
                hidden, mask = encoder_inputs(batch, length, torch.float16, "cuda")
                row = {"batch": batch, "seq_len": length}
                row["original_ms"] = time_p50(
                    lambda: base.encoder(hidden, mask, output_hidden_states=False), steps, warmup)
                for backend, encoder in prepared.items():
                    encoder.activate_shape(length)
                    plans = encoder.active_plans
                    row[f"{backend}_ms"] = time_p50(
                        lambda: encoder.forward_prepared(hidden, mask, plans,  # noqa: B023
                                                         output_hidden_states=False),
                        steps, warmup)
                # the hip encoder replayed from a HIP graph (input copies included)
                bucket = capture_deberta_buckets(prepared["hip"], [(batch, length)])[
                    (batch, length)]
                row["hip_graph_ms"] = time_p50(lambda: bucket(hidden, mask),  # noqa: B023
                                               steps, warmup)
                del bucket
                row = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in row.items()}
                log(json.dumps(row))
                rows.append(row)
    return rows


def bench_gemm_table(reps: int = 20):
    """Per-GEMM device time of the encoder projections, hipBLASLt against the
    hand-written GEMM's tile configurations, at C3 (base, fp16) and C4 (xlarge,
    bf16) widths and few to many rows.  Each entry replays a HIP graph of ``reps``
    back-to-back calls, so host launch cost is excluded; us per call.  hipBLASLt
    is ``F.linear`` (plus ``F.gelu`` for the intermediate; the residual of the
    dense layers folds into the following add + LayerNorm there)."""

    import torch.nn.functional as F

    from disentangled_flash import _lib

    lib = _lib.load()

    def graph_us(fn):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                fn()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                fn()
        for _ in range(10):
            graph.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(10):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / 10 / reps * 1e3

    gen = torch.Generator().manual_seed(31)
    rows = []
    for width, dtype, row_counts in ((768, torch.float16, (512, 2048, 8192, 16384)),
                                     (1536, torch.bfloat16, (512, 2048))):
        shapes = (("qkv", width, 3 * width, 0), ("attention_output", width, width, 2),
                  ("ffn_intermediate_gelu", width, 4 * width, 1),
                  ("ffn_output", 4 * width, width, 2))
        for m in row_counts:
            for name, k, n, epilogue in shapes:
                x = (torch.randn(m, k, generator=gen) * 0.5).to("cuda", dtype)
                w = (torch.randn(n, k, generator=gen) * 0.02).to("cuda", dtype)
                b = (torch.randn(n, generator=gen) * 0.02).to("cuda", dtype)
                r = torch.randn(m, n, generator=gen).to("cuda", dtype)
                y = torch.empty(m, n, device="cuda", dtype=dtype)
                if epilogue == 1:
                    library = graph_us(lambda: F.gelu(F.linear(x, w, b)))  # noqa: B023
                else:
                    library = graph_us(lambda: F.linear(x, w, b))  # noqa: B023
                row = {"hidden": width, "dtype": str(dtype).replace("torch.", ""), "rows": m,
                       "gemm": name, "hipblaslt_us": round(library, 2)}
                for config in (2, 3, 4, 5):
                    def call(config=config):
                        return lib.dflash_linear_fwd(
                            x.data_ptr(), w.data_ptr(), b.data_ptr(), r.data_ptr(),  # noqa: B023
                            y.data_ptr(), m, n, k, epilogue | (config << 8),  # noqa: B023
                            _lib.DTYPE_CODES[dtype], _lib.current_stream_handle(x.device))  # noqa: B023
                    if call() != 0:
                        continue
                    row[f"config{config}_us"] = round(graph_us(call), 2)
                log(json.dumps(row))
                rows.append(row)
    return rows


def bench_edge(steps: int, warmup: int):
    """C5 edge sweep: the fused attention op for d=128/H=8 (B=16, L=512) and d=32/H=16
    (B=16, L=384) in fp16/bf16/fp32 x {c2p, p2c, c2p|p2c}, boundary valid lengths
    {1, 63, 64, 65, 127, 129, 383, 384, 511, 512} mixed in the batch."""

    boundary = (1, 63, 64, 65, 127, 129, 383, 384, 511, 512)
    rows = []
    for dim, heads, length in ((128, 8, 512), (32, 16, 384)):
        for name, (dtype, strict) in KERNEL_DTYPES.items():
            inp = c2_inputs(dtype, padded=True, batch=16, heads=heads, length=length, dim=dim,
                            valid_lengths=boundary)
            for mode, (c2p, p2c) in (("c2p", (True, False)), ("p2c", (False, True)),
                                     ("c2p|p2c", (True, True))):
                ms = time_launches(fused_call(inp, c2p, p2c, strict_fp32=strict), steps, warmup)
                row = {"head_dim": dim, "heads": heads, "batch": 16, "seq_len": length,
                       "dtype": name, "mode": mode, "us": round(ms * 1e3, 1),
                       "tflops_f_attn": round(attention_flops(inp) / ms / 1e9, 1)}
                log(json.dumps(row))
                rows.append(row)
            del inp
            torch.cuda.empty_cache()
    return rows


KERNEL_SHAPES = {
    # name: (batch, heads, length, head_dim, boundary valid lengths?)
    "c2": (32, 12, 512, 64, False),
    "c5_d32": (16, 16, 384, 32, True),
    "c5_d128": (16, 8, 512, 128, True),
}
BOUNDARY_LENGTHS = (1, 63, 64, 65, 127, 129, 383, 384, 511, 512)


def kernel_inputs(shape: str, dtype):
    batch, heads, length, dim, boundary = KERNEL_SHAPES[shape]
    return c2_inputs(dtype, padded=False, batch=batch, heads=heads, length=length, dim=dim,
                     valid_lengths=BOUNDARY_LENGTHS if boundary else None)


def bench_tile_sweep(steps: int, warmup: int):
    """Per-shape tile evidence: the fused fp16 op (c2p|p2c, no split) over batch sizes for
    d=64 (H=12, L=512), d=32 (H=16, L=384) and d=128 (H=8, L=512).  The tile the library
    picks can be forced per process with DFLASH_REL_QW=16 or 32 (d=32 and 16-bit d=128 have both)."""

    import os

    rows = []
    cases = ([(64, 12, 512, b) for b in (1, 2, 4, 8, 12, 16, 24, 32, 48)]
             + [(32, 16, 384, b) for b in (1, 4, 8, 10, 11, 12, 13, 14, 16, 24, 32)]
             + [(128, 8, 512, b) for b in (1, 4, 8, 16, 32)])
    for dim, heads, length, batch in cases:
        inp = c2_inputs(torch.float16, padded=False, batch=batch, heads=heads, length=length,
                        dim=dim)
        ms = time_launches(fused_call(inp, key_splits=1), steps, warmup)
        row = {"head_dim": dim, "heads": heads, "seq_len": length, "batch": batch,
               "qw32_workgroups": batch * heads * ((length + 127) // 128),
               "forced_qw": os.environ.get("DFLASH_REL_QW", "table"), "us": round(ms * 1e3, 2)}
        log(json.dumps(row))
        rows.append(row)
        del inp
    return rows


def bench_c4(steps: int, warmup: int):
    """C4: 24-layer DeBERTa-v2-xlarge-shaped encoder, bf16, B=8, one batch per bucket.

    Valid lengths are log-normal (median 60) clipped to [16, 256]; each batch holds the
    lengths that fall in its bucket {64, 128, 256}, padded to the bucket.
    """

    import copy

    from transformers import DebertaV2Config, DebertaV2Model

    from disentangled_flash import capture_deberta_buckets, enable_deberta_inference

    config = DebertaV2Config(
        vocab_size=128100, hidden_size=1536, num_hidden_layers=24, num_attention_heads=24,
        intermediate_size=6144, hidden_act="gelu", hidden_dropout_prob=0.0,
        attention_probs_dropout_prob=0.0, max_position_embeddings=512, type_vocab_size=0,
        initializer_range=0.02, layer_norm_eps=1e-7, relative_attention=True,
        max_relative_positions=512, position_buckets=256, pos_att_type=["p2c", "c2p"],
        norm_rel_ebd="layer_norm", share_att_key=True, conv_kernel_size=3, conv_act="gelu",
        position_biased_input=False,
    )
    torch.manual_seed(17)
    base = DebertaV2Model(config).to("cuda", torch.bfloat16).eval()
    buckets = (64, 128, 256)
    prepared = {}
    for backend in ("optimized", "hip"):
        model = copy.deepcopy(base)
        enable_deberta_inference(model, backend=backend, sequence_lengths=list(buckets))
        prepared[backend] = model.encoder
    gen = torch.Generator().manual_seed(23)
    pool = torch.exp(torch.randn(4096, generator=gen) * 0.75 + math.log(60.0)).clamp(16, 256)
    pool = pool.long()
    rows = []
    with torch.inference_mode():
        lower = 0
        for bucket in buckets:
            in_bucket = (pool > lower) & (pool <= bucket)
            lengths = pool[in_bucket][:8]
            share = float(in_bucket.float().mean())
            lower = bucket
            mask = (torch.arange(bucket)[None] < lengths[:, None]).long().cuda()
            hidden = (torch.randn(8, bucket, 1536, generator=gen) * 0.5).to("cuda", torch.bfloat16)
            hidden = hidden * mask[..., None]
            row = {"bucket": bucket, "batch": 8, "bucket_share": round(share, 3),
                   "mean_valid": round(float(lengths.float().mean()), 1)}
            row["original_ms"] = time_p50(
                lambda: base.encoder(hidden, mask, output_hidden_states=False), steps, warmup)
            for backend, encoder in prepared.items():
                encoder.activate_shape(bucket)
                plans = encoder.active_plans
                row[f"{backend}_ms"] = time_p50(
                    lambda: encoder.forward_prepared(hidden, mask, plans,  # noqa: B023
                                                     output_hidden_states=False),
                    steps, warmup)
            graph = capture_deberta_buckets(prepared["hip"], [(8, bucket)])[(8, bucket)]
            row["hip_graph_ms"] = time_p50(lambda: graph(hidden, mask), steps, warmup)  # noqa: B023
            del graph
            row = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in row.items()}
            log(json.dumps(row))
            rows.append(row)
    return rows


def cpu_baseline(target_seconds: float = 12.0, c1_seconds: float = 4.0):
    """Oracle restatement of the ``optimized`` equation, fp32, on the host CPU.

    C2 (the reported value): a bounded sample of the C2 workload, one sequence
    (B=1 of 32) at L=512, H=12, d=64 per call, repeated for about
    ``target_seconds``, in the headline unit (F_attn TFLOP/s).  C1: the
    CPU-runnable single layer (B=2, L=128, hidden 768, fused QKV projection
    included), median milliseconds per call.

    Threads: every host CPU, capped at the 16 a one-GPU box grants a job; both
    the thread count and the host's CPU count are reported.
    """

    from oracle.optimized import optimized_attention, optimized_core
    from oracle.positions import compact_plan, dense_map

    host_cpus = os.cpu_count() or 1
    cores = min(host_cpus, 16)
    torch.set_num_threads(cores)

    def timed(fn, seconds):
        for _ in range(2):
            fn()
        samples = []
        start = time.perf_counter()
        while time.perf_counter() - start < seconds or len(samples) < 5:
            t0 = time.perf_counter()
            fn()
            samples.append(time.perf_counter() - t0)
        return statistics.median(samples), len(samples), sum(samples)

    def pair_map(length):
        lut = compact_plan(length, position_buckets=256, max_relative_positions=512,
                           position_embedding_size=256)[1]
        return torch.from_numpy(dense_map(lut, length))

    inp = c2_inputs(torch.float32, padded=True, batch=1, device="cpu")
    pair = pair_map(512)
    args = (inp["q"], inp["k"], inp["v"], inp["pos_key"], inp["pos_query"], pair, inp["mask"],
            math.sqrt(192))
    median, calls, total = timed(lambda: optimized_core(*args), target_seconds)

    # C1: B=2, L=128, hidden 768, 12 heads, weights N(0, 0.02), lengths U[64, 128].
    gen = torch.Generator().manual_seed(17)
    hidden = torch.randn(2, 128, 768, generator=gen)
    weight = torch.randn(3 * 768, 768, generator=gen) * 0.02
    bias = torch.zeros(3 * 768)
    s1 = compact_plan(128, position_buckets=256, max_relative_positions=512,
                      position_embedding_size=256)[0].size
    pk, pq = (torch.randn(12, s1, 64, generator=gen) * 0.02 for _ in range(2))
    lengths = torch.randint(64, 129, (2,), generator=gen)
    mask1 = torch.arange(128)[None] < lengths[:, None]
    pair1 = pair_map(128)
    c1_median, c1_calls, _ = timed(
        lambda: optimized_attention(hidden, weight, bias, pk, pq, pair1, mask1, 12, 64), c1_seconds)
    return {
        "value": attention_flops(inp) / median / 1e12,
        "unit": "TFLOP/s",
        "cores": cores,
        "host_cpus": host_cpus,
        "kind": "port",
        "sample": (f"oracle/optimized.py optimized_core, fp32, {cores} threads of {host_cpus} "
                   f"host CPUs, B=1 of the B=32 C2 batch (L=512 H=12 d=64, padded), {calls} "
                   f"calls in {total:.1f}s, median {median * 1e3:.2f} ms/call"),
        "c1_layer_ms": round(c1_median * 1e3, 3),
        "c1_sample": (f"oracle/optimized.py optimized_attention (fused QKV linear + attention), "
                      f"fp32, C1 B=2 L=128 hidden 768 H=12, {c1_calls} calls, median"),
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--encoder-steps", type=int, default=20)
    parser.add_argument("--skip-encoder", action="store_true")
    parser.add_argument("--skip-cpu", action="store_true")
    parser.add_argument("--kernel-only", action="store_true",
                        help="launch only the fused C2 kernel: the clock ramp, then --steps "
                             "launches (profiling driver)")
    parser.add_argument("--kernel-shape", choices=sorted(KERNEL_SHAPES), default="c2",
                        help="shape of --kernel-only: c2 (B=32 L=512 H=12 d=64), c5_d32 "
                             "(B=16 L=384 H=16 d=32), c5_d128 (B=16 L=512 H=8 d=128); the C5 "
                             "shapes mix the boundary valid lengths")
    parser.add_argument("--kernel-dtype", choices=sorted(KERNEL_DTYPES), default="fp16")
    parser.add_argument("--table-only", action="store_true",
                        help="launch only the reference-contract kernel (dflash_attention_fwd) on "
                             "precomputed C2 fp16 c2p/p2c tables: the clock ramp, then --steps "
                             "launches (profiling driver)")
    parser.add_argument("--tile-sweep", action="store_true",
                        help="fused op over batch sizes for d=32/64/128 (tile-table evidence)")
    parser.add_argument("--encoder-only", action="store_true",
                        help="time only the hip 12-layer encoder (profiling driver)")
    parser.add_argument("--sweep", action="store_true",
                        help="C3 encoder sweep B x L (original / optimized / hip), one JSON line")
    parser.add_argument("--edge", action="store_true",
                        help="C5 head-dim / precision / mode sweep of the fused op, one JSON line")
    parser.add_argument("--c4", action="store_true",
                        help="C4 24-layer xlarge bf16 encoder per bucket, one JSON line")
    parser.add_argument("--gemm-table", action="store_true",
                        help="per-GEMM device times in HIP graphs, hipBLASLt vs the hand-written "
                             "configurations, one JSON line")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="one 256 MiB device-to-device copy (HBM counter calibration)")
    args = parser.parse_args()
    if args.gpus != 1:
        print("bench.py measures the single-GPU hot path only: this build runs on one GPU "
              "(the attention grid shards over batch and heads with no exchange); use --gpus 1.",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1

    from disentangled_flash import _lib

    _lib.load()
    torch.backends.cuda.matmul.allow_tf32 = False
    log(f"device: {torch.cuda.get_device_name(0)}")

    if args.copy_calibration:
        src = torch.ones(128 * 1024 * 1024, dtype=torch.float16, device="cuda")  # 256 MiB
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copied {src.numel() * src.element_size()} bytes")
        return 0
    if args.edge:
        print(json.dumps({"edge": "C5 fused attention", "rows": bench_edge(args.steps, args.warmup)}),
              flush=True)
        return 0
    if args.c4:
        rows = bench_c4(max(5, args.encoder_steps // 2), 3)
        print(json.dumps({"c4": "24-layer xlarge bf16 encoder, ms (median)", "rows": rows}),
              flush=True)
        return 0
    if args.sweep:
        rows = bench_sweep(max(5, args.encoder_steps // 2), 3)
        print(json.dumps({"sweep": "C3 12-layer encoder fp16, ms (median)", "rows": rows}),
              flush=True)
        return 0
    if args.encoder_only:
        enc = bench_encoder(32, 512, args.encoder_steps, 3, backends=("hip",))
        log(f"encoder: {enc}")
        return 0
    if args.gemm_table:
        print(json.dumps({"gemm_table": "us per call, HIP-graph replay", "rows": bench_gemm_table()}),
              flush=True)
        return 0
    if args.tile_sweep:
        print(json.dumps({"tile_sweep": "fused fp16 c2p|p2c, unsplit, us",
                          "rows": bench_tile_sweep(args.steps, args.warmup)}), flush=True)
        return 0
    if args.table_only:
        call = table_call(c2_inputs(torch.float16, padded=False), precomputed=True)
        ramp_clocks(call)
        torch.cuda.synchronize()
        for _ in range(args.steps):
            call()
        torch.cuda.synchronize()
        log(f"launched the reference-contract C2 kernel {args.steps} times")
        return 0
    if args.kernel_only:
        dtype, strict = KERNEL_DTYPES[args.kernel_dtype]
        inp = kernel_inputs(args.kernel_shape, dtype)
        call = fused_call(inp, strict_fp32=strict)
        ramp_clocks(call)
        torch.cuda.synchronize()
        for _ in range(args.steps):
            call()
        torch.cuda.synchronize()
        log(f"launched the fused {args.kernel_shape} kernel {args.steps} times")
        return 0

    # ---- headline: fused fp16 attention, C2 without padding (every FLOP real) ----
    full = c2_inputs(torch.float16, padded=False)
    f_attn = attention_flops(full)
    f_rel = relative_flops(full)
    ms = time_launches(fused_call(full), args.steps, args.warmup)
    tflops = f_attn / (ms * 1e-3) / 1e12
    log(f"fused fp16 unpadded: {ms * 1e3:.1f} us  {tflops:.1f} TFLOP/s (F_attn)")

    extra = {}
    padded = c2_inputs(torch.float16, padded=True)
    ms_pad = time_launches(fused_call(padded), args.steps, args.warmup)
    extra["fp16_padded"] = {"us": ms_pad * 1e3, "tflops_f_attn": f_attn / ms_pad / 1e9,
                            "valid_fraction": padded["valid_fraction"]}
    for name in ("bf16",):
        inp = c2_inputs(DTYPES[name], padded=False)
        t = time_launches(fused_call(inp), args.steps, args.warmup)
        extra[f"{name}_unpadded"] = {"us": t * 1e3, "tflops_f_attn": f_attn / t / 1e9}
        del inp
    t_table = time_launches(table_call(full), max(5, args.steps // 5), 3)
    extra["reference_dataflow_fp16_us"] = t_table * 1e3
    t_contract = time_launches(table_call(full, precomputed=True), max(5, args.steps // 5), 3)
    extra["reference_contract_kernel_fp16_us"] = t_contract * 1e3
    t_torch = time_launches(torch_optimized_call(full), max(5, args.steps // 5), 2)
    extra["torch_optimized_attention_fp16_us"] = t_torch * 1e3
    extra["speedup_vs_torch_optimized_attention"] = t_torch / ms
    log(f"table data flow {t_table * 1e3:.1f} us (kernel alone {t_contract * 1e3:.1f} us), "
        f"torch optimized {t_torch * 1e3:.1f} us")
    del padded
    torch.cuda.empty_cache()

    traffic = None
    if TRAFFIC_FILE.exists():
        traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")

    line = {
        "metric": "fused attn TFLOP/s (% MFMA peak) + 12-layer encoder ms, B=32 L=512 fp16",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": "attention microbench (BASELINE configs[1]): fused disentangled attention, "
                        "c2p|p2c, no padding; F_attn = 4*B*H*L^2*d numerator",
            "batch": full["batch"], "seq_len": full["length"], "heads": full["heads"],
            "head_dim": full["dim"], "active_slots": full["slots"], "position_buckets": 256,
            "max_relative_positions": 512, "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(tflops, 2),
            "peak": PEAK_TFLOPS["fp16"],
            "unit": "TFLOP/s",
            "frac": round(tflops / PEAK_TFLOPS["fp16"], 4),
            "traffic": traffic,
            "f_total_tflops": round((f_attn + f_rel) / (ms * 1e-3) / 1e12, 2),
            "f_total_frac": round((f_attn + f_rel) / (ms * 1e-3) / 1e12 / PEAK_TFLOPS["fp16"], 4),
            "algorithmic_bytes": algorithmic_bytes(full),
            "algorithmic_gbs": round(algorithmic_bytes(full) / (ms * 1e-3) / 1e9, 1),
        },
        "extra": extra,
    }
    del full
    torch.cuda.empty_cache()

    if not args.skip_encoder:
        enc = bench_encoder(32, 512, args.encoder_steps, 3)
        line["encoder"] = {"batch": 32, "seq_len": 512, "layers": 12, "dtype": "fp16",
                           **{k: _sig(v) for k, v in enc.items()}}
        log(f"encoder: {enc}")
        # fp32 at the same shape (the reference publishes its fp32 encoder latency
        # there, README.md:210): strict and the bf16x3 fast mode, a few forwards each.
        enc32 = bench_encoder(32, 512, 5, 2, dtype=torch.float32)
        fast32 = bench_encoder(32, 512, 5, 2, backends=("hip",), dtype=torch.float32,
                               fp32_precision="fast")
        line["encoder"]["fp32"] = {
            **{k: _sig(v) for k, v in enc32.items()},
            "hip_fast_ms": _sig(fast32["hip_ms"]),
            "hip_fast_peak_gb": _sig(fast32["hip_peak_gb"]),
            "hip_fast_max_abs_err_vs_original": _sig(fast32["hip_max_abs_err_vs_original"]),
        }
        log(f"encoder fp32: {line['encoder']['fp32']}")
        # A launch-bound C3 cell (B=8, L=128): eager forward_prepared, as the reference's
        # benchmark times it (benchmark_cuda.py:781-782), and the HIP-graph replay.
        small = bench_sweep(args.encoder_steps, 3, batches=(8,), lengths=(128,))[0]
        line["encoder"]["c3_b8_l128"] = {k: _sig(v) for k, v in small.items()
                                         if k not in ("batch", "seq_len")}
    if not args.skip_cpu:
        line["cpu_baseline"] = cpu_baseline()
        log(f"cpu baseline: {line['cpu_baseline']}")
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
