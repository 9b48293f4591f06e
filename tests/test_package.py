"""CPU tests of the package: public API, plans, torch backend, encoder wrapper, C ABI exports."""

from __future__ import annotations

import copy
import math
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import REPO, load_case
from oracle.attention import original_attention
from oracle.positions import compact_plan


def test_public_api_imports():
    import disentangled_flash as df

    assert callable(df.optimize_deberta)
    assert callable(df.enable_deberta_inference)
    assert callable(df.compile_deberta_buckets)
    assert df.DisentangledFlashAttention.__name__ == "HipInferenceDisentangledSelfAttention"
    assert re.match(r"^\d+\.\d+\.\d+$", df.__version__)


def test_position_plan_matches_oracle():
    from disentangled_flash.position import SharedPositionPlanCache

    cache = SharedPositionPlanCache(position_buckets=256, max_relative_positions=512,
                                    position_embedding_size=256)
    for length in (1, 17, 65, 128, 129, 384, 512, 700):
        plan = cache.compact(length, "cpu")
        active, lut = compact_plan(length, position_buckets=256, max_relative_positions=512,
                                   position_embedding_size=256)
        np.testing.assert_array_equal(plan.active_slots.numpy(), active)
        np.testing.assert_array_equal(plan.delta_to_local.numpy(), lut)
        assert plan.delta_to_local.dtype == torch.int32
    assert cache.compact(65, "cpu") is cache.compact(65, "cpu")
    dense = cache.dense(9, "cpu")
    assert dense.pair_to_local.shape == (1, 1, 9, 9)
    with pytest.raises(ValueError):
        cache.compact(0, "cpu")


def _config(case_spec, **overrides):
    from disentangled_flash.modeling import DebertaAttentionConfig

    fields = dict(
        hidden_size=case_spec.hidden_size, num_attention_heads=case_spec.num_heads,
        attention_head_size=case_spec.head_dim, relative_attention=True,
        max_relative_positions=case_spec.max_relative_positions,
        position_buckets=case_spec.position_buckets, share_att_key=case_spec.share_att_key,
        pos_att_type=case_spec.pos_att_type, hidden_dropout_prob=0.0,
        attention_probs_dropout_prob=0.0, norm_rel_ebd="none",
    )
    fields.update(overrides)
    return DebertaAttentionConfig(**fields)


def _load_params(module, params):
    with torch.no_grad():
        for name, value in params.items():
            proj, kind = name.rsplit("_", 1)
            getattr(module, f"{proj}_proj").__getattr__(kind).copy_(torch.from_numpy(value))


@pytest.mark.parametrize("case", ["v3_small", "c2p_separate_buckets16", "p2c_d128_unbucketed",
                                  "fully_masked_row", "length1"])
def test_original_module_matches_golden(case):
    from disentangled_flash.modeling import DisentangledSelfAttention

    spec, params, hidden, rel, mask, expected = load_case(case)
    module = DisentangledSelfAttention(_config(spec)).double().eval()
    _load_params(module, params)
    m = torch.from_numpy(mask)
    pair = m[:, None, None, :] & m[:, None, :, None]
    with torch.no_grad():
        out, _ = module(torch.from_numpy(hidden).double(), pair,
                        rel_embeddings=torch.from_numpy(rel).double())
    np.testing.assert_allclose(out.numpy(), expected, atol=1e-10)


@pytest.mark.parametrize("case", ["v3_small", "c2p_separate_buckets16", "p2c_d128_unbucketed",
                                  "fully_masked_row", "no_relative"])
def test_torch_backend_matches_oracle(case):
    from disentangled_flash._torch import TorchInferenceDisentangledSelfAttention

    spec, params, hidden, rel, mask, _ = load_case(case)
    module = TorchInferenceDisentangledSelfAttention(_config(spec)).double().eval()
    _load_params(module, params)
    module.prepare_for_inference(torch.from_numpy(rel).double())
    with torch.inference_mode():
        out, _ = module(torch.from_numpy(hidden).double(), torch.from_numpy(mask))
    exact = original_attention(spec, params, hidden, rel, mask,
                               scale=math.sqrt(spec.head_dim * spec.scale_factor))
    np.testing.assert_allclose(out.numpy(), exact, atol=1e-10)


@pytest.mark.parametrize("case", ["v3_small", "c2p_separate_buckets16", "p2c_d128_unbucketed"])
@pytest.mark.parametrize("rel_kind", ["standard", "shifted", "4d"])
def test_torch_backend_custom_relative_pos_matches_original(case, rel_kind):
    """Caller-provided relative_pos (the dynamic plan path) against the HF original module."""

    from disentangled_flash._torch import TorchInferenceDisentangledSelfAttention
    from disentangled_flash.modeling import DisentangledSelfAttention, build_relative_position

    spec, params, hidden, rel, mask, _ = load_case(case)
    config = _config(spec)
    original = DisentangledSelfAttention(config).double().eval()
    fast = TorchInferenceDisentangledSelfAttention(config).double().eval()
    _load_params(original, params)
    _load_params(fast, params)
    h = torch.from_numpy(hidden).double()
    length = h.size(1)
    probe = h.view(h.size(0), 1, length, -1)
    rpos = build_relative_position(probe, probe, spec.position_buckets,
                                   spec.max_relative_positions)       # [1, L, L]
    if rel_kind == "shifted":
        rpos = (rpos + 3)[0]                                           # [L, L], off-centre
    elif rel_kind == "4d":
        rpos = rpos[None]                                              # [1, 1, L, L]
    m = torch.from_numpy(mask)
    pair = m[:, None, None, :] & m[:, None, :, None]
    r = torch.from_numpy(rel).double()
    with torch.inference_mode():
        want, _ = original(h, pair, relative_pos=rpos, rel_embeddings=r)
        got, _ = fast(h, m, relative_pos=rpos, rel_embeddings=r)
    # The original divides by sqrt(d*f) rounded to float32 (its dtype-cast scale);
    # the prepared path uses the exact value: ~1e-7 apart.  A wrong slot would
    # move scores by O(0.1).
    torch.testing.assert_close(got, want, atol=1e-6, rtol=0)
    with pytest.raises(ValueError, match="2, 3, or 4"):
        with torch.inference_mode():
            fast(h, m, relative_pos=rpos.reshape(-1), rel_embeddings=r)


def test_qkv_is_always_fused_after_prepare():
    """Reference tests/test_fused_qkv.py:7-30."""

    from disentangled_flash._torch import TorchInferenceDisentangledSelfAttention
    from disentangled_flash.modeling import DebertaAttentionConfig

    config = DebertaAttentionConfig(
        hidden_size=64, num_attention_heads=1, attention_head_size=64, relative_attention=True,
        max_relative_positions=64, max_position_embeddings=64, position_buckets=32,
        share_att_key=True, pos_att_type=("c2p", "p2c"), norm_rel_ebd="none",
    )
    module = TorchInferenceDisentangledSelfAttention(config).eval()
    module.prepare_for_inference(torch.randn(config.position_buckets * 2, config.hidden_size))
    assert module.prepared.qkv_weight.shape == (192, 64)
    with torch.inference_mode():
        q, k, v = module._project_qkv(torch.randn(2, 8, 64))
    assert q.shape == k.shape == v.shape == (2, 8, 64)


def test_inference_guards_and_cache_invalidation():
    from disentangled_flash._torch import TorchInferenceDisentangledSelfAttention
    from disentangled_flash.modeling import DebertaAttentionConfig

    module = TorchInferenceDisentangledSelfAttention(DebertaAttentionConfig(hidden_size=64,
                                                                            num_attention_heads=2))
    with pytest.raises(RuntimeError, match="eval"):
        module.prepare_for_inference(torch.randn(512, 64))
    module.eval().prepare_for_inference(torch.randn(512, 64))
    with pytest.raises(RuntimeError, match="no_grad"):
        module(torch.randn(1, 4, 64), torch.ones(1, 4))
    assert module.prepared is not None
    module.load_state_dict(module.state_dict())
    assert module.prepared is None
    module.prepare_for_inference(torch.randn(512, 64))
    module.double()
    assert module.prepared is None
    module.prepare_for_inference(torch.randn(512, 64, dtype=torch.float64))
    module.train()
    assert module.prepared is None


def test_hip_module_validation_errors_on_cpu():
    from disentangled_flash.kernel import HipInferenceDisentangledSelfAttention, _require_2d_padding_mask
    from disentangled_flash.modeling import DebertaAttentionConfig

    config = DebertaAttentionConfig(hidden_size=64, num_attention_heads=2)
    with pytest.raises(ValueError, match="fp32_precision"):
        HipInferenceDisentangledSelfAttention(config, fp32_precision="tf32")
    with pytest.raises(ValueError, match="relative_mode"):
        HipInferenceDisentangledSelfAttention(config, relative_mode="dense")
    module = HipInferenceDisentangledSelfAttention(config).eval()
    module.prepare_for_inference(torch.randn(512, 64))
    with torch.inference_mode(), pytest.raises(RuntimeError, match="GPU"):
        module(torch.randn(1, 4, 64), torch.ones(1, 4))
    with pytest.raises(ValueError, match="prepared on a GPU"):
        module.prepare_shape(4, "cpu")
    with pytest.raises(ValueError, match="factorized"):
        _require_2d_padding_mask(torch.ones(1, 1, 4, 4), 1, 4)
    with pytest.raises(ValueError, match="does not match"):
        _require_2d_padding_mask(torch.ones(2, 4), 1, 4)
    from disentangled_flash.kernel import deberta_attention_rel

    qkv = torch.zeros(1, 4, 3 * 64, dtype=torch.float16)
    rows = torch.zeros(2, 7, 32, dtype=torch.float16)
    with pytest.raises(ValueError, match="key_splits"):
        deberta_attention_rel(qkv, rows, rows, torch.zeros(7, dtype=torch.int32),
                              torch.ones(1, 4, dtype=torch.uint8), 2, 32, 1.0, True, True,
                              False, key_splits=-1)


def test_table_op_checks_its_tensors_before_launching():
    """deberta_attention (the reference op's contract) rejects tensors whose shape,
    layout or dtype differ from what the kernel will address, on the host."""

    from disentangled_flash.kernel import deberta_attention

    b, h, length, d, s = 2, 3, 5, 32, 9
    q, k, v = (torch.zeros(b, h, length, d, dtype=torch.float16) for _ in range(3))
    c2p = torch.zeros(b, h, length, s, dtype=torch.float16)
    lut = torch.zeros(2 * length - 1, dtype=torch.int32)
    mask = torch.ones(b, length, dtype=torch.bool)

    def call(**over):
        args = dict(query=q, key=k, value=v, c2p=c2p, p2c=c2p, delta_to_local=lut,
                    attention_mask=mask, num_heads=h, sequence_length=length, active_slots=s,
                    score_scale_log2=1.0, has_c2p=True, has_p2c=True, is_bf16=False,
                    is_fp32=False, strict_fp32=True)
        args.update(over)
        return deberta_attention(*args.values())

    with pytest.raises(ValueError, match="c2p must be"):
        call(c2p=torch.zeros(b, h, length, s - 1, dtype=torch.float16))
    with pytest.raises(ValueError, match="p2c must be"):
        call(p2c=c2p.float())
    with pytest.raises(ValueError, match="key must be contiguous"):
        call(key=torch.zeros(b, h, d, length, dtype=torch.float16).transpose(-1, -2))
    with pytest.raises(ValueError, match="value must match"):
        call(value=torch.zeros(b, h, length + 1, d, dtype=torch.float16))
    with pytest.raises(ValueError, match="does not match num_heads"):
        call(num_heads=h + 1)
    with pytest.raises(TypeError, match="int32"):
        call(delta_to_local=lut.long())
    with pytest.raises(ValueError, match="2L-1"):
        call(delta_to_local=lut[:-1])
    with pytest.raises(ValueError, match="attention_mask shape"):
        call(attention_mask=torch.ones(b, length + 1, dtype=torch.bool))
    with pytest.raises(TypeError, match="not fp16"):
        call(query=q.double(), key=k.double(), value=v.double())


def _tiny_deberta(layers=2, conv=3):
    from transformers import DebertaV2Config, DebertaV2Model

    config = DebertaV2Config(
        vocab_size=100, hidden_size=64, num_hidden_layers=layers, num_attention_heads=2,
        intermediate_size=128, hidden_dropout_prob=0.0, attention_probs_dropout_prob=0.0,
        max_position_embeddings=64, type_vocab_size=0, relative_attention=True,
        position_buckets=16, max_relative_positions=-1, pos_att_type=["p2c", "c2p"],
        norm_rel_ebd="layer_norm", share_att_key=True, conv_kernel_size=conv,
        conv_act="gelu", position_biased_input=False,
    )
    torch.manual_seed(0)
    return DebertaV2Model(config).eval()


@pytest.mark.parametrize("backend", ["torch", "optimized"])
def test_encoder_torch_backend_matches_huggingface(backend):
    from disentangled_flash import DebertaV2InferenceEncoder, enable_deberta_inference

    model = _tiny_deberta().double()
    fast = enable_deberta_inference(copy.deepcopy(model), backend=backend,
                                    sequence_lengths=[24, 40])
    assert isinstance(fast.encoder, DebertaV2InferenceEncoder)
    assert set(fast.state_dict()) == set(model.state_dict())
    ids = torch.randint(1, 100, (3, 40))
    mask = (torch.arange(40)[None] < torch.tensor([[40], [23], [5]])).long()
    with torch.inference_mode():
        expected = model(input_ids=ids, attention_mask=mask).last_hidden_state
        fast.encoder.activate_shape(40)
        got = fast(input_ids=ids, attention_mask=mask).last_hidden_state
    torch.testing.assert_close(got, expected, atol=1e-9, rtol=0)


def test_encoder_api_errors():
    from disentangled_flash import enable_deberta_inference
    from disentangled_flash.deberta import resolve_backend

    assert resolve_backend("triton") == "hip" and resolve_backend("optimized") == "torch"
    with pytest.raises(ValueError, match="backend"):
        resolve_backend("cuda")
    model = _tiny_deberta(layers=1, conv=0)
    with pytest.raises(TypeError):
        enable_deberta_inference(torch.nn.Linear(2, 2))
    enable_deberta_inference(model, backend="torch", sequence_lengths=[16])
    with pytest.raises(TypeError, match="already"):
        enable_deberta_inference(model, backend="torch")
    encoder = model.encoder
    with pytest.raises(ValueError, match="not prepared"):
        encoder.activate_shape(32)
    h = torch.randn(2, 16, 64)
    with torch.inference_mode():
        with pytest.raises(ValueError, match=r"\[B, L\]"):
            encoder(h, torch.ones(2, 1, 16, 16))
        with pytest.raises(ValueError, match="active bucket"):
            encoder(torch.randn(2, 8, 64), torch.ones(2, 8))
        with pytest.raises(ValueError, match="output_attentions"):
            encoder(h, torch.ones(2, 16), output_attentions=True)
    with pytest.raises(RuntimeError, match="no_grad"):
        encoder(h, torch.ones(2, 16))
    trained = _tiny_deberta(layers=1, conv=0).train()
    with pytest.raises(RuntimeError, match="eval"):
        enable_deberta_inference(trained, backend="torch", sequence_lengths=[8])


def test_c_abi_library_exports_every_header_symbol():
    import ctypes

    from disentangled_flash import _lib

    path = _lib.library_path()
    if not path.exists():
        pytest.skip("libdflash.so not built (run python __graft_entry__.py)")
    header = (REPO / "include" / "dflash.h").read_text()
    declared = re.findall(r"DFLASH_API\s+[\w\s\*]+?\b(dflash_\w+)\s*\(", header)
    assert {"dflash_attention_fwd", "dflash_attention_rel_fwd", "dflash_error_string",
            "dflash_abi_version"} <= set(declared)
    lib = ctypes.CDLL(str(path))
    for name in declared:
        assert hasattr(lib, name), name
    loaded = _lib.load()
    assert loaded.dflash_abi_version() == _lib.ABI_VERSION
    assert b"success" == loaded.dflash_error_string(0)


def test_no_product_module_imports_the_oracle():
    package = REPO / "disentangled-flash_amd"
    for path in list(package.rglob("*.py")) + list(package.rglob("*.hip")):
        text = path.read_text()
        assert "oracle" not in re.findall(r"^\s*(?:from|import)\s+(\w+)", text, re.M), path


def test_fusable_output_block_rules():
    from torch import nn
    from transformers import DebertaV2Config
    from transformers.models.deberta_v2.modeling_deberta_v2 import DebertaV2SelfOutput

    from disentangled_flash.layers import fusable_output_block

    cfg = DebertaV2Config(hidden_size=64, intermediate_size=128, hidden_dropout_prob=0.0)
    block = DebertaV2SelfOutput(cfg)
    assert fusable_output_block(block)
    block.dense = nn.Linear(64, 64, bias=False)
    assert not fusable_output_block(block)
    other = DebertaV2SelfOutput(cfg)
    other.LayerNorm = nn.LayerNorm(64, elementwise_affine=False)
    assert not fusable_output_block(other)
    assert not fusable_output_block(nn.Linear(4, 4))


def test_fusable_conv_layer_rules_and_tap_decomposition():
    """The fused ConvLayer path's eligibility, and the tap split it relies on.

    The convolution output at position l is z_0[l-1] + z_1[l] + z_2[l+1] + bias
    with z = x . conv_taps(module)^T, the out-of-range taps dropped; checked
    against torch's own Conv1d on the CPU.
    """

    from torch.nn import functional as F
    from transformers import DebertaV2Config
    from transformers.models.deberta_v2.modeling_deberta_v2 import ConvLayer

    from disentangled_flash.layers import conv_taps, fusable_conv_layer

    def make(**kw):
        cfg = DebertaV2Config(hidden_size=32, conv_kernel_size=kw.get("k", 3),
                              conv_act=kw.get("act", "gelu"), conv_groups=kw.get("groups", 1),
                              hidden_dropout_prob=0.0)
        return ConvLayer(cfg).eval()

    assert fusable_conv_layer(make())
    assert fusable_conv_layer(make(act="tanh")) and fusable_conv_layer(make(act="relu"))
    assert not fusable_conv_layer(make(act="sigmoid"))
    assert not fusable_conv_layer(make(k=5))
    assert not fusable_conv_layer(make(groups=2))
    assert not fusable_conv_layer(None)

    module = make()
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(2, 7, 32, generator=gen, dtype=torch.float64)
    conv = module.conv.double()
    expected = F.conv1d(x.transpose(1, 2), conv.weight, conv.bias, padding=1).transpose(1, 2)
    z = x.reshape(14, 32) @ conv_taps(module).double().t()
    z = z.reshape(2, 7, 3, 32)
    got = z[:, :, 1] + conv.bias
    got[:, 1:] += z[:, :-1, 0]
    got[:, :-1] += z[:, 1:, 2]
    assert torch.allclose(got, expected, atol=1e-12)


def test_bench_refuses_more_than_one_gpu():
    """The benchmark measures the single-GPU path; --gpus N > 1 exits with a message."""

    import subprocess
    import sys

    result = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"],
                            capture_output=True, text=True, timeout=300)
    assert result.returncode == 2
    assert "single-GPU" in result.stderr
