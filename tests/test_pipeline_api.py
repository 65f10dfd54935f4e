"""Constructor / argument behaviour of the eviction API, mirroring the reference's
tests/test_core.py:214-266 (no GPU needed), plus the keep-mask arithmetic."""

import pytest
import torch

import nexusquant_amd as nq
from nexusquant_amd.ops import keep_plan
from oracle import torch_ref as T


def test_evict_init_defaults():
    c = nq.NexusQuantEvict()
    assert c.head_dim == 128 and c.eviction_rate == 0.6
    assert c.key_bits == 2 and c.value_bits == 2
    assert c.soft_eviction is False and c.adaptive_context is False


def test_evict_init_auto_params():
    c = nq.NexusQuantEvict(eviction_rate="auto", protect_boundary="auto")
    assert c.eviction_rate == "auto" and c.protect_boundary == "auto"


@pytest.mark.parametrize("kw", [{"eviction_rate": "bad_string"}, {"scorer": "unknown"},
                                {"protect_boundary": "maybe"}])
def test_evict_invalid_arguments_raise(kw):
    with pytest.raises(ValueError):
        nq.NexusQuantEvict(**kw)


def test_evict_asymmetric_bits():
    c = nq.NexusQuantEvict(key_bits=3, value_bits=2)
    assert (c.key_bits, c.value_bits, c.key_levels, c.value_levels) == (3, 2, 8, 4)


def test_graduated_profile_levels():
    c = nq.NexusQuantEvict(key_bits=3, value_bits=2, layer_bit_profile="graduated")
    assert c._resolve_layer_levels(0, 32) == (8, 8)
    assert c._resolve_layer_levels(16, 32) == (8, 4)
    assert c._resolve_layer_levels(31, 32) == (8, 8)


@pytest.mark.parametrize("seq,rate,sw", [(8192, 0.25, 32), (8192, 0.35, 32), (16384, 0.6, 32),
                                         (16384, 0.8, 32), (64, 0.5, 8), (50, 0.8, 4), (20, 0.6, 32),
                                         (33, 0.0, 32), (200, 0.6, 10)])
def test_keep_plan_matches_reference_counts(seq, rate, sw):
    prefix, k = keep_plan(seq, rate, sw)
    g = torch.Generator().manual_seed(seq)
    imp = torch.rand(1, seq, generator=g)
    keep = T.build_keep_mask(imp, seq, rate, sw)
    window = set(range(max(0, seq - sw), seq)) | {0}
    assert int(keep.sum()) == len(window) + k


def test_survey_keep_counts():
    # the kept counts the configs evict down to (BOS + top-k + window)
    def kept(seq, rate):
        prefix, k = keep_plan(seq, rate, 32)
        return 1 + k + min(32, seq)
    assert kept(8192, 0.25) == 6153
    assert kept(8192, 0.35) == 5337
    assert kept(16384, 0.60) == 6573
    assert kept(16384, 0.80) == 3303


def test_truncate_batch_gt1_error_message_matches_reference():
    class Cache:
        key_cache = [torch.zeros(2, 1, 4, 128)]
        value_cache = [torch.zeros(2, 1, 4, 128)]
    with pytest.raises(ValueError, match="does not support batch_size > 1"):
        nq.NexusQuantEvictTruncate().compress(Cache())


def test_merge_eviction_needs_the_device_path():
    # merge eviction is built; like every path it refuses host tensors
    from nexusquant_amd._lib import NexusQuantError

    class Cache:
        key_cache = [torch.zeros(1, 1, 4, 128)]
        value_cache = [torch.zeros(1, 1, 4, 128)]
    comp = nq.NexusQuantEvict(merge_eviction=True)
    assert comp.merge_eviction
    with pytest.raises(NexusQuantError):
        comp.compress(Cache())


def test_presets_match_reference_table():
    from nexusquant_amd.huggingface import _EVICT_PRESETS
    assert _EVICT_PRESETS["high"] == {"eviction_rate": 0.35, "bits": 2, "key_bits": 3}
    assert _EVICT_PRESETS["balanced"] == {"eviction_rate": 0.60, "bits": 2}
    assert _EVICT_PRESETS["max"] == {"eviction_rate": 0.80, "bits": 2}
    assert _EVICT_PRESETS["asym"] == {"eviction_rate": 0.60, "bits": 2, "key_bits": 3}


def test_model_config_detection_reads_transformers5_rope_parameters():
    from transformers import LlamaConfig
    from nexusquant_amd.huggingface import _detect_model_config

    class M:
        config = LlamaConfig(rope_theta=500000.0, num_key_value_heads=8, hidden_size=1024,
                             num_attention_heads=8, num_hidden_layers=2)
    mc = _detect_model_config(M())
    assert mc["rope_base"] == 500000.0 and mc["head_dim"] == 128 and mc["num_layers"] == 2
