"""Pin the Tier-A eviction options (oracle/torch_ref.py) without a GPU: the
reference's own properties (tests/test_core.py:283-418 of the reference) and
closed forms of the rate, boundary and sliding-window-layer rules
(pipeline.py:670-710, 838-893, 1093-1100, 1126-1127)."""

import math
from types import SimpleNamespace

import pytest
import torch

from oracle import torch_ref as T


class Cache:
    def __init__(self, ks, vs):
        self.key_cache, self.value_cache = list(ks), list(vs)


def _cache(n_layers=2, b=1, h=4, s=64, d=128, seed=0, scale=None):
    g = torch.Generator().manual_seed(seed)
    ks, vs = [], []
    for li in range(n_layers):
        f = 1.0 if scale is None else scale[li]
        ks.append((torch.randn(b, h, s, d, generator=g) * f).half())
        vs.append((torch.randn(b, h, s, d, generator=g) * 0.5).half())
    return Cache(ks, vs)


def test_reference_properties_of_the_mask_path():
    # test_core.py:283-330: (cache, mask) with BOS and the sliding window kept,
    # about (1 - rate) of the prefix kept, shapes unchanged
    c = _cache(s=200)
    _, mask, rate, _ = T.evict_compress(c, 4, 4, 0.6, sliding_window=10)
    assert mask.shape == (1, 200) and mask[0, 0] == 1 and mask[0, -10:].sum() == 10
    assert 10 < mask.sum() < 200 * (1 - 0.6 + 0.15)
    assert c.key_cache[0].shape == (1, 4, 200, 128) and c.key_cache[0].dtype == torch.float16


def test_min_context_passes_short_prefix_through():
    # test_core.py:372-383: all-ones mask, the cache not touched
    c = _cache(s=50)
    before = [k.clone() for k in c.key_cache]
    _, mask, _, _ = T.evict_compress(c, 4, 4, 0.8, min_context_for_compression=200)
    assert mask.sum() == mask.numel()
    assert all(torch.equal(a, b) for a, b in zip(before, c.key_cache))


def test_adaptive_context_rates():
    # test_core.py:386-396 (seq < 256 keeps everything) and pipeline.py:1093-1100
    c = _cache(s=100)
    _, mask, rate, _ = T.evict_compress(c, 4, 4, 0.8, sliding_window=4, adaptive_context=True)
    assert rate == 0.0 and mask.sum() == mask.numel()
    assert T.adaptive_context_rate(0.8, 255) == 0.0
    assert T.adaptive_context_rate(0.8, 256) == 0.4 and T.adaptive_context_rate(0.8, 511) == 0.4
    assert T.adaptive_context_rate(0.8, 512) == pytest.approx(0.6) and T.adaptive_context_rate(0.8, 1023) == 0.8 * 0.75
    assert T.adaptive_context_rate(0.8, 1024) == 0.8


def test_auto_rate_closed_form():
    # uniform importance: normalised entropy ~1 -> 0.7 - 0.5 = 0.2; one spike -> 0.7
    s = 1000
    assert T.auto_eviction_rate(torch.ones(1, s), s) == pytest.approx(0.2, abs=1e-5)
    spike = torch.zeros(1, s)
    spike[0, 3] = 1.0
    assert T.auto_eviction_rate(spike, s) == pytest.approx(0.7, abs=1e-5)
    # half the mass on 10 tokens: entropy in between, clamped to [0.1, 0.7]
    imp = torch.ones(1, s)
    imp[0, :10] = 99.0
    p = imp[0] / imp[0].sum()
    ent = float(-(p * p.log()).sum())
    assert T.auto_eviction_rate(imp, s) == pytest.approx(max(0.1, min(0.7, 0.7 - 0.5 * ent / math.log(s))), abs=1e-5)


def test_auto_boundary_probe():
    assert T.auto_detect_boundary(_cache(n_layers=5, scale=[5, 1, 1, 1, 5])) == 0   # fewer than 6 layers
    assert T.auto_detect_boundary(_cache(n_layers=6, scale=[1] * 6)) == 0
    assert T.auto_detect_boundary(_cache(n_layers=6, scale=[3, 1, 1, 1, 1, 3])) == 2
    assert T.auto_detect_boundary(_cache(n_layers=8, scale=[1.5, 1, 1, 1, 1, 1, 1, 1.5])) == 0


def test_sliding_window_layers_from_config():
    assert T.swa_layers_from_config(SimpleNamespace(num_hidden_layers=12, sliding_window_pattern=6)) == \
        {i for i in range(12) if (i + 1) % 6}
    cfg = SimpleNamespace(num_hidden_layers=4, layer_types=["sliding_attention", "full_attention"] * 2)
    assert T.swa_layers_from_config(cfg) == {0, 2}
    assert T.swa_layers_from_config(SimpleNamespace(text_config=cfg)) == {0, 2}
    assert T.swa_layers_from_config(SimpleNamespace(num_hidden_layers=10, num_kv_shared_layers=3)) == {7, 8, 9}
    assert T.swa_layers_from_config(SimpleNamespace(num_hidden_layers=4)) == set()


def test_global_only_scores_first_global_layer_and_skips_sliding_layers():
    c = _cache(n_layers=4, s=300)
    ref = _cache(n_layers=4, s=300)
    imp = T.score_keykey(c.key_cache[1].float(), 32)
    _, mask, _, skip = T.evict_compress(c, 4, 4, 0.5, swa_layers={0, 2})
    assert skip == {0, 2}
    assert torch.equal(mask.bool(), T.build_keep_mask(imp, 300, 0.5, 32))
    # sliding layers keep their rows (masked, fp16), global layers are quantized
    m4 = mask[:, None, :, None].half()
    assert torch.equal(c.key_cache[0], ref.key_cache[0] * m4)
    assert not torch.equal(c.key_cache[1], ref.key_cache[1] * m4)


def test_distance_ramp_prefers_late_tokens():
    s = 400
    imp = torch.full((1, s), 0.5)
    keep_plain = T.build_keep_mask(imp, s, 0.5, 32)
    keep_ramp = T.build_keep_mask(imp, s, 0.5, 32, distance_graduated=True)
    prefix = s - 32
    n_keep = int(prefix * 0.5)
    # flat scores: ties keep any n_keep prefix tokens; with the ramp exactly the latest ones
    assert int(keep_plain[0, 1:prefix].sum()) == n_keep == int(keep_ramp[0, 1:prefix].sum())
    assert keep_ramp[0, prefix - n_keep:prefix].all() and not keep_ramp[0, 1:prefix - n_keep].any()
