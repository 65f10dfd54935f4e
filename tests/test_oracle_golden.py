"""Pin the Tier-A torch oracle against fixtures written by the real reference.

The oracle repeats the reference's torch op sequence, so on this CPU it must
reproduce the fixtures bit for bit (tests/golden/make_golden.py wrote them).
"""

import numpy as np
import pytest
import torch

from oracle import torch_ref as T


class ListCache:
    def __init__(self, ks, vs):
        self.key_cache = list(ks)
        self.value_cache = list(vs)


def _t(a):
    return torch.from_numpy(np.asarray(a))


def _cache(g):
    return ListCache([_t(k).clone() for k in g["k_in"]], [_t(v).clone() for v in g["v_in"]])


def _stack(c, attr):
    return torch.stack(getattr(c, attr)).numpy()


def test_e8_nearest_point_matches_reference(golden):
    g = golden("e8_nearest")
    p = T.e8_nearest_point(_t(g["x"]).clone()).numpy()
    assert np.array_equal(p, g["p"])


@pytest.mark.parametrize("levels", [2, 4, 8, 16])
def test_e8_quantize_perhead_matches_reference(golden, levels):
    g = golden("e8_perhead")
    q = T.e8_quantize_perhead(_t(g["x"]).clone(), levels=levels).numpy()
    assert np.array_equal(q, g[f"q{levels}"])


def test_rope_far_positions_match_reference(golden):
    g = golden("rope_far")
    x = _t(g["x"])
    assert np.array_equal(T.inverse_rope(x, seq_offset=131008, base=500000.0).numpy(), g["inv"])
    assert np.array_equal(T.forward_rope(x, seq_offset=131008, base=500000.0).numpy(), g["fwd"])
    sc = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
          "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}
    assert np.array_equal(
        T.inverse_rope(x, seq_offset=40000, base=500000.0, rope_scaling=sc).numpy(), g["inv_scaled"])


@pytest.mark.parametrize("tag", ["b1e4", "b5e5"])
def test_quant_only_matches_reference(golden, tag):
    g = golden(f"quant_only_{tag}")
    base = float(g["base"])
    c = _cache(g)
    T.quant_only_compress(c, 8, 4, rope_base=base)
    assert np.array_equal(_stack(c, "key_cache"), g["k_k3v2"])
    assert np.array_equal(_stack(c, "value_cache"), g["v_k3v2"])
    assert np.all(g["mask"] == 1.0)
    c = _cache(g)
    T.quant_only_compress(c, 8, 8, rope_base=base)
    assert np.array_equal(_stack(c, "key_cache"), g["k_k3v3"])
    assert np.array_equal(_stack(c, "value_cache"), g["v_k3v3"])


def test_quant_only_d256_and_bf16_match_reference(golden):
    g = golden("quant_only_d256")
    c = _cache(g)
    T.quant_only_compress(c, 4, 4, rope_base=10000.0)
    assert np.array_equal(_stack(c, "key_cache"), g["k_out"])
    assert np.array_equal(_stack(c, "value_cache"), g["v_out"])
    g = golden("quant_only_bf16")
    c = ListCache([_t(k).to(torch.bfloat16) for k in g["k_in"]],
                  [_t(v).to(torch.bfloat16) for v in g["v_in"]])
    T.quant_only_compress(c, 8, 4, rope_base=500000.0)
    assert np.array_equal(_stack(c, "key_cache"), g["k_out"])
    assert np.array_equal(_stack(c, "value_cache"), g["v_out"])


def test_keykey_scorer_and_mask_eviction_match_reference(golden):
    g = golden("evict_mask_b4")
    imp = T.score_keykey(_t(g["k_in"][0]).float(), 32)
    assert np.array_equal(imp.numpy(), g["importance"])
    c = _cache(g)
    _, mask = T.evict_mask_compress(c, 8, 4, 0.25, sliding_window=32, obs_window=32,
                                    rope_base=10000.0)
    assert np.array_equal(mask.numpy(), g["mask"])
    assert np.array_equal(_stack(c, "key_cache"), g["k_out"])
    assert np.array_equal(_stack(c, "value_cache"), g["v_out"])


def test_boundary_protected_eviction_matches_reference(golden):
    g = golden("evict_mask_boundary")
    c = _cache(g)
    skip = T.boundary_skip_layers(len(c.key_cache), 2)
    _, mask = T.evict_mask_compress(c, 4, 4, 0.6, sliding_window=16, rope_base=10000.0,
                                    skip_layers=skip)
    assert np.array_equal(mask.numpy(), g["mask"])
    assert np.array_equal(_stack(c, "key_cache"), g["k_out"])
    assert np.array_equal(_stack(c, "value_cache"), g["v_out"])


def test_soft_eviction_matches_reference(golden):
    g = golden("evict_soft")
    imp = T.score_keykey(_t(g["k_in"][0]).float(), 32)
    assert np.array_equal(imp.numpy(), g["importance"])
    c = _cache(g)
    skip = T.boundary_skip_layers(len(c.key_cache), 1)
    _, mask = T.evict_soft_compress(c, 8, 4, 0.5, sliding_window=16, rope_base=10000.0,
                                    skip_layers=skip)
    assert np.array_equal(mask.numpy(), g["mask"])
    assert np.array_equal(_stack(c, "key_cache"), g["k_out"])
    assert np.array_equal(_stack(c, "value_cache"), g["v_out"])


@pytest.mark.parametrize("rate", [25, 60])
def test_truncation_matches_reference(golden, rate):
    g = golden(f"evict_truncate_r{rate}")
    c = _cache(g)
    _, n_kept = T.evict_truncate_compress(c, 8, 4, rate / 100, sliding_window=32,
                                          rope_base=10000.0)
    assert n_kept == int(g["n_kept"])
    assert np.array_equal(_stack(c, "key_cache"), g["k_out"])
    assert np.array_equal(_stack(c, "value_cache"), g["v_out"])


def test_real_scorer_matches_transformers_eager(golden):
    g = golden("real_scorer")
    q = [_t(x) for x in g["q"]]
    k = [_t(x) for x in g["k"]]
    imp = T.score_real_from_qk(q, k, float(g["scaling"]))
    assert np.allclose(imp.numpy(), g["importance"], rtol=0, atol=1e-6)
    assert np.array_equal(imp.numpy(), g["importance"])


@pytest.mark.parametrize("name", ["real_scorer_mistral", "real_scorer_gemma2"])
def test_real_scorer_window_and_softcap_match_transformers_eager(golden, name):
    # the reference's _score_importance_real on a tiny Mistral (sliding window
    # 48 < seq 160) and a tiny Gemma-2 (soft-cap 50, a sliding layer of 40 and a
    # full layer), fp16: the oracle's eager restatement gives the same importance
    g = golden(name)
    q = [_t(x) for x in g["q"]]
    k = [_t(x) for x in g["k"]]
    win = [int(w) or None for w in g["window"]]
    cap = [float(c) or None for c in g["softcap"]]
    assert len(set(float(x) for x in g["scaling"])) == 1
    imp = T.score_real_from_qk(q, k, float(g["scaling"][0]), windows=win, softcaps=cap)
    assert np.array_equal(imp.numpy(), g["importance"])
    # the window and the cap change the result: without them it differs
    plain = T.score_real_from_qk(q, k, float(g["scaling"][0]))
    assert not np.allclose(plain.numpy(), g["importance"], rtol=0, atol=1e-4)
    # the window's edge is pinned: one key more (j >= i - W, a window of W + 1)
    # does not reproduce the fixture
    if any(w is not None for w in win):
        wider = [w + 1 if w is not None else None for w in win]
        off = T.score_real_from_qk(q, k, float(g["scaling"][0]), windows=wider, softcaps=cap)
        assert not np.array_equal(off.numpy(), g["importance"])
    # and so is the cap's value
    if any(c is not None for c in cap):
        other = [c * 1.01 if c is not None else None for c in cap]
        off = T.score_real_from_qk(q, k, float(g["scaling"][0]), windows=win, softcaps=other)
        assert not np.array_equal(off.numpy(), g["importance"])
