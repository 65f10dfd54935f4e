"""Host logic of the nexusquant_evict hook's two modes (no GPU): the
reference's per-layer compression (default) and the full-cache mode.  The
GPU compressor is replaced by a recorder; the model is a tiny Llama on the CPU."""

import pytest
import torch

import nexusquant_amd as nq
from nexusquant_amd.pipeline import NexusQuantEvict, get_layer_kv, num_layers, set_layer_kv


@pytest.fixture
def calls(monkeypatch):
    rec = []

    def fake_compress(self, cache, model=None, input_ids=None):
        n = num_layers(cache)
        rec.append([get_layer_kv(cache, i)[0].shape[-2] for i in range(n)])
        for i in range(n):
            k, v = get_layer_kv(cache, i)
            set_layer_kv(cache, i, torch.full_like(k, float(len(rec) * 100 + i)), v)
        k0 = get_layer_kv(cache, 0)[0]
        return cache, torch.ones(k0.shape[0], k0.shape[2])

    monkeypatch.setattr(NexusQuantEvict, "compress", fake_compress)
    return rec


def _tiny(layers=4):
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(0)
    cfg = LlamaConfig(vocab_size=64, hidden_size=64, intermediate_size=128, num_hidden_layers=layers,
                      num_attention_heads=2, num_key_value_heads=1, max_position_embeddings=256)
    cfg._attn_implementation = "eager"
    return LlamaForCausalLM(cfg).eval()


def _ids(n, seed=1):
    return torch.randint(0, 64, (1, n), generator=torch.Generator().manual_seed(seed))


def test_default_mode_compresses_each_layer_alone(calls):
    from transformers import DynamicCache
    model = _tiny(4)
    with torch.no_grad():
        cache = DynamicCache()
        with nq.nexusquant_evict(model, quality="high", verbose=False):
            model(_ids(40), past_key_values=cache, use_cache=True)
            model(_ids(1), past_key_values=cache, use_cache=True)     # decode step: no compression
    assert calls == [[40], [40], [40], [40]]
    assert "forward" not in model.__dict__


def test_full_cache_mode_compresses_every_layer_once_after_the_forward(calls):
    from transformers import DynamicCache
    model = _tiny(4)
    ids = _ids(40)
    with torch.no_grad():
        plain = model(ids, use_cache=False).logits
        cache = DynamicCache()
        with nq.nexusquant_evict(model, quality="high", verbose=False, compat_reference_hook=False):
            out = model(ids, past_key_values=cache, use_cache=True)
            assert calls == [[40, 40, 40, 40]]
            # the prefill attention saw the uncompressed keys and values
            assert torch.equal(out.logits, plain)
            for i in range(4):
                assert torch.all(cache.layers[i].keys == 100 + i)
            model(_ids(1, seed=2), past_key_values=cache, use_cache=True)
        assert calls == [[40, 40, 40, 40]]
    for i in range(4):
        assert cache.layers[i].keys.shape[-2] == 41
        assert torch.all(cache.layers[i].keys[..., :40, :] == 100 + i)
    assert "forward" not in model.__dict__


def test_full_cache_mode_compresses_before_the_next_update_or_at_exit(calls):
    # the inner decoder is called directly, so only the update hook and the
    # context exit can trigger the compression
    from transformers import DynamicCache
    model = _tiny(3)
    with torch.no_grad():
        cache = DynamicCache()
        with nq.nexusquant_evict(model, quality="high", verbose=False, compat_reference_hook=False):
            model.model(_ids(30), past_key_values=cache, use_cache=True)
            assert calls == []
            model.model(_ids(1, seed=3), past_key_values=cache, use_cache=True)
            assert calls == [[30, 30, 30]]
            assert cache.layers[0].keys.shape[-2] == 31
            assert torch.all(cache.layers[2].keys[..., :30, :] == 102)
            cache2 = DynamicCache()
            model.model(_ids(20, seed=4), past_key_values=cache2, use_cache=True)
            assert len(calls) == 1
        assert calls == [[30, 30, 30], [20, 20, 20]]
        assert torch.all(cache2.layers[1].keys == 201)


def test_full_cache_mode_restores_an_existing_forward_override(calls):
    model = _tiny(2)
    marker = []

    def own_forward(*a, **k):
        marker.append(1)
        return type(model).forward(model, *a, **k)

    model.forward = own_forward
    with torch.no_grad():
        with nq.nexusquant_evict(model, quality="high", verbose=False, compat_reference_hook=False):
            model(_ids(24), use_cache=True)
    assert marker == [1] and calls == [[24, 24]]
    assert model.__dict__["forward"] is own_forward
