"""GPU parity of the remaining eviction options against the Tier-A oracle:
eviction_rate="auto" (pipeline.py:838-861), protect_boundary="auto" (:863-893),
adaptive_context (:1093-1100), distance_graduated (:935-941), global_only
sliding-window detection (:670-710), min_context_for_compression
(:1126-1127), the graduated bit profile (:740-754); and the reference's own
API properties (tests/test_core.py:283-418 of the reference) on this build."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import torch_ref as T

from gpu_helpers import assert_close_rows, keep_sets_match

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


class Cache:
    def __init__(self, ks, vs):
        self.key_cache, self.value_cache = list(ks), list(vs)


def _kv(n_layers, b, h, s, d, seed, scale=None):
    """Keys: N(0,1) with outlier channels and a sink, RoPE base 1e4; values N(0, 0.25)."""
    g = torch.Generator().manual_seed(seed)
    ks, vs = [], []
    for li in range(n_layers):
        kp = torch.randn(b, h, s, d, generator=g)
        kp[..., ::32] *= 8
        kp[:, :, 0, :] *= 4
        kp *= 1.0 if scale is None else scale[li]
        ks.append(T.forward_rope(kp, base=10000.0).half())
        vs.append((torch.randn(b, h, s, d, generator=g) * 0.5).half())
    return ks, vs


GEMMA2_LIKE = SimpleNamespace(num_hidden_layers=6, layer_types=["sliding_attention", "full_attention"] * 3)

VARIANTS = {
    "auto_rate": (dict(eviction_rate="auto"), {}),
    "auto_boundary_bright": (dict(eviction_rate=0.5, protect_boundary="auto"), dict(scale=[3, 1, 1, 1, 1, 3])),
    "auto_boundary_flat": (dict(eviction_rate=0.5, protect_boundary="auto"), {}),
    "adaptive_200": (dict(eviction_rate=0.6, adaptive_context=True), dict(s=200)),
    "adaptive_400": (dict(eviction_rate=0.6, adaptive_context=True), dict(s=400)),
    "adaptive_800": (dict(eviction_rate=0.6, adaptive_context=True), dict(s=800)),
    "distance_graduated": (dict(eviction_rate=0.6, distance_graduated=True), {}),
    "global_only": (dict(eviction_rate=0.6, compress_layers="global_only"), dict(config=GEMMA2_LIKE)),
    "min_context": (dict(eviction_rate=0.6, min_context_for_compression=1000), dict(s=500)),
    "graduated_protected": (dict(key_bits=3, value_bits=2, eviction_rate=0.35, layer_bit_profile="graduated",
                                 protected_layers={2}, protect_boundary=1), {}),
}


@pytest.mark.parametrize("name", sorted(VARIANTS))
def test_eviction_option_matches_oracle(name):
    import nexusquant_amd as nq
    kw, shape = VARIANTS[name]
    print(f"[gpu] eviction option {name}", flush=True)
    n, b, h, s, d = 6, 2, 2, shape.get("s", 600), 128
    ks, vs = _kv(n, b, h, s, d, seed=len(name) * 7 + s, scale=shape.get("scale"))
    comp = nq.NexusQuantEvict(rope_base=10000.0, sliding_window=32, obs_window=32, **kw)
    cfg = shape.get("config")
    swa = None
    if cfg is not None:
        comp.set_model_config(cfg)
        swa = T.swa_layers_from_config(cfg)
        assert comp._swa_layer_indices == swa and swa == {0, 2, 4}
    c = Cache([k.to(DEV) for k in ks], [v.to(DEV) for v in vs])
    before = [k for k in c.key_cache]
    _, mask = comp.compress(c)
    ref = Cache([k.clone() for k in ks], [v.clone() for v in vs])
    _, mask_ref, rate_ref, skip_ref = T.evict_compress(
        ref, comp.key_levels, comp.value_levels, kw["eviction_rate"], sliding_window=32, obs_window=32,
        rope_base=10000.0, protected_layers=kw.get("protected_layers", ()),
        protect_boundary=kw.get("protect_boundary", 0),
        min_context_for_compression=kw.get("min_context_for_compression", 0),
        adaptive_context=kw.get("adaptive_context", False), distance_graduated=kw.get("distance_graduated", False),
        swa_layers=swa, layer_bit_profile=kw.get("layer_bit_profile", "uniform"))
    skip = comp._skip_layers(c, n)
    assert skip == skip_ref
    if name == "auto_boundary_bright":
        assert skip == {0, 1, 4, 5}
    if name == "min_context":
        assert torch.all(mask == 1) and all(a is bb for a, bb in zip(before, c.key_cache))
        return
    m, mr = mask.cpu().numpy().astype(bool), mask_ref.numpy().astype(bool)
    assert int(m.sum()) == int(mr.sum())  # same resolved rate
    if not np.array_equal(m, mr):
        score_layer = 1 if swa else 0
        imp = T.score_keykey(ks[score_layer].float(), 32)
        if kw.get("distance_graduated"):
            prefix = s - 32
            ramp = torch.linspace(0.0, 1.0, prefix - 1)
            imp[:, 1:prefix] += ramp * imp[:, 1:prefix].max() * 0.25
        assert keep_sets_match(imp.numpy(), imp.numpy(), m, mr)
    for li in range(n):
        assert c.key_cache[li].dtype == torch.float16
        if li in skip:   # fp16 passthrough with evicted rows zeroed: exact
            assert torch.equal(c.key_cache[li].cpu(), ref.key_cache[li])
            assert torch.equal(c.value_cache[li].cpu(), ref.value_cache[li])
        else:
            assert_close_rows(c.key_cache[li], ref.key_cache[li].numpy())
            assert_close_rows(c.value_cache[li], ref.value_cache[li].numpy())


def test_auto_rate_equals_the_entropy_rule_on_the_same_importance():
    import nexusquant_amd as nq
    comp = nq.NexusQuantEvict(eviction_rate="auto")
    for seed in range(4):
        imp = torch.rand(1, 3000, generator=torch.Generator().manual_seed(seed)) ** (seed + 1)
        got = comp._resolve_rate(imp.to(DEV), 3000)
        assert got == pytest.approx(T.auto_eviction_rate(imp, 3000), abs=1e-6)


# ---- the reference's API properties (tests/test_core.py:283-418), on this build ----

def _fake(b=1, h=4, seq=64, d=128, n_layers=2, seed=0):
    g = torch.Generator().manual_seed(seed)
    return Cache([torch.randn(b, h, seq, d, generator=g).half().to(DEV) for _ in range(n_layers)],
                 [torch.randn(b, h, seq, d, generator=g).half().to(DEV) for _ in range(n_layers)])


def test_reference_api_properties_mask_path():
    import nexusquant_amd as nq
    out = nq.NexusQuantEvict(head_dim=128, eviction_rate=0.5, sliding_window=8).compress(_fake())
    assert isinstance(out, tuple) and len(out) == 2 and out[1].shape == (1, 64)
    _, mask = nq.NexusQuantEvict(eviction_rate=0.8, sliding_window=4).compress(_fake(seq=50))
    assert mask[0, 0].item() == 1.0
    _, mask = nq.NexusQuantEvict(eviction_rate=0.9, sliding_window=8).compress(_fake(seq=60))
    assert mask[0, -8:].sum().item() == 8.0
    _, mask = nq.NexusQuantEvict(eviction_rate=0.6, sliding_window=10).compress(_fake(seq=200))
    assert 10 < mask[0].sum().item() < 200 * (1 - 0.6 + 0.15)
    c = _fake(n_layers=2)
    nq.NexusQuantEvict(eviction_rate=0.5).compress(c)
    assert c.key_cache[0].shape == (1, 4, 64, 128) and c.value_cache[0].shape == (1, 4, 64, 128)
    c = _fake(n_layers=2)
    nq.NexusQuantEvict(eviction_rate=0.5, protected_layers={0}).compress(c)
    assert c.key_cache[0].dtype == torch.float16
    _, mask = nq.NexusQuantEvict(eviction_rate=0.8, min_context_for_compression=200).compress(_fake(seq=50))
    assert mask.sum().item() == mask.numel()
    _, mask = nq.NexusQuantEvict(eviction_rate=0.8, sliding_window=4, adaptive_context=True).compress(_fake(seq=100))
    assert mask.sum().item() == mask.numel()
    _, mask = nq.NexusQuantEvict(eviction_rate=0.6, sliding_window=8, soft_eviction=True).compress(_fake(seq=64))
    assert mask.sum().item() == mask.numel()


def test_reference_api_properties_truncate_path():
    import nexusquant_amd as nq
    c = _fake(seq=64)
    out = nq.NexusQuantEvictTruncate(head_dim=128, eviction_rate=0.5, sliding_window=8).compress(c)
    assert isinstance(out, tuple) and len(out) == 2 and isinstance(out[1], int)
    assert c.key_cache[0].shape[2] < 64
    _, next_pos = nq.NexusQuantEvictTruncate(eviction_rate=0.5, sliding_window=10).compress(_fake(seq=100))
    assert 10 < next_pos < 100
