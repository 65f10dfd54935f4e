"""Pin the merge-eviction oracle (CPU).

Tier A (oracle/torch_ref.py merge_*) must reproduce the reference's own merge
eviction (tests/golden/evict_merge.npz, written by NexusQuantEvict with
merge_eviction=True) bit for bit.  The head-mean reduction order that the
device centroids restate (runs of 16 heads summed from zero, runs added in
order) is pinned against torch's CPU reduction here.
"""

import numpy as np
import pytest
import torch

from oracle import torch_ref as T


class Cache:
    def __init__(self, ks, vs):
        self.key_cache, self.value_cache = list(ks), list(vs)


def test_tier_a_reproduces_reference_merge(golden):
    g = golden("evict_merge")
    vs = [torch.from_numpy(v) for v in g["v_in"]]
    keep = torch.from_numpy(g["keep"])
    imp = torch.from_numpy(g["importance"])
    for bi in range(keep.shape[0]):
        assert torch.equal(T.merge_centroids(vs, bi), torch.from_numpy(g["centroids"][bi]))
        ev, kp, nearest, _ = T.merge_survivors(T.merge_centroids(vs, bi), keep[bi])
        assert np.array_equal(kp[nearest].numpy(), g["survivor"][bi][ev.numpy()])
    merged = T.merge_eviction_values(vs, keep, imp)
    for li, m in enumerate(merged):
        assert np.array_equal(m.numpy(), g["v_merged"][li])
    c = Cache([torch.from_numpy(k) for k in g["k_in"]], vs)
    _, mask = T.evict_merge_compress(c, 8, 4, 0.5, sliding_window=8, importance=imp, skip_layers={0, 2})
    assert np.array_equal(mask.numpy(), g["mask"])
    for li in range(3):
        assert np.array_equal(c.key_cache[li].numpy(), g["k_out"][li])
        assert np.array_equal(c.value_cache[li].numpy(), g["v_out"][li])


@pytest.mark.parametrize("h", [1, 3, 8, 16, 17, 24, 40, 100])
def test_head_mean_order_is_runs_of_16(h):
    rng = np.random.default_rng(h)
    x = (rng.standard_normal((h, 50, 64)) * 3).astype(np.float32)
    want = torch.from_numpy(x).mean(dim=0).numpy()
    total = None
    for h0 in range(0, h, 16):
        run = np.zeros((50, 64), np.float32)
        for i in range(h0, min(h0 + 16, h)):
            run = (run + x[i]).astype(np.float32)
        total = run if total is None else (total + run).astype(np.float32)
    got = (total / np.float32(h)).astype(np.float32)
    assert np.array_equal(got, want)
    # a plain left-to-right sum differs for some h > 16 (the order is not arbitrary)
    if h in (24, 40, 100):
        seq = np.zeros((50, 64), np.float32)
        for i in range(h):
            seq = (seq + x[i]).astype(np.float32)
        assert not np.array_equal((seq / np.float32(h)).astype(np.float32), want)


def test_explicit_survivors_reproduce_the_argmax_path(golden):
    g = golden("evict_merge")
    vs = [torch.from_numpy(v) for v in g["v_in"]]
    keep = torch.from_numpy(g["keep"])
    imp = torch.from_numpy(g["importance"])
    surv = [T.merge_survivors(T.merge_centroids(vs, bi), keep[bi])[2] for bi in range(keep.shape[0])]
    a = T.merge_eviction_values(vs, keep, imp)
    b = T.merge_eviction_values(vs, keep, imp, survivors=surv)
    assert all(torch.equal(x, y) for x, y in zip(a, b))
    # a different survivor choice changes the result (the override is honoured)
    surv2 = [torch.zeros_like(s) for s in surv]
    c = T.merge_eviction_values(vs, keep, imp, survivors=surv2)
    assert not all(torch.equal(x, y) for x, y in zip(a, c))
