"""GPU parity of merge eviction (nq_merge_values) against the Tier-A restatement
and the reference's own fixture.

Bit for bit: centroids (the reference's reduction order), and the merged
values given the same survivors.  Survivors: identical except where two
kept tokens' cosines lie within 1e-6 (the reference's cosines come from an
MKL GEMM whose summation order differs).
"""

import numpy as np
import pytest
import torch

from oracle import torch_ref as T

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


class Cache:
    def __init__(self, ks, vs):
        self.key_cache, self.value_cache = list(ks), list(vs)


def _kept_lists(keep):
    b, s = keep.shape
    kept = torch.zeros(b, s, dtype=torch.int32)
    n = torch.zeros(b, dtype=torch.int32)
    for bi in range(b):
        idx = torch.nonzero(keep[bi]).flatten()
        kept[bi, :len(idx)] = idx.to(torch.int32)
        n[bi] = len(idx)
    return kept, n


def _check_survivors(vs_cpu, keep, surv_gpu, tol=1e-6):
    """Survivors equal the oracle's argmax except at cosine near ties; returns
    the per-row kept-list indices of the GPU's survivors."""
    local = []
    for bi in range(keep.shape[0]):
        cent = T.merge_centroids(vs_cpu, bi)
        ev, kp, nearest, cos = T.merge_survivors(cent, keep[bi])
        got_pos = torch.from_numpy(surv_gpu[bi][ev.numpy()]).long()
        pos_to_local = torch.full((keep.shape[1],), -1, dtype=torch.long)
        pos_to_local[kp] = torch.arange(len(kp))
        got = pos_to_local[got_pos]
        assert torch.all(got >= 0)
        bad = got != nearest
        if bad.any():
            rows = torch.nonzero(bad).flatten()
            c_got = cos[rows, got[rows]]
            c_ref = cos[rows, nearest[rows]]
            assert torch.all((c_ref - c_got).abs() <= tol), (c_ref - c_got).abs().max()
        assert np.all(surv_gpu[bi][kp.numpy()] == -1)
        local.append(got)
    return local


def _run(vs_cpu, keep, imp):
    from nexusquant_amd.ops import merge_values
    kept, n = _kept_lists(keep)
    return merge_values([v.to(DEV) for v in vs_cpu], keep.to(DEV), kept.to(DEV), n.to(DEV), imp.to(DEV),
                        centroids=True, survivors=True)


def test_merge_parts_match_reference_fixture(golden):
    print("[gpu] merge fixture parts", flush=True)
    g = golden("evict_merge")
    vs = [torch.from_numpy(v) for v in g["v_in"]]
    keep = torch.from_numpy(g["keep"])
    imp = torch.from_numpy(g["importance"])
    merged, cent, surv = _run(vs, keep, imp)
    torch.cuda.synchronize()
    assert np.array_equal(cent.cpu().numpy(), g["centroids"])
    surv = surv.cpu().numpy()
    local = _check_survivors(vs, keep, surv)
    want = T.merge_eviction_values(vs, keep, imp, survivors=local)
    for li in range(len(vs)):
        assert np.array_equal(merged[li].cpu().numpy(), want[li].numpy())
    if np.array_equal(surv, g["survivor"]):
        for li in range(len(vs)):
            assert np.array_equal(merged[li].cpu().numpy(), g["v_merged"][li])


def test_merge_eviction_pipeline_matches_reference_fixture(golden):
    import nexusquant_amd as nq
    from test_gpu_evict import _assert_close_rows
    print("[gpu] merge eviction pipeline fixture", flush=True)
    g = golden("evict_merge")
    c = Cache([torch.from_numpy(k).to(DEV) for k in g["k_in"]], [torch.from_numpy(v).to(DEV) for v in g["v_in"]])
    comp = nq.NexusQuantEvict(key_bits=3, value_bits=2, eviction_rate=0.5, sliding_window=8, rope_base=10000.0,
                              merge_eviction=True, protect_boundary=1)
    imp = torch.from_numpy(g["importance"]).to(DEV)
    comp._score_importance = lambda k, _imp=imp: _imp  # the reference's scores: identical merge weights
    _, mask = comp.compress(c)
    assert np.array_equal(mask.cpu().numpy(), g["mask"])
    for li in range(3):
        if li in (0, 2):  # protected layers: merged values cast to fp16
            assert np.array_equal(c.key_cache[li].cpu().numpy(), g["k_out"][li])
            assert np.array_equal(c.value_cache[li].cpu().numpy(), g["v_out"][li])
        else:
            _assert_close_rows(c.key_cache[li], g["k_out"][li])
            _assert_close_rows(c.value_cache[li], g["v_out"][li])


@pytest.mark.parametrize("dtype,d,s,h,b", [(torch.float16, 128, 3000, 4, 2), (torch.bfloat16, 96, 700, 2, 3),
                                           (torch.float32, 64, 1100, 3, 1), (torch.float16, 256, 500, 2, 1),
                                           (torch.float16, 128, 40, 24, 2), (torch.float16, 128, 32768, 2, 1)])
def test_merge_values_match_oracle(dtype, d, s, h, b):
    from nexusquant_amd.ops import keep_mask
    print(f"[gpu] merge {dtype} d={d} s={s} h={h} b={b}", flush=True)
    gen = torch.Generator().manual_seed(s + d)
    vs = [(torch.randn(b, h, s, d, generator=gen) * 0.7).to(dtype) for _ in range(3)]
    imp = torch.rand(b, s, generator=gen) + 1e-3
    keep_d, _, _ = keep_mask(imp.to(DEV), 0.4, 16)
    keep = keep_d.cpu().bool()
    merged, cent, surv = _run(vs, keep, imp)
    torch.cuda.synchronize()
    for bi in range(b):
        assert torch.equal(cent[bi].cpu(), T.merge_centroids(vs, bi))
    local = _check_survivors(vs, keep, surv.cpu().numpy())
    want = T.merge_eviction_values(vs, keep, imp, survivors=local)
    for li in range(3):
        assert merged[li].dtype == dtype
        assert torch.equal(merged[li].cpu(), want[li])


def test_merge_survivor_ties_take_the_first_kept_token():
    print("[gpu] merge ties", flush=True)
    b, h, s, d = 1, 2, 64, 128
    gen = torch.Generator().manual_seed(4)
    v = torch.randn(b, h, s, d, generator=gen).half()
    # kept positions 5 and 9 and evicted position 7 share one value vector in
    # every layer: their cosines tie exactly and the first kept token wins
    v[:, :, 9] = v[:, :, 5]
    v[:, :, 7] = v[:, :, 5] * 2
    vs = [v.clone(), v.clone()]
    keep = torch.zeros(b, s, dtype=torch.bool)
    keep[:, [0, 5, 9, 20, 33]] = True
    keep[:, s - 8:] = True
    imp = torch.rand(b, s, generator=gen)
    merged, _, surv = _run(vs, keep, imp)
    torch.cuda.synchronize()
    assert surv[0, 7].item() == 5
    local = _check_survivors(vs, keep, surv.cpu().numpy(), tol=0.0)
    want = T.merge_eviction_values(vs, keep, imp, survivors=local)
    assert all(torch.equal(m.cpu(), w) for m, w in zip(merged, want))
