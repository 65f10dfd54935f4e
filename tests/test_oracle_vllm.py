"""Pin the vLLM page caller's oracles (CPU).

Tier A (oracle/torch_ref.py vllm_*) must reproduce the reference's own outputs
(tests/golden/vllm_pages.npz, written by integrations/vllm_backend.py) bit for
bit.  The Tier-B page arithmetic (oracle/nq_spec.c) must stay within the
parity tolerance of them and satisfy closed forms.  The chunk planner of the
paged decode consumer is checked against a brute-force token walk.
"""

import numpy as np
import pytest
import torch

from oracle import spec as S
from oracle import torch_ref as T

CASES = [("b2", 2, 10000.0), ("b3", 3, 500000.0), ("b4", 4, 10000.0)]


def _t(a):
    return torch.from_numpy(np.asarray(a))


@pytest.mark.parametrize("tag,bits,base", CASES)
def test_tier_a_reproduces_reference_pages(golden, tag, bits, base):
    g = golden("vllm_pages")
    kc, vc, ks, vs = T.vllm_compress_page(_t(g[f"{tag}_k"]), _t(g[f"{tag}_v"]), _t(g[f"{tag}_pos"]), bits, base)
    for got, name in ((kc, "kc"), (vc, "vc"), (ks, "ks"), (vs, "vs")):
        assert np.array_equal(got.numpy(), g[f"{tag}_{name}"]), name
    kd, vd = T.vllm_decompress_page(kc, vc, ks, vs, _t(g[f"{tag}_pos"]), base)
    assert np.array_equal(kd.numpy(), g[f"{tag}_kdec"])
    assert np.array_equal(vd.numpy(), g[f"{tag}_vdec"])
    lg = T.vllm_decompress_for_attention(kc, ks, _t(g[f"{tag}_pos"]), _t(g[f"{tag}_q"]), base)
    assert np.array_equal(lg.numpy(), g[f"{tag}_logits"])


def test_tier_a_reproduces_reference_nibbles_and_forward(golden):
    g = golden("vllm_pages")
    assert np.array_equal(T.pack_codes_nibble(_t(g["nib_codes"])).numpy(), g["nib_packed"])
    assert np.array_equal(T.unpack_codes_nibble(_t(g["nib_packed"]), 33).numpy(), g["nib_unpacked"])
    pages = {i: tuple(_t(g[n][i]) for n in ("fwd_kc", "fwd_vc", "fwd_ks", "fwd_vs", "fwd_pos")) for i in range(6)}
    out = T.vllm_paged_forward(_t(g["fwd_query"]), pages, [[0, 1, 2], [3, 99, 4], [5], [2, 0]],
                               g["fwd_ctx"].tolist(), 10000.0)
    assert np.array_equal(out.numpy(), g["fwd_out"])


def _rows(x, pos, d, base, key):
    """Page [h, n, d] -> rows [h*n, d] and per-row tables at the token positions."""
    h, n, _ = x.shape
    rows = np.asarray(x, np.float32).reshape(-1, d)
    if not key:
        return rows, None, None
    c, s = T.rope_cos_sin(_t(pos).float(), d, base)
    return rows, np.tile(c.numpy(), (h, 1)), np.tile(s.numpy(), (h, 1))


@pytest.mark.parametrize("tag,bits,base", CASES)
def test_page_encode_spec_within_tolerance_of_reference(golden, tag, bits, base):
    g = golden("vllm_pages")
    L = 2 ** bits
    for role, key in (("k", True), ("v", False)):
        x = g[f"{tag}_{role}"]
        d = x.shape[-1]
        rows, c, s = _rows(x, g[f"{tag}_pos"], d, base, key)
        codes, scales, margin = S.page_encode(rows, L, c, s)
        ref = g[f"{tag}_{role}c"].reshape(-1, d)
        mism = (codes.reshape(-1, 8) != ref.reshape(-1, 8)).any(1)
        assert mism.mean() <= 1e-2
        assert np.all(margin.reshape(-1)[mism] < 1e-5)
        rs = g[f"{tag}_{role}s"].reshape(-1)
        diff = scales.view(np.uint16).astype(np.int32) - rs.view(np.uint16).astype(np.int32)
        assert np.all(np.abs(diff) <= 1) and (diff != 0).mean() <= 0.05


@pytest.mark.parametrize("tag,bits,base", CASES)
def test_page_decode_spec_within_tolerance_of_reference(golden, tag, bits, base):
    g = golden("vllm_pages")
    for role, key in (("k", True), ("v", False)):
        codes = g[f"{tag}_{role}c"]
        h, n, d = codes.shape
        _, c, s = _rows(np.zeros((h, n, d), np.float32), g[f"{tag}_pos"], d, base, key)
        got = S.page_decode(codes.reshape(-1, d), g[f"{tag}_{role}s"].reshape(-1), key, c, s)
        ref = g[f"{tag}_{role}dec"].reshape(-1, d)
        same = (got.view(np.uint16) == ref.view(np.uint16)) | ((got == 0) & (ref == 0))
        # the spec's integer transform gives exact zeros where the reference's GEMM
        # leaves rounding noise (fp16 subnormals): most of the differing entries
        assert same.mean() >= 0.98
        # where they differ: one fp16 ulp, or a few fp32 ulps of the row's largest
        # term where the rotation cancels (the reference rounds the GEMM and each
        # rotation product separately)
        g32, r32 = got.astype(np.float32), ref.astype(np.float32)
        big = np.maximum(np.abs(g32), np.abs(r32))
        tol = np.spacing(big.astype(np.float16)).astype(np.float32) + 1e-6 * np.abs(r32).max(1, keepdims=True)
        assert np.all(np.abs(g32 - r32) <= tol)


def test_page_decode_spec_closed_form():
    # One nonzero code c_j = 2 (p = 1) decodes to +-fp16(2 g) with the sign of
    # the Sylvester entry S[i, j] and g = fl(fl(scale/2) h_D); keys then rotate
    # each pair (i, i+D/2) by the position's angle.  A transposed operand, a
    # dropped scale factor or a wrong pair index fails this.
    D = 128
    H = np.sign(T.hadamard_matrix(D).numpy())
    sc = np.float16(0.375)
    hD = np.float32(S.hadamard_constant(D))
    g2 = np.float32(2.0) * (np.float32(0.5) * np.float32(sc) * hD)
    for j in (0, 5, 64, 127):
        codes = np.zeros((1, D), np.int8)
        codes[0, j] = 2
        vals = S.page_decode(codes, np.array([sc]), False)
        assert np.array_equal(vals[0], (H[:, j] * g2).astype(np.float16))
        pos = 1234
        c, s = T.rope_cos_sin(torch.tensor([float(pos)]), D, 10000.0)
        keys = S.page_decode(codes, np.array([sc]), True, c.numpy(), s.numpy())[0].astype(np.float64)
        u = H[:, j] * np.float64(g2)
        lo, hi = u[:D // 2], u[D // 2:]
        cc, ss = c.numpy()[0].astype(np.float64), s.numpy()[0].astype(np.float64)
        want = np.concatenate([lo * cc - hi * ss, lo * ss + hi * cc])
        tol = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64) + 1e-7
        assert np.all(np.abs(keys - want) <= tol)


def test_chunk_plan_walks_the_reference_token_order():
    from nexusquant_amd.vllm_backend import build_chunk_plan
    rng = np.random.default_rng(12)
    for trial in range(60):
        cap = int(rng.choice([16, 64, 512]))
        rows, ctx, want = [], [], []
        for b in range(int(rng.integers(1, 5))):
            row = [(int(rng.integers(0, 20)), int(rng.choice([1, 7, 16, 16, 33, 600]))) for _ in range(int(rng.integers(0, 6)))]
            stream = [(slot, t) for slot, n in row for t in range(n)]
            c = int(rng.choice([0, 5, 40, 10 ** 6, -3, -10 ** 6]))
            rows.append(row)
            ctx.append(c)
            want.append(stream[:c] if c != 0 else [])
        parts, total = build_chunk_plan(rows, ctx, cap)
        segs = parts["segs"].reshape(-1, 4)
        units = parts["units"].reshape(-1, 2)
        cu, cr, ct, rc = parts["chunk_units"], parts["chunk_row"], parts["chunk_tokens"], parts["row_chunks"]
        assert total == sum(len(w) for w in want)
        assert len(cu) == len(cr) + 1 and len(rc) == len(rows) + 1 and cu[-1] == len(units)
        for b in range(len(rows)):
            got = []
            for c in range(rc[b], rc[b + 1]):
                assert cr[c] == b and 0 < ct[c] <= cap
                seen = np.zeros(ct[c], bool)
                for u in range(cu[c], cu[c + 1]):
                    seg, t0 = units[u]
                    slot, first, n, off = segs[seg]
                    for t in range(t0, min(t0 + 16, n)):
                        assert not seen[off + t]
                        seen[off + t] = True
                        got.append((off + t, slot, first + t))
                assert seen.all()
                got[-ct[c]:] = sorted(got[-ct[c]:])
            assert [(s, t) for _, s, t in got] == want[b]
