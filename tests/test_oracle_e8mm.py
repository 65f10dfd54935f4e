"""CPU checks pinning the oracle's e8_dequant_matmul (e8_triton.py:373-444, 613-660).

The reference's own tests do not exercise it, so the oracle is pinned by a
brute-force loop on tiny inputs, by the identity query (the product then equals
the decoded codes * scales exactly) and by linearity in the query.
"""

import numpy as np
import torch

from oracle import torch_ref as T


def _inputs(k, h_pad, h, qc, seed):
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(-8, 9, (k, h_pad), generator=g, dtype=torch.int8)
    scales = torch.rand(k, generator=g) * 0.1 + 1e-3
    query = torch.randn(h, qc, generator=g)
    return codes, scales, query


def test_matches_brute_force_loops():
    codes, scales, query = _inputs(5, 16, 13, 3, 0)
    got = T.e8_dequant_matmul(codes, scales, query).numpy()
    want = np.zeros((5, 3))
    for k in range(5):
        for j in range(3):
            acc = 0.0
            for h in range(13):  # pad columns 13..15 ignored
                v = np.float32(np.float32(codes[k, h].item()) * np.float32(scales[k].item()))
                acc += float(v) * float(np.float32(query[h, j].item()))
            want[k, j] = acc
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_identity_query_gives_decoded_codes():
    codes, scales, _ = _inputs(7, 24, 24, 1, 1)
    out = T.e8_dequant_matmul(codes, scales, torch.eye(24))
    dec = (codes.float() * scales[:, None]).double()
    assert torch.equal(out, dec)


def test_linear_in_the_query():
    codes, scales, q1 = _inputs(9, 32, 30, 4, 2)
    _, _, q2 = _inputs(9, 32, 30, 4, 3)
    a = T.e8_dequant_matmul(codes, scales, q1) + 2.0 * T.e8_dequant_matmul(codes, scales, q2)
    b = T.e8_dequant_matmul(codes, scales, q1.double().add(2.0 * q2.double()).float())
    np.testing.assert_allclose(a.numpy(), b.numpy(), rtol=1e-6, atol=1e-6)


def test_padding_columns_are_ignored():
    codes, scales, query = _inputs(4, 16, 10, 2, 4)
    c2 = codes.clone()
    c2[:, 10:] = 127
    assert torch.equal(T.e8_dequant_matmul(codes, scales, query), T.e8_dequant_matmul(c2, scales, query))
