"""GPU parity of the fused E8 dequant + matrix product (nq_e8_dequant_matmul)
against the oracle (e8_triton.py:373-444, 613-660).

Every product of the kernel is exact and its sums are fp32, so the bound is the
fp32 summation error: 2^-18 of sum_h |codes * scale * query| per entry (H <= 256
terms).  The identity query must reproduce codes * scales bit for bit.
"""

import numpy as np
import pytest
import torch

from oracle import torch_ref as T

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _case(k, h_pad, h, qc, seed, qscale=1.0, lo=-128, hi=127):
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(lo, hi + 1, (k, h_pad), generator=g, dtype=torch.int8)
    scales = torch.rand(k, generator=g) * 0.05 + 1e-4
    query = torch.randn(h, qc, generator=g) * qscale
    return codes, scales, query


def _check(codes, scales, query):
    from nexusquant_amd.kernels import e8_dequant_matmul
    out = e8_dequant_matmul(codes.to(DEV), scales.to(DEV), query.to(DEV))
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and out.shape == (codes.shape[0], query.shape[1])
    ref = T.e8_dequant_matmul(codes, scales, query).numpy()
    h = query.shape[0]
    mag = (codes[:, :h].double().abs() * scales.double()[:, None]) @ query.double().abs()
    got = out.cpu().double().numpy()
    assert np.all(np.abs(got - ref) <= 2.0 ** -18 * mag.numpy() + 1e-37)


@pytest.mark.parametrize("k,h_pad,h,qc", [(1000, 128, 128, 32), (77, 104, 100, 5), (4096, 256, 256, 64),
                                          (16, 8, 3, 1), (33, 64, 64, 17), (131, 96, 96, 48), (5, 256, 250, 3)])
def test_matches_oracle(k, h_pad, h, qc):
    print(f"[gpu] e8_dequant_matmul K={k} H_pad={h_pad} H={h} Q={qc}", flush=True)
    _check(*_case(k, h_pad, h, qc, k + h + qc))


@pytest.mark.parametrize("qscale", [1e-30, 1e20])
def test_query_magnitudes_beyond_fp16(qscale):
    """The query's three bf16 parts keep fp32's exponent range."""
    print(f"[gpu] e8_dequant_matmul query scale {qscale}", flush=True)
    _check(*_case(300, 128, 128, 8, 7, qscale=qscale))


def test_identity_query_reproduces_decoded_codes_exactly():
    from nexusquant_amd.kernels import e8_dequant_matmul
    print("[gpu] e8_dequant_matmul identity", flush=True)
    codes, scales, _ = _case(513, 128, 128, 1, 9)
    out = e8_dequant_matmul(codes.to(DEV), scales.to(DEV), torch.eye(128, device=DEV)).cpu()
    assert torch.equal(out, codes.float() * scales[:, None])


def test_empty_and_errors():
    from nexusquant_amd.kernels import e8_dequant_matmul
    from nexusquant_amd._lib import NexusQuantError
    print("[gpu] e8_dequant_matmul empty / errors", flush=True)
    codes, scales, query = _case(0, 16, 16, 4, 1)
    out = e8_dequant_matmul(codes.to(DEV), scales.to(DEV), query.to(DEV))
    assert out.shape == (0, 4)
    codes, scales, query = _case(8, 16, 16, 0, 1)
    assert e8_dequant_matmul(codes.to(DEV), scales.to(DEV), query.to(DEV)).shape == (8, 0)
    codes, scales, query = _case(8, 16, 24, 4, 1)
    with pytest.raises(ValueError):
        e8_dequant_matmul(codes.to(DEV), scales.to(DEV), query.to(DEV))  # H > H_pad
    codes, scales, query = _case(8, 264, 264, 4, 1)
    with pytest.raises(ValueError):
        e8_dequant_matmul(codes.to(DEV), scales.to(DEV), query.to(DEV))  # H_pad > 256
    with pytest.raises(AssertionError, match="codes must be"):
        e8_dequant_matmul(codes[0].to(DEV), scales.to(DEV), query.to(DEV))
    with pytest.raises(NexusQuantError):
        e8_dequant_matmul(codes, scales, query)  # host tensors
