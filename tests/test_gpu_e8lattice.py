"""GPU parity of the standalone relaxed-E8 primitives (nq_e8_nearest_point,
nq_e8_quantize_perhead) against the reference's own outputs (tests/golden
e8_nearest / e8_perhead, written by E8Lattice) and the C spec (oracle/nq_spec.c).

The kernels decide half vs integer candidate by sum |x - rint(x)| against 2 or
1 + 2 min |x - rint(x)|, the spec's form of d_half < d_int; they equal the spec
bit for bit and the reference except on groups whose spec margin is < 1e-6.
"""

import numpy as np
import pytest
import torch

from oracle import spec as S
from oracle import torch_ref as T

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_nearest_point_matches_reference_fixture_except_near_ties(golden):
    from nexusquant_amd.kernels import e8_nearest_point
    print("[gpu] e8_nearest_point fixture", flush=True)
    g = golden("e8_nearest")
    got = e8_nearest_point(torch.from_numpy(g["x"]).to(DEV)).cpu().numpy()
    p_spec, _, margin = S.e8_groups(g["x"], 1 << 20)  # no clamp in range
    assert np.array_equal(got, p_spec)
    diff = (got != g["p"]).any(axis=1)
    assert diff.mean() < 1e-4
    assert np.all(margin[diff] < 1e-6)


def test_nearest_point_equals_spec_on_wide_inputs():
    from nexusquant_amd.kernels import e8_nearest_point
    print("[gpu] e8_nearest_point wide inputs", flush=True)
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((50000, 8)) * np.array([0.3, 1, 3, 30, 200, 0.01, 5, 1])).astype(np.float32)
    x[:64] = np.round(x[:64] * 2) / 2      # exact half-integers and integers: gaps of 0 and 0.5
    x[64:96] = 0.0
    got = e8_nearest_point(torch.from_numpy(x).to(DEV).reshape(2, 25000, 8)).reshape(-1, 8).cpu().numpy()
    want, _, _ = S.e8_groups(x, 1 << 20)
    assert np.array_equal(got, want)
    assert e8_nearest_point(torch.empty(0, 8, device=DEV)).shape == (0, 8)
    with pytest.raises(AssertionError, match="last dim must be 8"):
        e8_nearest_point(torch.zeros(3, 7, device=DEV))


@pytest.mark.parametrize("levels", [2, 4, 8, 16])
def test_quantize_perhead_matches_reference_fixture_except_near_ties(golden, levels):
    from nexusquant_amd.kernels import e8_quantize_perhead
    print(f"[gpu] e8_quantize_perhead fixture L={levels}", flush=True)
    g = golden("e8_perhead")
    x = g["x"]
    got = e8_quantize_perhead(torch.from_numpy(x).to(DEV), levels=levels).cpu().numpy()
    ref = g[f"q{levels}"]
    # rows with a near-tie group (spec margin < 1e-6 on the normalised groups) may differ
    xt = torch.from_numpy(x)
    amax = xt.abs().amax(dim=-1, keepdim=True).clamp(min=1e-8)
    norm = (xt / (amax / (levels / 2))).numpy()
    _, _, margin = S.e8_groups(norm.reshape(-1, 8), levels)
    near = (margin.reshape(x.shape[0], -1) < 1e-6).any(axis=1)
    diff = (got != ref).any(axis=1)
    assert np.all(near[diff])
    assert diff.mean() < 0.01
    assert np.array_equal(got[~near], ref[~near])


@pytest.mark.parametrize("d,levels,dtype", [(100, 4, torch.float32), (8, 8, torch.float32),
                                            (256, 3, torch.float32), (128, 8, torch.float16),
                                            (37, 16, torch.float32)])
def test_quantize_perhead_equals_oracle_on_other_shapes(d, levels, dtype):
    """d not a multiple of 8 (zero padding), an odd level count, fp16 input
    (computed in fp32, returned as fp16), and a zero row (amax clamp)."""
    from nexusquant_amd.kernels import e8_quantize_perhead
    print(f"[gpu] e8_quantize_perhead d={d} L={levels} {dtype}", flush=True)
    g = torch.Generator().manual_seed(d + levels)
    x = torch.randn(3, 97, d, generator=g).to(dtype)
    x[1, 5] = 0
    got = e8_quantize_perhead(x.to(DEV), levels=levels).cpu()
    assert got.dtype == dtype and got.shape == x.shape
    ref = T.e8_quantize_perhead(x.float(), levels=levels).to(dtype)
    xf = x.float().reshape(-1, d)
    amax = xf.abs().amax(dim=-1, keepdim=True).clamp(min=1e-8)
    norm = torch.nn.functional.pad(xf / (amax / (levels / 2)), (0, (8 - d % 8) % 8)).numpy()
    _, _, margin = S.e8_groups(norm.reshape(-1, 8), levels)
    near = torch.from_numpy((margin.reshape(xf.shape[0], -1) < 1e-6).any(axis=1))
    same = (got.reshape(-1, d) == ref.reshape(-1, d)).all(dim=1)
    assert bool((same | near).all())
    assert bool((got.reshape(-1, d)[97 + 5] == 0).all())  # the zero row x[1, 5]
