"""The no-allocation key-key entry point (nq_score_keykey_noalloc) against the
workspace one (nq_score_keykey), through the C ABI: identical importance on two
calls in a row, the second smaller (the static scratch keeps the first call's
contents).  The host-side size check is tested without a GPU in test_abi.py."""

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _keys(b, h, s, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(b, h, s, d, generator=g)
    k[..., ::32] *= 8
    k[:, :, 0, :] *= 4
    return k.to(dtype).to(DEV)


@pytest.mark.parametrize("shapes", [
    # (b, h, s, d, dtype, obs): first call, then a smaller one
    [(4, 8, 8192, 128, torch.float16, 32), (2, 4, 1000, 128, torch.float16, 32)],
    [(1, 8, 3000, 96, torch.bfloat16, 48), (1, 2, 77, 96, torch.bfloat16, 10)],
    [(2, 4, 700, 256, torch.float16, 32), (1, 1, 33, 64, torch.float32, 32)],
])
def test_noalloc_equals_workspace_entry_point_twice(shapes):
    from nexusquant_amd import _lib
    from nexusquant_amd.ops import score_keykey, score_keykey_noalloc
    lib = _lib.load()
    for (b, h, s, d, dtype, obs) in shapes:
        print(f"[gpu] keykey noalloc b={b} h={h} s={s} d={d} {dtype} obs={obs}", flush=True)
        k = _keys(b, h, s, d, dtype, seed=b * 1000 + s)
        want = score_keykey(k, obs)
        out = torch.full((b, s), float("nan"), device=DEV)
        got = score_keykey_noalloc(k, obs, out=out)
        torch.cuda.synchronize()
        assert got.data_ptr() == out.data_ptr()
        assert torch.equal(got, want), (got - want).abs().max()
        assert lib.nq_score_keykey_workspace(b, h, s, obs) <= (8 << 20)
