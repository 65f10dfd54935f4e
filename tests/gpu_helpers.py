"""Shared helpers of the GPU parity tests: the C spec run with the kernel's row
selection, and fp16 comparison up to the sign of zero."""

import numpy as np
import torch

from oracle import spec as S
from oracle import torch_ref as T


def spec_tensor(x, L, is_key, base=10000.0, scaling=None, gather=None, keep=None):
    """Run the C spec on a [b, h, s, d] float32 array with the kernel's row selection."""
    b, h, s, d = x.shape
    s_out = s if gather is None else gather.shape[1]
    t_in = np.tile(np.arange(s_out), (b, 1)) if gather is None else gather
    rows = np.empty((b, h, s_out, d), np.float32)
    for bi in range(b):
        rows[bi] = x[bi][:, t_in[bi], :]
        if keep is not None:
            rows[bi][:, keep[bi][t_in[bi]] == 0, :] = 0.0
    rows = rows.reshape(-1, d)
    kw = {}
    if is_key:
        n = max(s, s_out)
        c, sn = T.rope_cos_sin(torch.arange(n, dtype=torch.float32), d, base, scaling)
        c, sn = c.numpy(), sn.numpy()
        pos_in = np.repeat(t_in[:, None, :], h, axis=1).reshape(-1)
        pos_out = np.tile(np.arange(s_out), b * h)
        kw = dict(cos_in=c[pos_in], sin_in=sn[pos_in], cos_out=c[pos_out], sin_out=sn[pos_out])
    return S.quant_rows(rows, L, **kw)


def assert_same_fp16(got, want):
    """Bit-exact fp16 up to the sign of zero.

    The kernel's cross-lane butterflies compute b - a where the spec computes
    a - b and fold the sign later, so an exact zero may come out as -0 where
    the spec has +0 (and vice versa); every other bit must match.
    """
    got = np.ascontiguousarray(got, dtype=np.float16)
    want = np.ascontiguousarray(want, dtype=np.float16)
    diff = got.view(np.uint16) != want.view(np.uint16)
    bad = diff & ~((got == 0) & (want == 0))
    rows = np.nonzero(bad.reshape(bad.shape[0], -1).any(1))[0] if bad.ndim > 1 else np.nonzero(bad)[0]
    assert rows.size == 0, f"{rows.size} fp16 rows differ, first {rows[:5]}"


def keep_sets_match(imp_gpu, imp_ref, keep_gpu, keep_ref, tol=1e-6, window=32):
    """Keep sets identical except positions whose reference score lies within tol
    of the k-th largest prefix score (a tie the two scorers may break differently)."""
    diff = keep_gpu != keep_ref
    for bi in range(keep_gpu.shape[0]):
        idx = np.nonzero(diff[bi])[0]
        if idx.size == 0:
            continue
        s = keep_ref.shape[1]
        prefix = max(s - window, 0)
        scores = np.sort(imp_ref[bi][1:prefix])[::-1]
        k = int(keep_ref[bi][1:prefix].sum())
        kth = scores[k - 1] if k > 0 else np.inf
        if np.any(np.abs(imp_ref[bi][idx] - kth) > tol):
            return False
    return True


def assert_close_rows(got, ref, max_flip_frac=1e-4):
    got = got.float().cpu().numpy().reshape(-1, got.shape[-1])
    ref = np.asarray(ref, np.float32).reshape(-1, got.shape[-1])
    num = np.linalg.norm(got - ref, axis=1)
    den = np.maximum(np.linalg.norm(ref, axis=1), 1e-30)
    flipped = (num / den) > 1e-2
    assert flipped.sum() <= max(1, int(max_flip_frac * got.size / 8)), flipped.sum()
    ok = ~flipped
    if ok.any() and np.linalg.norm(ref[ok]) > 0:
        assert np.linalg.norm(got[ok] - ref[ok]) / np.linalg.norm(ref[ok]) <= 1e-3
