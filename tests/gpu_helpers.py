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
