"""Pin the rANS restatement and the host frequency-table rule (CPU).

tests/golden/rans.npz holds the reference coder's own symbols, frequency
tables and 16-bit word streams (entropy_coder.py) for E8 code streams at
levels 4, 8, 16, an integer-only stream, a skewed stream and one symbol.
"""

import numpy as np
import pytest
import torch

from oracle import rans_ref as R

CASES = ["l8", "l4", "l16", "int", "skew", "one"]


@pytest.mark.parametrize("tag", CASES)
def test_restatement_reproduces_reference_words(golden, tag):
    g = golden("rans")
    L = int(g[f"{tag}_levels"])
    sym, has_half, alpha = R.lattice_to_symbols(g[f"{tag}_points"], L)
    assert np.array_equal(sym, g[f"{tag}_symbols"])
    assert has_half == bool(g[f"{tag}_has_half"]) and alpha == int(g[f"{tag}_alphabet"])
    words = R.rans_encode(sym, g[f"{tag}_freqs"])
    assert np.array_equal(np.array(words, np.uint16), g[f"{tag}_words"])
    assert np.array_equal(R.rans_decode(words, len(sym), g[f"{tag}_freqs"]), sym)


@pytest.mark.parametrize("tag", CASES)
def test_product_frequency_table_matches_reference(golden, tag):
    from nexusquant_amd.entropy import build_freq_table
    g = golden("rans")
    alpha = int(g[f"{tag}_alphabet"])
    counts = np.bincount(g[f"{tag}_symbols"], minlength=alpha)
    assert np.array_equal(build_freq_table(counts).astype(np.int64), g[f"{tag}_freqs"].astype(np.int64))


def test_frequency_table_edge_rules():
    from nexusquant_amd.entropy import build_freq_table
    # empty stream: uniform, remainder on symbol 0
    f = build_freq_table(np.zeros(9, np.int64))
    assert f.sum() == 4096 and f[0] == 4096 // 9 + 4096 % 9 and np.all(f[1:] == 4096 // 9)
    # every seen symbol keeps at least one slot even at 1 count in 10^9
    f = build_freq_table(np.array([10 ** 9, 1, 0, 1], np.int64))
    assert f.sum() == 4096 and f[1] >= 1 and f[3] >= 1 and f[2] == 0


def test_nqr1_container_roundtrip_on_host():
    from nexusquant_amd.entropy import RansStream, pack_nqr1, unpack_nqr1
    rng = np.random.default_rng(3)
    s = RansStream(words=torch.from_numpy(rng.integers(-2 ** 15, 2 ** 15, 777).astype(np.int16)),
                   offsets=torch.tensor([0, 300, 777], dtype=torch.int64),
                   freq=np.array([1000, 3000, 96], np.uint16), levels=2, has_half=False, n=8000, chunk=4096,
                   shape=(2, 4000))
    blob = pack_nqr1(s, scales=torch.arange(5, dtype=torch.float32))
    t, sc = unpack_nqr1(blob, shape=(2, 4000), device="cpu")
    assert torch.equal(t.words, s.words) and torch.equal(t.offsets, s.offsets)
    assert np.array_equal(t.freq, s.freq) and (t.levels, t.has_half, t.n, t.chunk) == (2, False, 8000, 4096)
    assert torch.equal(sc, torch.arange(5, dtype=torch.float32))
