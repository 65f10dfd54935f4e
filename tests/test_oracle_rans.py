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


def _good_blob():
    from nexusquant_amd.entropy import RansStream, pack_nqr1
    rng = np.random.default_rng(4)
    s = RansStream(words=torch.from_numpy(rng.integers(-2 ** 15, 2 ** 15, 900).astype(np.int16)),
                   offsets=torch.tensor([0, 500, 900], dtype=torch.int64),
                   freq=np.array([1000, 3000, 96], np.uint16), levels=2, has_half=False, n=8000, chunk=4096,
                   shape=(8000,))
    return s, pack_nqr1(s, scales=torch.ones(3))


def _patch(blob, fmt, offset, *vals):
    import struct
    b = bytearray(blob)
    struct.pack_into(fmt, b, offset, *vals)
    return bytes(b)


@pytest.mark.parametrize("what", ["n_chunks", "n_symbols", "chunk0", "alphabet", "freq_sum", "offset0",
                                  "offsets_order", "offset_end", "truncated", "scales_tail",
                                  "shape"])
def test_nqr1_rejects_inconsistent_containers(what):
    # every header field the decoder trusts is checked on the host, so a
    # corrupted or truncated container raises instead of reaching the device
    from nexusquant_amd.entropy import unpack_nqr1
    _, blob = _good_blob()
    # magic, then '<HBBHHQII' (24 bytes): alphabet at 8, n at 12, chunk at 20, n_chunks at 24
    head = 28
    freq_at = head
    off_at = head + 8                # 3 freqs (6 bytes) padded to 8
    shape = None
    if what == "n_chunks":
        blob = _patch(blob, "<I", 24, 1)
    elif what == "n_symbols":
        blob = _patch(blob, "<Q", 12, 20000)
    elif what == "chunk0":
        blob = _patch(blob, "<I", 20, 0)
    elif what == "alphabet":
        blob = _patch(blob, "<H", 8, 5)
    elif what == "freq_sum":
        blob = _patch(blob, "<H", freq_at, 999)
    elif what == "offset0":
        blob = _patch(blob, "<Q", off_at, 1)
    elif what == "offsets_order":
        blob = _patch(blob, "<Q", off_at + 8, 950)
    elif what == "offset_end":
        blob = _patch(blob, "<Q", off_at + 16, 899)
    elif what == "truncated":
        blob = blob[:off_at + 24 + 100]
    elif what == "scales_tail":
        blob = blob + b"\0\0"
    elif what == "shape":
        shape = (7999,)
    with pytest.raises(ValueError):
        unpack_nqr1(blob, shape=shape, device="cpu")


def test_nqr1_rejects_chunk_with_too_many_words():
    from nexusquant_amd.entropy import RansStream, pack_nqr1, unpack_nqr1
    s = RansStream(words=torch.zeros(20, dtype=torch.int16), offsets=torch.tensor([0, 12, 20], dtype=torch.int64),
                   freq=np.array([1000, 3000, 96], np.uint16), levels=2, has_half=False, n=15, chunk=8,
                   shape=(15,))
    with pytest.raises(ValueError, match="more words"):
        unpack_nqr1(pack_nqr1(s), device="cpu")   # chunk 0: 8 symbols, at most 10 words
    s.offsets = torch.tensor([0, 10, 19], dtype=torch.int64)
    s.words = torch.zeros(19, dtype=torch.int16)
    t, _ = unpack_nqr1(pack_nqr1(s), device="cpu")
    assert t.n == 15 and t.offsets.tolist() == [0, 10, 19]


@pytest.mark.parametrize("change", ["offsets_in_place", "offsets_reassigned", "freq_in_place", "n"])
def test_decode_rechecks_a_stream_changed_after_its_check(change):
    # a checked stream skips the host check only while its tensors, their
    # in-place versions and the frequency table are unchanged; any change is
    # checked again (and raises here before any device work)
    from nexusquant_amd.entropy import rans_decode, unpack_nqr1
    _, blob = _good_blob()
    st, _ = unpack_nqr1(blob, device="cpu")
    assert st._checked == st._layout_key()
    if change == "offsets_in_place":
        st.offsets[1] += 450
    elif change == "offsets_reassigned":
        st.offsets = torch.tensor([0, 950, 900], dtype=torch.int64)
    elif change == "freq_in_place":
        st.freq[0] = 999
    else:
        st.n = 20000
    assert st._checked != st._layout_key()
    with pytest.raises(ValueError):
        rans_decode(st)


def test_single_chain_limit_is_stated_and_checked_on_the_host():
    # chunks (and so encode_e8 / decode_e8 containers) take up to 2^31 - 1
    # symbols; larger requests are refused before any device work
    import struct
    from nexusquant_amd import entropy as E
    E.check_stream_header(8, True, 17, (1 << 31) - 1, (1 << 31) - 1, 1)
    with pytest.raises(ValueError, match="2\\^31 - 1"):
        E.check_stream_header(8, True, 17, 1 << 31, 1 << 31, 1)
    big = torch.zeros(1).expand((1 << 31) + 8)         # no memory behind the view
    with pytest.raises(ValueError, match="2\\^31 - 1"):
        E.encode_e8(big, torch.ones(1))
    n_groups = 1 << 28                                 # 2^31 symbols
    freq = struct.pack("<H", 9) + b"\x00\x02" * 9
    blob = (E.E8_HEADER.pack(n_groups, 8, 0, 8 * n_groups) + E.E8_LENGTHS.pack(len(freq), 2, 4)
            + freq + b"\x00" * 6)
    with pytest.raises(ValueError, match="2\\^31 - 1"):
        E.decode_e8(blob)
