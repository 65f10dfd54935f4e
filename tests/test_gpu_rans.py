"""GPU parity of the chunked rANS stage (nq_rans_*): one chunk reproduces the
reference encoder's word stream exactly; many chunks decode losslessly, each
chunk equal to the restated encoder on its symbols, at near-Shannon size."""

import numpy as np
import pytest
import torch

from oracle import rans_ref as R

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("tag", ["l8", "l4", "l16", "int", "skew", "one"])
def test_single_chunk_equals_reference_words(golden, tag):
    from nexusquant_amd.entropy import rans_decode, rans_encode
    print(f"[gpu] rans fixture {tag}", flush=True)
    g = golden("rans")
    L = int(g[f"{tag}_levels"])
    codes = torch.from_numpy(np.round(g[f"{tag}_points"] * 2).astype(np.int8))
    st = rans_encode(codes.to(DEV), L, chunk=1 << 20)
    assert st.has_half == bool(g[f"{tag}_has_half"])
    assert np.array_equal(st.freq.astype(np.int64), g[f"{tag}_freqs"].astype(np.int64))
    words = st.words.cpu().numpy().view(np.uint16)
    assert np.array_equal(words, g[f"{tag}_words"])
    assert torch.equal(rans_decode(st).cpu(), codes)


@pytest.mark.parametrize("levels,n,chunk", [(8, 1_000_003, 4096), (8, 300_001, 2048), (4, 262_144, 1024), (16, 70_000, 4096),
                                            (2, 4096, 4096), (8, 1, 4096), (4, 50_001, 1000), (8, 40_000, 200)])
def test_chunked_roundtrip_and_chunk_words(levels, n, chunk):
    from nexusquant_amd.entropy import pack_nqr1, rans_decode, rans_encode, shannon_bits, unpack_nqr1
    from nexusquant_amd.ops import quantize_tensors
    from nexusquant_amd.codec import codes_int8
    print(f"[gpu] rans L={levels} n={n} chunk={chunk}", flush=True)
    rows = (n + 127) // 128
    x = torch.randn(1, 1, rows, 128, generator=torch.Generator().manual_seed(n)).half().to(DEV)
    _, cd = quantize_tensors([x], is_key=False, levels=levels, recon=False, codes=True)
    codes = codes_int8(cd)[0].reshape(-1)[:n].contiguous()
    st = rans_encode(codes, levels, chunk=chunk)
    back = rans_decode(st)
    assert torch.equal(back, codes)
    c = codes.cpu().numpy()
    sym = (c.astype(np.int32) + levels) if st.has_half else (c.astype(np.int32) // 2 + levels // 2)
    offs = st.offsets.cpu().numpy()
    words = st.words.cpu().numpy().view(np.uint16)
    n_chunks = len(offs) - 1
    for k in sorted({0, n_chunks // 2, n_chunks - 1}):
        want = R.rans_encode(sym[k * chunk:(k + 1) * chunk], st.freq)
        assert np.array_equal(words[offs[k]:offs[k + 1]], np.array(want, np.uint16))
    counts = np.bincount(sym, minlength=st.alphabet)
    bits = 16 * words.size
    assert bits <= 1.01 * shannon_bits(counts) + 32 * n_chunks + 64
    blob = pack_nqr1(st, scales=cd[0].scales)
    st2, sc = unpack_nqr1(blob, shape=codes.shape, device=DEV)
    assert torch.equal(rans_decode(st2), codes)
    assert torch.equal(sc, cd[0].scales.cpu().reshape(-1))


@pytest.mark.parametrize("case", ["constant", "rare", "runs"])
def test_skewed_streams_roundtrip_and_chunk_words(case):
    """Streams with long stretches of no renormalisation (one symbol at
    probability 1, or nearly): the decoder's word ring stays full and the
    encoder emits little but the final states."""
    from nexusquant_amd.entropy import rans_decode, rans_encode
    print(f"[gpu] rans skewed {case}", flush=True)
    rng = np.random.default_rng(5)
    n, chunk, levels = 300_000, 4096, 4
    c = np.zeros(n, np.int8)
    if case == "rare":
        hit = rng.random(n) < 0.003
        c[hit] = rng.choice(np.array([-4, -2, 2, 4], np.int8), hit.sum())
    elif case == "runs":
        for s0 in range(0, n, 20_000):  # dense bursts between long constant runs
            c[s0:s0 + 3000] = rng.choice(np.array([-4, -2, 0, 2, 4], np.int8), 3000)
    codes = torch.from_numpy(c).to(DEV)
    st = rans_encode(codes, levels, chunk=chunk)
    assert torch.equal(rans_decode(st), codes)
    sym = c.astype(np.int32) // 2 + levels // 2
    offs = st.offsets.cpu().numpy()
    words = st.words.cpu().numpy().view(np.uint16)
    for k in sorted({0, 1, 5, len(offs) - 2}):
        want = R.rans_encode(sym[k * chunk:(k + 1) * chunk], st.freq)
        assert np.array_equal(words[offs[k]:offs[k + 1]], np.array(want, np.uint16))


@pytest.mark.parametrize("n_chunks", [3 * 32768 + 1000, 6 * 32768 + 1001])
@pytest.mark.parametrize("has_half", [False, True])
def test_offsets_across_scan_segments_and_compact_strides(has_half, n_chunks):
    """99,304 chunks of 32 codes, the last one ragged: the chunk offsets are
    scanned in segments of 4,096 chunks, and the compaction's waves take the
    chunks in groups of 8 and stride over them, most waves coming back for a
    second group; chunks on either side of segment boundaries and at both
    ends are checked against the restated encoder, and offsets against the
    cumulative sums of those per-chunk word counts.  At 197,609 chunks the
    decoder runs six waves per block and the encoder four, the last block of
    each partly empty; 32-code chunks take the encoder's 16-code path."""
    from nexusquant_amd.entropy import rans_decode, rans_encode
    print(f"[gpu] rans offsets across scan segments has_half={has_half} n_chunks={n_chunks}", flush=True)
    chunk, levels = 32, 8
    n = n_chunks * chunk - 7
    rng = np.random.default_rng(11)
    vals = np.arange(-levels, levels + 1) if has_half else np.arange(-levels, levels + 1, 2)
    p = np.exp(-0.5 * (vals / 3.0) ** 2)
    c = rng.choice(vals, n, p=p / p.sum()).astype(np.int8)
    codes = torch.from_numpy(c).to(DEV)
    st = rans_encode(codes, levels, chunk=chunk)
    assert st.has_half == has_half
    assert torch.equal(rans_decode(st), codes)
    sym = (c.astype(np.int32) + levels) if has_half else (c.astype(np.int32) // 2 + levels // 2)
    offs = st.offsets.cpu().numpy()
    words = st.words.cpu().numpy().view(np.uint16)
    assert len(offs) == n_chunks + 1 and offs[0] == 0 and offs[-1] == words.size
    ks = sorted({0, 1, 4095, 4096, 4097, 32767, 32768, 65535, 65536, 65537, 98303, 98304, n_chunks - 2, n_chunks - 1})
    for k in ks:
        want = R.rans_encode(sym[k * chunk:(k + 1) * chunk], st.freq)
        assert np.array_equal(words[offs[k]:offs[k + 1]], np.array(want, np.uint16)), k
    for k0 in (4090, 98300):
        lens = [len(R.rans_encode(sym[k * chunk:(k + 1) * chunk], st.freq)) for k in range(k0, k0 + 12)]
        assert np.array_equal(np.diff(offs[k0:k0 + 13]), np.array(lens)), k0


@pytest.mark.parametrize("levels", [2, 4, 8, 16])
@pytest.mark.parametrize("n", [1, 15, 16, 17, 4097, 1_000_003, 9 * (1 << 20) * 16 + 9])
def test_histogram_equals_bincount(levels, n):
    """The code histogram (levels 2 and 4 count in packed registers, 8 and 16
    with LDS atomics) equals numpy's count of c + levels, at ragged lengths
    including a remainder past the last 16-byte group and lengths whose
    16-byte groups outnumber the grid's threads several times."""
    from nexusquant_amd.entropy import _code_counts
    print(f"[gpu] rans histogram L={levels} n={n}", flush=True)
    rng = np.random.default_rng(n + levels)
    c = rng.integers(-levels, levels + 1, n).astype(np.int8)
    c[: min(n, 7)] = levels  # the extreme bins, at the head of the stream
    c[-1] = -levels
    got = _code_counts(torch.from_numpy(c).to(DEV), levels)
    want = np.bincount(c.astype(np.int64) + levels, minlength=2 * levels + 1)
    assert np.array_equal(np.asarray(got, np.int64), want)


def test_stream_longer_than_2_31_codes_roundtrips():
    """One stream of 2.5e9 codes whose most frequent code passes 2^31: its
    histogram is counted in pieces, so the frequency table (and the stream)
    stays right.  Every code is checked after the round trip."""
    from nexusquant_amd.entropy import _code_counts, rans_decode, rans_encode
    print("[gpu] rans stream of 2.5e9 codes", flush=True)
    n, levels = 2_500_000_000, 4
    g = torch.Generator(device=DEV).manual_seed(9)
    u = torch.rand(n, device=DEV, generator=g)
    codes = torch.zeros(n, dtype=torch.int8, device=DEV)
    codes[u < 0.04] = 2
    codes[u > 0.96] = -2
    codes[(u > 0.5) & (u < 0.51)] = 4
    del u
    counts = _code_counts(codes, levels)
    assert counts.sum() == n and counts[levels] > (1 << 31)
    assert counts[levels + 2] == int((codes == 2).sum()) and counts[levels + 4] == int((codes == 4).sum())
    st = rans_encode(codes, levels)
    back = rans_decode(st)
    assert torch.equal(back, codes)


def test_encode_many_and_decode_many_equal_the_single_calls():
    """rans_encode_many / rans_decode_many run many tensors' launches on worker
    streams at once: 20 tensors (two groups of at most 16), every level, an
    empty and a one-code tensor, ragged and multi-chunk sizes, a view at an odd
    byte offset (cloned to 16-byte alignment) and per-tensor has_half.  Every
    stream's words, offsets, frequency table and alphabet equal rans_encode's
    on the same tensor, and every stream decodes to its codes."""
    from nexusquant_amd.entropy import rans_decode_many, rans_encode, rans_encode_many
    print("[gpu] rans encode_many / decode_many against single calls", flush=True)
    rng = np.random.default_rng(21)
    sizes = [(0, 8), (1, 8), (4097, 4), (300_001, 8), (70_000, 2), (2048 * 40 + 5, 16), (131_072, 8)]
    tensors, levels = [], []
    for k in range(20):
        n, lv = sizes[k % len(sizes)]
        half = k % 3 != 0
        vals = np.arange(-lv, lv + 1) if half else np.arange(-lv, lv + 1, 2)
        p = np.exp(-0.5 * (vals / (1.0 + lv / 4)) ** 2)
        c = rng.choice(vals, n, p=p / p.sum()).astype(np.int8)
        if k == 5:  # a view 1 byte into its buffer
            t = torch.from_numpy(np.concatenate([np.zeros(1, np.int8), c])).to(DEV)[1:]
        else:
            t = torch.from_numpy(c).to(DEV)
        tensors.append(t)
        levels.append(lv)
    many = rans_encode_many(tensors, levels)
    assert len(many) == len(tensors)
    for t, lv, st in zip(tensors, levels, many):
        one = rans_encode(t, lv)
        assert st.has_half == one.has_half and st.n == one.n and st.shape == one.shape
        assert np.array_equal(st.freq, one.freq)
        assert torch.equal(st.offsets, one.offsets)
        assert torch.equal(st.words, one.words)
    back = rans_decode_many(many)
    for t, b in zip(tensors, back):
        assert torch.equal(b, t)
