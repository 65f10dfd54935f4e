"""Temporal delta + zlib container: the oracle against the reference's bytes,
element loops, and the host side of nexusquant_amd.temporal_codec (no GPU)."""

import struct
import zlib

import numpy as np
import pytest

from conftest import load_golden
from golden.make_golden_cases import CASE_NAMES
from oracle import temporal as OT

FIX = None


def fixture():
    global FIX
    if FIX is None:
        FIX = load_golden("temporal_codec")
    return FIX


def case(name):
    f = fixture()
    n_tokens, use_delta, level = (int(v) for v in f[f"{name}_meta"])
    return f[f"{name}_coords"], n_tokens, bool(use_delta), level, f[f"{name}_blob"].tobytes(), f[f"{name}_decoded"]


@pytest.mark.parametrize("name", CASE_NAMES)
def test_oracle_writes_and_reads_the_reference_bytes(name):
    coords, n_tokens, use_delta, level, blob, decoded = case(name)
    assert OT.compress(coords, n_tokens, use_delta, level) == blob
    out = OT.decompress(blob)
    assert out.dtype == np.int8 and np.array_equal(out, decoded)
    if use_delta:
        assert np.array_equal(OT.delta_encode(coords.astype(np.int8), n_tokens), fixture()[f"{name}_delta"])


def _wrap(v):
    return ((v + 128) % 256) - 128


@pytest.mark.parametrize("n_tokens,n_per", [(5, 8), (3, 16), (7, 24), (1, 8)])
def test_oracle_delta_against_element_loops(n_tokens, n_per):
    rng = np.random.default_rng(n_tokens * 100 + n_per)
    x = rng.integers(-128, 128, n_tokens * n_per).astype(np.int8)
    d = OT.delta_encode(x, n_tokens)
    for t in range(n_tokens):
        for c in range(n_per):
            i = t * n_per + c
            want = int(x[i]) if t == 0 else _wrap(int(x[i]) - int(x[i - n_per]))
            assert int(d[i]) == want
    back = OT.delta_decode(d, n_tokens)
    for c in range(n_per):
        acc = 0
        for t in range(n_tokens):
            acc = _wrap(acc + int(d[t * n_per + c]))
            assert int(back[t * n_per + c]) == acc
    assert np.array_equal(back, x)


def test_reference_quirk_is_in_the_fixture():
    # rows of 12 bytes: the encoder stores raw coordinates, the decoder still
    # takes running sums (temporal_codec.py:44-45 against :67-68)
    coords, n_tokens, _, _, blob, decoded = case("width12")
    assert struct.unpack_from("<IIBB", blob) == (480, 40, 1, 0)
    assert np.array_equal(np.frombuffer(zlib.decompress(blob[12:]), np.int8), coords)
    assert not np.array_equal(decoded, coords)
    assert np.array_equal(decoded, np.cumsum(coords.reshape(40, 12), 0).astype(np.int8).ravel())


def test_reference_measurement_values():
    f = fixture()
    keys = [str(k) for k in f["measure_keys"]]
    got = dict(zip(keys, f["measure_values"]))
    coords = f["delta_coords"]
    for use_delta, label in ((False, "raw"), (True, "delta")):
        n = len(OT.compress(coords, 48, use_delta))
        assert got[f"{label}_bytes"] == n
        assert got[f"{label}_total"] == n + 48 * 8 * 2
        assert got[f"{label}_ratio"] == pytest.approx(48 * 64 * 2 / (n + 48 * 8 * 2), rel=1e-12)


# --- host side of the product module (paths that need no GPU) ---------------

def test_header_layout_matches_the_reference():
    from nexusquant_amd import temporal_codec as TC
    assert TC.HEADER.size == 12 and TC.HEADER.format == "<IIBBxx"


@pytest.mark.parametrize("name", ["raw", "ragged"])
def test_product_writes_reference_bytes_when_no_delta_runs(name):
    # use_delta=False, or a length n_tokens does not divide: zlib only, no device work
    from nexusquant_amd import temporal_codec as TC
    coords, n_tokens, use_delta, level, blob, decoded = case(name)
    assert TC.compress_indices(coords, n_tokens, use_delta=use_delta, level=level) == blob
    if not use_delta:
        out = TC.decompress_indices(blob)
        assert isinstance(out, np.ndarray) and out.dtype == np.int8 and np.array_equal(out, decoded)


def test_product_zstd_container_roundtrip_without_delta():
    from nexusquant_amd import temporal_codec as TC
    coords = case("delta")[0]
    blob = TC.compress_indices(coords, 48, use_delta=False, compressor="zstd")
    assert struct.unpack_from("<IIBB", blob) == (len(coords), 48, 0, 1)
    assert np.array_equal(TC.decompress_indices(blob), coords)
    with pytest.raises(ValueError):
        TC.compress_indices(coords, 48, use_delta=False, compressor="lz4")


def test_product_errors_match_the_reference():
    from nexusquant_amd import temporal_codec as TC
    coords = case("delta")[0]
    with pytest.raises(ZeroDivisionError):
        TC.compress_indices(coords, 0)
    with pytest.raises(ValueError):
        TC.temporal_delta_encode(coords.reshape(48, 64), 48)
    with pytest.raises(TypeError):
        TC.temporal_delta_encode(coords.astype(np.float32), 48)


def test_product_delta_has_no_cpu_fallback():
    import torch
    from nexusquant_amd import _lib
    from nexusquant_amd import temporal_codec as TC
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(_lib.NexusQuantError):
        TC.compress_indices(case("delta")[0], 48)
    with pytest.raises(_lib.NexusQuantError):
        TC.decompress_indices(case("delta")[4])
