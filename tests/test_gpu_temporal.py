"""GPU parity of the temporal codec: the reference's container bytes, and the
delta kernels against the oracle at sizes that take the chunked scan."""

import ctypes

import numpy as np
import pytest
import torch

from conftest import load_golden
from golden.make_golden_cases import CASE_NAMES
from oracle import codes as OC
from oracle import temporal as OT

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def case(name):
    f = load_golden("temporal_codec")
    n_tokens, use_delta, level = (int(v) for v in f[f"{name}_meta"])
    return (f[f"{name}_coords"], n_tokens, bool(use_delta), level, f[f"{name}_blob"].tobytes(),
            f[f"{name}_decoded"], f.get(f"{name}_delta"))


@pytest.mark.parametrize("name", CASE_NAMES)
def test_container_bytes_match_the_reference(name):
    from nexusquant_amd import temporal_codec as TC
    print(f"[gpu] temporal codec fixture {name}", flush=True)
    coords, n_tokens, use_delta, level, blob, decoded, delta = case(name)
    assert TC.compress_indices(coords, n_tokens, use_delta=use_delta, level=level) == blob
    out = TC.decompress_indices(blob)
    assert isinstance(out, np.ndarray) and out.dtype == np.int8 and np.array_equal(out, decoded)
    dev = TC.decompress_indices(blob, device=DEV)
    assert dev.is_cuda and np.array_equal(dev.cpu().numpy(), decoded)
    t = torch.from_numpy(coords).to(DEV)
    assert TC.compress_indices(t, n_tokens, use_delta=use_delta, level=level) == blob
    if delta is not None:
        assert np.array_equal(TC.temporal_delta_encode(coords.astype(np.int8), n_tokens), delta)


def test_measure_compression_matches_the_reference():
    from nexusquant_amd import temporal_codec as TC
    f = load_golden("temporal_codec")
    want = dict(zip([str(k) for k in f["measure_keys"]], f["measure_values"]))
    got = TC.measure_compression(f["delta_coords"], 48, fp16_bytes=48 * 64 * 2, scale_bytes=48 * 8 * 2)
    assert sorted(got) == sorted(want)
    for k in want:
        assert got[k] == pytest.approx(want[k], rel=1e-12)


SHAPES = [(4096, 1024), (100000, 8), (1000, 24), (333, 5), (17, 4096), (64, 65536), (2, 8), (4, 1000),
          (7, 262144), (5000, 16)]


@pytest.mark.parametrize("n_tokens,n_per", SHAPES)
def test_delta_kernels_against_oracle(n_tokens, n_per):
    from nexusquant_amd import temporal_codec as TC
    print(f"[gpu] temporal delta tokens={n_tokens} width={n_per}", flush=True)
    rng = np.random.default_rng(n_tokens + n_per)
    x = rng.integers(-128, 128, n_tokens * n_per).astype(np.int8)
    xt = torch.from_numpy(x).to(DEV)
    enc = TC.temporal_delta_encode(xt, n_tokens)
    want = OT.delta_encode(x, n_tokens)
    assert np.array_equal(enc.cpu().numpy(), want)
    dec = TC.temporal_delta_decode(xt, n_tokens)      # decode runs for any width n_tokens divides
    assert np.array_equal(dec.cpu().numpy(), OT.delta_decode(x, n_tokens))
    if n_per % 8 == 0:
        assert torch.equal(TC.temporal_delta_decode(enc, n_tokens), xt)


def test_container_roundtrip_at_cache_size():
    # a 16 MiB coordinate stream ([4096 tokens][4096 coords]) through both
    # compressors, against the oracle's zlib bytes
    from nexusquant_amd import temporal_codec as TC
    print("[gpu] temporal codec 16 MiB round trip", flush=True)
    rng = np.random.default_rng(5)
    steps = rng.integers(-1, 2, size=(4096, 4096), dtype=np.int8)
    coords = np.clip(np.cumsum(steps, axis=0, dtype=np.int16), -8, 8).astype(np.int8).ravel()
    t = torch.from_numpy(coords).to(DEV)
    blob = TC.compress_indices(t, 4096, level=1)
    assert blob == OT.compress(coords, 4096, True, 1)
    assert torch.equal(TC.decompress_indices(blob, device=DEV), t)
    z = TC.compress_indices(t, 4096, level=3, compressor="zstd")
    assert z[9] == 1 and torch.equal(TC.decompress_indices(z, device=DEV), t)


def _ptrs(ts):
    return torch.tensor([x.data_ptr() for x in ts], dtype=torch.int64, device=DEV)


@pytest.mark.parametrize("streams,seq,coords", [(5, 300, 64), (3, 70, 12), (2, 2000, 3), (1, 513, 4096)])
def test_c_abi_streams_tensors_and_in_place(streams, seq, coords):
    # several tensors and streams per call, and nq_delta_decode with out == deltas
    from nexusquant_amd import _lib
    print(f"[gpu] delta C-ABI streams={streams} seq={seq} coords={coords}", flush=True)
    lib = _lib.load()
    rng = np.random.default_rng(streams * seq + coords)
    xs = [rng.integers(-128, 128, (streams, seq, coords)).astype(np.int8) for _ in range(3)]
    src = [torch.from_numpy(x).to(DEV) for x in xs]
    enc = [torch.empty_like(s) for s in src]
    ps, pe = _ptrs(src), _ptrs(enc)
    st = lib.nq_delta_encode(ctypes.c_void_p(ps.data_ptr()), ctypes.c_void_p(pe.data_ptr()), 3, streams, seq,
                             coords, None)
    _lib.check(st, "nq_delta_encode")
    torch.cuda.synchronize()
    for x, e in zip(xs, enc):
        assert np.array_equal(e.cpu().numpy(), OC.delta_tokens(x))
    st = lib.nq_delta_decode(ctypes.c_void_p(pe.data_ptr()), ctypes.c_void_p(pe.data_ptr()), 3, streams, seq,
                             coords, None)
    _lib.check(st, "nq_delta_decode")
    torch.cuda.synchronize()
    for s, e in zip(src, enc):
        assert torch.equal(e, s)
