"""Host entropy stage and container layout (no GPU)."""

import os
import struct

import numpy as np

from nexusquant_amd import codec


def test_zstd_roundtrip_and_levels():
    z = codec.Zstd.get()
    rng = np.random.default_rng(0)
    data = (rng.integers(-2, 3, 200000)).astype(np.int8).tobytes() + os.urandom(5000)
    for level in (1, 3, 19):
        c = z.compress(data, level)
        assert z.decompress(c, len(data)) == data
        assert len(c) < len(data)


def test_nqc1_header_is_24_bytes_like_the_reference():
    # compression_accounting.py:23-46 packs '<4sHHHIBHBBxxxxx' (24 bytes)
    assert codec._NQC1.size == 24
    h = codec._NQC1.pack(b"NQC1", 80, 8, 128, 131072, 3, 0, 1, 22)
    assert h[:4] == b"NQC1" and struct.unpack_from("<HHHI", h, 4) == (80, 8, 128, 131072)
