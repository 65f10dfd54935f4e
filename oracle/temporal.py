"""Temporal delta + zlib container of E8 coordinates, restated in numpy.

Test infrastructure only: tests/, the smoke check and the CPU baseline of
bench.py use it as the checker; the product path never calls it.

Follows the reference's nexusquant/core/temporal_codec.py (v0.5.0), zlib
branch (the `zstandard` package is absent here, so the reference writes zlib):
  delta_encode  temporal_codec.py:30-52   row-wise token deltas, first row raw,
                                          skipped unless n_tokens | n and the
                                          row width is a multiple of 8
  delta_decode  temporal_codec.py:55-73   running sums, skipped unless n_tokens | n
  compress      temporal_codec.py:76-106  '<IIBBxx' header + zlib(min(level, 9))
  decompress    temporal_codec.py:109-132
Pinned by tests/golden/temporal_codec.npz (bytes written by the reference) and
by element-by-element loops on small inputs (tests/test_oracle_temporal.py).
"""

from __future__ import annotations

import struct
import zlib

import numpy as np

HEADER = struct.Struct("<IIBBxx")


def delta_encode(coords: np.ndarray, n_tokens: int) -> np.ndarray:
    n_total = len(coords)
    n_per = n_total // n_tokens
    if n_total % n_tokens != 0 or n_per % 8 != 0:
        return coords
    rows = coords.reshape(n_tokens, n_per)
    out = np.zeros_like(rows)
    out[0] = rows[0]
    out[1:] = rows[1:] - rows[:-1]
    return out.ravel().astype(np.int8)


def delta_decode(delta: np.ndarray, n_tokens: int) -> np.ndarray:
    n_total = len(delta)
    n_per = n_total // n_tokens
    if n_total % n_tokens != 0:
        return delta
    rows = delta.reshape(n_tokens, n_per)
    return np.cumsum(rows, axis=0, dtype=np.int64).astype(np.int8).ravel()


def compress(coords: np.ndarray, n_tokens: int, use_delta: bool = True, level: int = 22) -> bytes:
    data = coords.astype(np.int8)
    if use_delta:
        data = delta_encode(data, n_tokens)
    payload = zlib.compress(data.tobytes(), min(level, 9))
    return HEADER.pack(len(coords), n_tokens, int(use_delta), 0) + payload


def decompress(data: bytes) -> np.ndarray:
    n_elements, n_tokens, use_delta, compressor = struct.unpack_from("<IIBB", data)
    if compressor != 0:
        raise ValueError("the oracle restates the zlib branch only")
    coords = np.frombuffer(zlib.decompress(data[HEADER.size:]), dtype=np.int8).copy()
    if use_delta:
        coords = delta_decode(coords, n_tokens)
    return coords
