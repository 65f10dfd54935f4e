"""Packed lattice-code format, restated in numpy.  Test infrastructure only.

The reference never stores codes from its pipeline; its storage format is the
vLLM page format, int8 code = round(2p) with a per-vector scale
(vllm_backend.py:267-338), and its delta stream is int8 coordinates with
token-to-token differences (compression_accounting.py:49-77).  The packed
format below is this build's own, lossless for the relaxed E8 points:

  per row of D padded coordinates (G = D/8 groups, C = D/32):
    * symbols in [0, L], b = bits_for(L) bits each: sym = p + L/2 on the
      integer coset; on the half coset sym = floor(p) + L/2 when L/2 is even
      and ceil(p) + L/2 when L/2 is odd (the clamp folds one edge point onto
      +L/2, respectively -L/2, because rint rounds half to even)
      (L=2:2, L=4:3, L=8:4, L=16:5).  The G groups occupy G*b bytes; slot k
      (b bytes at byte offset k*b, symbol j at bit j*b, little endian) holds
      group g = 4*(k mod C) + (k div C).
    * coset bitmap: D/64 bytes, bit g set when group g is a half-integer point.
    * scale: fp32.
  decode (2p form): integer coset 2*sym - L; half coset min(2*sym - L + 1, L)
  when L/2 is even, max(2*sym - L - 1, -L) when L/2 is odd.
"""

from __future__ import annotations

import numpy as np


def bits_for(levels: int) -> int:
    return {2: 2, 4: 3, 8: 4, 16: 5}[levels]


def slot_to_group(D: int) -> np.ndarray:
    G, C = D // 8, D // 32
    k = np.arange(G)
    return 4 * (k % C) + (k // C)


def pack_symbols(sym: np.ndarray, levels: int) -> np.ndarray:
    """sym [n, D] uint8 -> packed [n, D/8*b] uint8."""
    n, D = sym.shape
    b = bits_for(levels)
    G = D // 8
    groups = sym.reshape(n, G, 8).astype(np.uint64)
    vals = np.zeros((n, G), np.uint64)
    for j in range(8):
        vals |= groups[:, :, j] << np.uint64(b * j)
    vals = vals[:, slot_to_group(D)]                      # slot order
    out = np.zeros((n, G, b), np.uint8)
    for byte in range(b):
        out[:, :, byte] = ((vals >> np.uint64(8 * byte)) & np.uint64(0xFF)).astype(np.uint8)
    return out.reshape(n, G * b)


def unpack_symbols(packed: np.ndarray, levels: int, D: int) -> np.ndarray:
    n = packed.shape[0]
    b = bits_for(levels)
    G = D // 8
    by = packed.reshape(n, G, b).astype(np.uint64)
    vals = np.zeros((n, G), np.uint64)
    for byte in range(b):
        vals |= by[:, :, byte] << np.uint64(8 * byte)
    nat = np.empty_like(vals)
    nat[:, slot_to_group(D)] = vals
    mask = np.uint64((1 << b) - 1)
    sym = np.zeros((n, G, 8), np.uint8)
    for j in range(8):
        sym[:, :, j] = ((nat >> np.uint64(b * j)) & mask).astype(np.uint8)
    return sym.reshape(n, D)


def pack_cosets(coset: np.ndarray) -> np.ndarray:
    """coset [n, G] 0/1 -> bitmap [n, G/8] uint8 (bit g of the little-endian row)."""
    n, G = coset.shape
    return np.packbits(coset.astype(np.uint8).reshape(n, G // 8, 8), axis=-1,
                       bitorder="little").reshape(n, G // 8)


def unpack_cosets(bitmap: np.ndarray, G: int) -> np.ndarray:
    n = bitmap.shape[0]
    return np.unpackbits(bitmap.reshape(n, G // 8, 1), axis=-1,
                         bitorder="little").reshape(n, G)


def codes_2p(sym: np.ndarray, coset: np.ndarray, levels: int) -> np.ndarray:
    """(sym [n, D], coset [n, G]) -> int8 2p [n, D] (vLLM code convention)."""
    c = np.repeat(coset.astype(bool), 8, axis=1)
    v = 2 * sym.astype(np.int16) - levels
    if (levels // 2) % 2 == 0:
        half = np.minimum(v + 1, levels)
    else:
        half = np.maximum(v - 1, -levels)
    return np.where(c, half, v).astype(np.int8)


def decode_points(sym: np.ndarray, coset: np.ndarray, levels: int) -> np.ndarray:
    """(sym, coset) -> lattice points p (float32)."""
    return codes_2p(sym, coset, levels).astype(np.float32) / 2


def delta_tokens(codes: np.ndarray) -> np.ndarray:
    """[streams, tokens, coords] int8 -> token deltas with int8 wrap."""
    x = codes.astype(np.int8)
    out = np.empty_like(x)
    out[:, :1] = x[:, :1]
    out[:, 1:] = x[:, 1:] - x[:, :-1]
    return out


def undelta_tokens(delta: np.ndarray) -> np.ndarray:
    return np.cumsum(delta.astype(np.int8), axis=1, dtype=np.int64).astype(np.int8)
