"""Restatement of the reference rANS coder (nexusquant/core/entropy_coder.py).

TEST INFRASTRUCTURE ONLY: tests/ use it to check the device coder; nothing in
nexusquant_amd/ imports it.  Pinned by tests/golden/rans.npz, written by the
reference's own functions.
"""

from __future__ import annotations

from typing import List

import numpy as np

PROB_BITS = 12
M = 1 << PROB_BITS
L = 1 << 16


def lattice_to_symbols(points: np.ndarray, levels: int):
    """(symbols, has_half, alphabet) (entropy_coder.py:35-75)."""
    frac = np.abs(points - np.round(points))
    has_half = bool(np.any(frac > 0.25))
    if has_half:
        alpha = 2 * levels + 1
        sym = np.clip(np.round(points * 2).astype(np.int32) + levels, 0, alpha - 1)
    else:
        alpha = levels + 1
        sym = np.clip(np.round(points).astype(np.int32) + levels // 2, 0, alpha - 1)
    return sym.astype(np.int32), has_half, alpha


def rans_encode(symbols: np.ndarray, freqs: np.ndarray) -> List[int]:
    """16-bit words, first word the high half of the final state (entropy_coder.py:246-295)."""
    cum = np.concatenate([[0], np.cumsum(freqs.astype(np.int64))])
    state = L
    out = []
    for i in range(len(symbols) - 1, -1, -1):
        s = int(symbols[i])
        fs, cs = int(freqs[s]), int(cum[s])
        while state >= (fs << (32 - PROB_BITS)):
            out.append(state & 0xFFFF)
            state >>= 16
        state = (state // fs) * M + (state % fs) + cs
    out.append(state & 0xFFFF)
    state >>= 16
    out.append(state & 0xFFFF)
    out.reverse()
    return out


def rans_decode(words: List[int], n: int, freqs: np.ndarray) -> np.ndarray:
    """Inverse of rans_encode (entropy_coder.py:298-349)."""
    cum = np.concatenate([[0], np.cumsum(freqs.astype(np.int64))])
    c2s = np.zeros(M, np.int32)
    for s in range(len(freqs)):
        c2s[cum[s]:cum[s + 1]] = s
    state = (int(words[0]) << 16) | int(words[1])
    pos = 2
    out = np.zeros(n, np.int32)
    for i in range(n):
        slot = state & (M - 1)
        s = int(c2s[slot])
        state = int(freqs[s]) * (state >> PROB_BITS) + slot - int(cum[s])
        while state < L and pos < len(words):
            state = (state << 16) | int(words[pos])
            pos += 1
        out[i] = s
    return out
