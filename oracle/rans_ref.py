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


def freq_table(symbols: np.ndarray, alphabet: int) -> np.ndarray:
    """Frequencies summing to M (entropy_coder.py:175-243): one per seen symbol,
    the rest shared in proportion to the counts (floored), the shortfall handed
    out by largest fractional part, an excess taken from the rarest symbols."""
    counts = np.bincount(np.asarray(symbols, np.int64), minlength=alphabet).astype(np.int64)
    total = int(counts.sum())
    if total == 0:
        f = np.full(alphabet, M // alphabet, np.int64)
        f[0] += M - int(f.sum())
        return f
    seen = np.flatnonzero(counts)
    f = np.zeros(alphabet, np.int64)
    f[seen] = 1
    budget = M - len(seen)
    if budget > 0:
        share = counts[seen].astype(np.float64) / total * budget
        whole = np.floor(share).astype(np.int64)
        f[seen] += whole
        short = M - int(f.sum())
        if short > 0:
            by_frac = seen[np.argsort(-(share - whole))]
            for i in range(short):
                f[by_frac[i % len(by_frac)]] += 1
        elif short < 0:
            left = -short
            for idx in seen[np.argsort(counts[seen])]:
                take = min(left, int(f[idx]) - 1)
                f[idx] -= take
                left -= take
                if left == 0:
                    break
    elif budget < 0:
        f[:] = 0
        f[seen[np.argsort(-counts[seen])][:M]] = 1
    return f


def encode_e8(quantized: np.ndarray, scales: np.ndarray, levels: int = 8) -> bytes:
    """encode_e8's bytes (entropy_coder.py:360-426): '<IBBI' header, '<III'
    section lengths, u16 alphabet + u16 freqs, fp16 scales, u16 words of one stream."""
    import struct
    flat = np.asarray(quantized, np.float32).reshape(-1, 8)
    sc = np.clip(np.asarray(scales, np.float32).reshape(-1, 1), 1e-8, None)
    sym, has_half, alpha = lattice_to_symbols((flat / sc).ravel(), levels)
    freqs = freq_table(sym, alpha)
    words = rans_encode(sym, freqs)
    freq_b = struct.pack("<H", alpha) + b"".join(struct.pack("<H", int(v)) for v in freqs)
    scale_b = sc.ravel().astype(np.float16).tobytes()
    rans_b = struct.pack(f"<{len(words)}H", *words)
    return (struct.pack("<IBBI", flat.shape[0], levels, int(has_half), len(sym))
            + struct.pack("<III", len(freq_b), len(scale_b), len(rans_b)) + freq_b + scale_b + rans_b)


def decode_e8(blob: bytes):
    """(values fp32 [n_groups, 8], scales fp32) of an encode_e8 container (:429-475)."""
    import struct
    n_groups, levels, has_half, n_sym = struct.unpack_from("<IBBI", blob, 0)
    at = 10
    f_len, s_len, r_len = struct.unpack_from("<III", blob, at)
    at += 12
    (alpha,) = struct.unpack_from("<H", blob, at)
    freqs = np.array(struct.unpack_from(f"<{alpha}H", blob, at + 2), np.int64)
    at += f_len
    sc = np.frombuffer(blob[at:at + s_len], np.float16).astype(np.float32).reshape(-1, 1)
    at += s_len
    words = list(struct.unpack_from(f"<{r_len // 2}H", blob, at))
    sym = rans_decode(words, n_sym, freqs)
    pts = (sym.astype(np.float64) - levels) / 2.0 if has_half else sym.astype(np.float32) - levels // 2
    return pts.astype(np.float32).reshape(n_groups, 8) * sc, sc.ravel()
