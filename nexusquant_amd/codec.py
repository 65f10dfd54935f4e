"""Code-side operations: dequantization, int8 codes, temporal deltas (GPU) and the
host entropy stage (zstd through the system libzstd).

Reference counterparts (side modules in the reference; nothing there calls them):
  vLLM page codes, int8 2p + scale         vllm_backend.py:267-338
  temporal delta + zstd, NQC1 header        compression_accounting.py:23-77
  temporal_delta_encode / compress_indices  temporal_codec.py:30-132
The delta stream layout is the accounting one: [layer][K, V][batch*head][token][coord].
"""

from __future__ import annotations

import ctypes
import ctypes.util
import struct
import threading
from typing import Dict, List, Sequence, Tuple

import numpy as np
import torch

from . import _lib
from .hadamard import hadamard_constant
from .ops import PackedCodes, _addr, _PtrArrays
from .rope import device_merged_table, device_table


def _codes_desc(codes: Sequence[PackedCodes], outs: Sequence[torch.Tensor], rope=None,
                head_dim=None) -> tuple:
    c0 = codes[0]
    head_dim = c0.padded_dim if head_dim is None else head_dim
    b, h, s = c0.scales.shape
    for c in codes:
        if c.scales.shape != c0.scales.shape or c.levels != c0.levels or c.padded_dim != c0.padded_dim:
            raise ValueError("all codes of one launch must share shape and levels")
    dev = c0.scales.device
    staged = _PtrArrays([[c.syms for c in codes], [c.cosets for c in codes], [c.scales for c in codes],
                         list(outs)], dev)
    arrays = staged.arrays
    cos = sin = dm = dp = None
    n_pos = 0
    if rope is not None:
        cos, sin = rope[0], rope[1]
        if len(rope) == 4:
            dm, dp = rope[2], rope[3]
        n_pos = cos.shape[0]
    desc = _lib.CodesDesc(n_tensors=len(codes), batch=b, heads=h, seq=s, head_dim=head_dim,
                          levels=c0.levels, is_key=int(rope is not None), syms=_addr(arrays[0]),
                          cosets=_addr(arrays[1]), scales=_addr(arrays[2]), out=_addr(arrays[3]),
                          rope_cos=_addr(cos), rope_sin=_addr(sin), rope_n_pos=n_pos,
                          rope_sin_minus_cos=_addr(dm), rope_cos_plus_sin=_addr(dp),
                          hadamard_scale=hadamard_constant(c0.padded_dim))
    return desc, staged


def dequantize(codes: Sequence[PackedCodes], rope_base: float = 10000.0,
               rope_scaling=None) -> List[torch.Tensor]:
    """fp16 reconstructions [b, h, s, d] of packed codes (keys re-rotated at 0..s-1)."""
    lib = _lib.load()
    if not codes:
        return []
    c0 = codes[0]
    _lib.require_device(c0.scales, "codes")
    b, h, s = c0.scales.shape
    dev = c0.scales.device
    outs = [torch.empty(b, h, s, c0.head_dim, dtype=torch.float16, device=dev) for _ in codes]
    rope = None
    if c0.is_key:
        rope = device_table(s, c0.head_dim, rope_base, rope_scaling, dev)
        if c0.head_dim != 96:
            rope = rope + device_merged_table(rope[0].shape[0], c0.head_dim, rope_base, rope_scaling, dev)
    desc, staged = _codes_desc(codes, outs, rope, head_dim=c0.head_dim)
    with torch.cuda.device(dev):
        try:
            st = lib.nq_dequantize(ctypes.byref(desc), ctypes.c_void_p(_lib.current_stream_handle(dev)))
        finally:
            staged.release()
    _lib.check(st, "nq_dequantize")
    return outs


def codes_int8(codes: Sequence[PackedCodes], delta: bool = False) -> List[torch.Tensor]:
    """int8 2p codes [b, h, s, D] (or their token deltas) of packed codes."""
    lib = _lib.load()
    if not codes:
        return []
    c0 = codes[0]
    _lib.require_device(c0.scales, "codes")
    b, h, s = c0.scales.shape
    dev = c0.scales.device
    outs = [torch.empty(b, h, s, c0.padded_dim, dtype=torch.int8, device=dev) for _ in codes]
    desc, staged = _codes_desc(codes, outs)
    with torch.cuda.device(dev):
        try:
            st = lib.nq_codes_to_int8(ctypes.byref(desc), int(delta),
                                      ctypes.c_void_p(_lib.current_stream_handle(dev)))
        finally:
            staged.release()
    _lib.check(st, "nq_codes_to_int8")
    return outs


def delta_decode(deltas: Sequence[torch.Tensor]) -> List[torch.Tensor]:
    """Inverse of codes_int8(..., delta=True): prefix sums along tokens (int8 wrap)."""
    lib = _lib.load()
    if not deltas:
        return []
    d0 = deltas[0]
    _lib.require_device(d0, "deltas")
    b, h, s, D = d0.shape
    src = [d.contiguous() for d in deltas]
    outs = [torch.empty_like(d) for d in src]
    staged = _PtrArrays([src, outs], d0.device)
    arrs = staged.arrays
    with torch.cuda.device(d0.device):
        try:
            st = lib.nq_delta_decode(_addr(arrs[0]), _addr(arrs[1]), len(src), b * h, s, D,
                                     ctypes.c_void_p(_lib.current_stream_handle(d0.device)))
        finally:
            staged.release()
    _lib.check(st, "nq_delta_decode")
    return outs


# ---------------------------------------------------------------------------
# Host entropy stage: zstd through the system libzstd (ctypes, no headers needed)
# ---------------------------------------------------------------------------

class Zstd:
    """Minimal binding of libzstd's one-shot API (ZSTD_compress / ZSTD_decompress)."""

    _inst = None
    _lock = threading.Lock()

    def __init__(self):
        name = ctypes.util.find_library("zstd") or "libzstd.so.1"
        L = ctypes.CDLL(name)
        L.ZSTD_compressBound.argtypes = [ctypes.c_size_t]
        L.ZSTD_compressBound.restype = ctypes.c_size_t
        L.ZSTD_compress.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        L.ZSTD_compress.restype = ctypes.c_size_t
        L.ZSTD_decompress.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t]
        L.ZSTD_decompress.restype = ctypes.c_size_t
        L.ZSTD_isError.argtypes = [ctypes.c_size_t]
        L.ZSTD_isError.restype = ctypes.c_uint
        L.ZSTD_getErrorName.argtypes = [ctypes.c_size_t]
        L.ZSTD_getErrorName.restype = ctypes.c_char_p
        L.ZSTD_versionNumber.restype = ctypes.c_uint
        self.lib = L

    @classmethod
    def get(cls) -> "Zstd":
        with cls._lock:
            if cls._inst is None:
                cls._inst = Zstd()
        return cls._inst

    def version(self) -> int:
        return int(self.lib.ZSTD_versionNumber())

    def _check(self, r: int, what: str) -> int:
        if self.lib.ZSTD_isError(r):
            raise RuntimeError(f"{what}: {self.lib.ZSTD_getErrorName(r).decode()}")
        return r

    def compress(self, data, level: int = 3) -> bytes:
        src = np.ascontiguousarray(np.frombuffer(memoryview(data), dtype=np.uint8))
        cap = self.lib.ZSTD_compressBound(src.size)
        dst = np.empty(cap, np.uint8)
        n = self._check(self.lib.ZSTD_compress(dst.ctypes.data, cap, src.ctypes.data, src.size, int(level)),
                        "ZSTD_compress")
        return dst[:n].tobytes()

    def decompress(self, data: bytes, size: int) -> bytes:
        src = np.frombuffer(data, dtype=np.uint8)
        dst = np.empty(size, np.uint8)
        n = self._check(self.lib.ZSTD_decompress(dst.ctypes.data, size, src.ctypes.data, src.size),
                        "ZSTD_decompress")
        if n != size:
            raise RuntimeError(f"ZSTD_decompress produced {n} bytes, expected {size}")
        return dst.tobytes()


# NQC1 header (compression_accounting.py:23-46):
#   magic 'NQC1', n_layers u16, n_heads u16, head_dim u16, n_tokens u32,
#   bits u8, pca_dims u16, use_delta u8, zstd_level u8, 5 reserved bytes.
_NQC1 = struct.Struct("<4sHHHIBHBBxxxxx")
_LEVEL_BITS = {2: 1, 4: 2, 8: 3, 16: 4}


def pack_nqc1(codes_by_layer: Dict[int, Tuple[PackedCodes, PackedCodes]], zstd_level: int = 3) -> dict:
    """Delta + zstd container of a compressed cache: GPU delta stream, host zstd.

    Returns {"blob": bytes, "fp16_bytes": int, "index_bytes": int, "scale_bytes": int,
             "ratio": float}.  Layout: NQC1 header (bits = key bits, the value bits
    follow in the first reserved byte), zstd frame of the int8 deltas in
    [layer][K, V][batch*head][token][coord] order, then fp32 scales.
    """
    layers = sorted(codes_by_layer)
    if not layers:
        raise ValueError("no layers to pack")
    ks, vs = zip(*[codes_by_layer[li] for li in layers])
    k0, v0 = ks[0], vs[0]
    b, h, s = k0.scales.shape
    dk = codes_int8(list(ks), delta=True)
    dv = codes_int8(list(vs), delta=True)
    parts = []
    for a, c in zip(dk, dv):
        parts.append(a.reshape(-1))
        parts.append(c.reshape(-1))
    stream = torch.cat(parts).cpu().numpy().tobytes()
    scales = torch.cat([t.scales.reshape(-1) for pair in zip(ks, vs) for t in pair]).cpu().numpy().tobytes()
    z = Zstd.get().compress(stream, zstd_level)
    header = bytearray(_NQC1.pack(b"NQC1", len(layers), b * h, k0.head_dim, s, _LEVEL_BITS[k0.levels], 0, 1,
                                  zstd_level))
    header[-5] = _LEVEL_BITS[v0.levels]
    blob = bytes(header) + struct.pack("<Q", len(z)) + z + scales
    fp16_bytes = 2 * sum(c.scales.numel() * c.head_dim for c in ks + vs)
    return {"blob": blob, "fp16_bytes": fp16_bytes, "index_bytes": len(z), "scale_bytes": len(scales),
            "raw_index_bytes": len(stream), "ratio": fp16_bytes / len(blob)}


def unpack_nqc1(blob: bytes, device="cuda") -> dict:
    """Inverse of pack_nqc1: int8 2p codes per layer and role, and fp32 scales."""
    magic, n_layers, n_bh, head_dim, n_tokens, kbits, _, use_delta, level = _NQC1.unpack_from(blob, 0)
    if magic != b"NQC1":
        raise ValueError("not an NQC1 container")
    vbits = blob[_NQC1.size - 5]
    D = 1
    while D < head_dim:
        D <<= 1
    off = _NQC1.size
    (zlen,) = struct.unpack_from("<Q", blob, off)
    off += 8
    per = n_bh * n_tokens * D
    raw = Zstd.get().decompress(blob[off:off + zlen], per * 2 * n_layers)
    off += zlen
    deltas = torch.from_numpy(np.frombuffer(raw, np.int8).copy()).to(device)
    deltas = deltas.reshape(n_layers * 2, 1, n_bh, n_tokens, D)
    codes = delta_decode([deltas[i] for i in range(n_layers * 2)]) if use_delta else list(deltas)
    scales = np.frombuffer(blob[off:], np.float32).reshape(n_layers * 2, n_bh, n_tokens)
    return {"codes": codes, "scales": scales, "key_bits": kbits, "value_bits": vbits, "head_dim": head_dim}
