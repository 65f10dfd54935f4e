"""Temporal delta + zlib / zstd container of E8 lattice coordinates.

Mirror of the reference's nexusquant/core/temporal_codec.py (v0.5.0): the same
functions, arguments, header and payload bytes.  The token deltas and their
inverse run on the GPU (nq_delta_encode / nq_delta_decode); the byte
compressor runs on the host (zlib from Python, zstd through the system
libzstd).

Container (temporal_codec.py:93-104): a 12-byte header struct '<IIBBxx' =
n_elements u32, n_tokens u32, use_delta u8, compressor u8 (0 zlib, 1 zstd) and
two zero pad bytes, then the compressed int8 stream.  The coordinates are a
flat array read as [n_tokens][n_total / n_tokens] rows; the delta runs down
the token axis.

Reference behaviour kept as it is:
  * the delta applies only when n_tokens divides n_total and the row width is
    a multiple of 8 (temporal_codec.py:44-45); otherwise the raw coordinates
    are stored, with use_delta still written as given;
  * decompression undoes the delta whenever n_tokens divides n_total
    (temporal_codec.py:67-68), without the multiple-of-8 test, so a container
    written with use_delta and a row width that is not a multiple of 8 decodes
    to the running sums of the raw coordinates, as the reference's does;
  * the compressor is zlib at min(level, 9) unless zstd is asked for; the
    reference picks zstd whenever the `zstandard` package is importable, which
    it is not in this image, so its bytes here are zlib's;
  * n_tokens == 0 with the delta raises ZeroDivisionError, as Python's
    integer division does in the reference.
Departures: zstd containers (compressor 1) decode through libzstd even without
the `zstandard` package (the reference then fails inside zlib), and only
one-dimensional integer (or bool) coordinate arrays are accepted.

Inputs may be numpy arrays (the reference's type; results come back as numpy)
or int tensors on a ROCm device (results stay on the device).
"""

from __future__ import annotations

import ctypes
import struct
import zlib
from typing import Optional, Union

import numpy as np
import torch

from . import _lib
from .ops import _addr, _PtrArrays

HEADER = struct.Struct("<IIBBxx")   # temporal_codec.py:103
ZLIB, ZSTD = 0, 1
_INT32_MAX = (1 << 31) - 1

Array = Union[np.ndarray, torch.Tensor]


def _length(coords: Array) -> int:
    if coords.ndim != 1:
        raise ValueError(f"coords must be one-dimensional, got shape {tuple(coords.shape)}")
    return int(coords.shape[0])


def _device_int8(coords: Array) -> torch.Tensor:
    """coords as a contiguous int8 tensor on a ROCm device (numpy input is uploaded)."""
    if torch.is_tensor(coords):
        _lib.require_device(coords, "coords")
        if coords.dtype.is_floating_point or coords.dtype.is_complex:
            raise TypeError(f"coords must be integer, got {coords.dtype}")
        return coords.to(torch.int8).contiguous()
    a = np.asarray(coords)
    if a.dtype.kind not in "iub":
        raise TypeError(f"coords must be integer, got {a.dtype}")
    if not torch.cuda.is_available():
        raise _lib.NexusQuantError("nexusquant_amd runs on MI355X (ROCm) devices only; no GPU is visible")
    return torch.from_numpy(np.ascontiguousarray(a.astype(np.int8, copy=False))).to(torch.cuda.current_device())


def _like(template: Array, t: torch.Tensor) -> Array:
    return t if torch.is_tensor(template) else t.cpu().numpy()


def _aligned(t: torch.Tensor, width: int) -> torch.Tensor:
    return t if t.data_ptr() % width == 0 else t.clone()


def _token_delta(x: torch.Tensor, n_tokens: int, n_per: int, encode: bool) -> torch.Tensor:
    """GPU delta (encode) or running sum (decode) of x read as [n_tokens][n_per] int8."""
    if x.numel() == 0:
        return x.clone()
    if n_tokens == 1:
        return x.clone()          # one row: both directions are the identity
    if n_tokens > _INT32_MAX or n_per > _INT32_MAX:
        raise ValueError(f"{n_tokens} tokens of {n_per} coordinates exceed the kernels' int32 geometry")
    width = 16 if n_per % 16 == 0 else 4 if n_per % 4 == 0 else 1
    x = _aligned(x, width)
    out = torch.empty_like(x)
    lib = _lib.load()
    fn = lib.nq_delta_encode if encode else lib.nq_delta_decode
    staged = _PtrArrays([[x], [out]], x.device)
    arrs = staged.arrays
    with torch.cuda.device(x.device):
        try:
            st = fn(_addr(arrs[0]), _addr(arrs[1]), 1, 1, n_tokens, n_per,
                    ctypes.c_void_p(_lib.current_stream_handle(x.device)))
        finally:
            staged.release()
    _lib.check(st, "nq_delta_encode" if encode else "nq_delta_decode")
    return out


def temporal_delta_encode(coords: Array, n_tokens: int) -> Array:
    """Token deltas of flat E8 coordinates, first token raw (temporal_codec.py:30-52).

    Returns `coords` itself when n_tokens does not divide its length or the
    row width is not a multiple of 8.
    """
    n_total = _length(coords)
    if n_tokens < 0:
        raise ValueError("n_tokens must be non-negative")
    n_per = n_total // n_tokens          # ZeroDivisionError at 0, as in the reference
    if n_total % n_tokens != 0 or n_per % 8 != 0:
        return coords
    return _like(coords, _token_delta(_device_int8(coords), n_tokens, n_per, encode=True))


def temporal_delta_decode(delta: Array, n_tokens: int) -> Array:
    """Running sums down the token axis, int8 wrap (temporal_codec.py:55-73).

    Returns `delta` itself when n_tokens does not divide its length.
    """
    n_total = _length(delta)
    if n_tokens < 0:
        raise ValueError("n_tokens must be non-negative")
    n_per = n_total // n_tokens
    if n_total % n_tokens != 0:
        return delta
    return _like(delta, _token_delta(_device_int8(delta), n_tokens, n_per, encode=False))


def _host_bytes(data: Array) -> bytes:
    if torch.is_tensor(data):
        return data.to(torch.int8).cpu().numpy().tobytes()
    return np.ascontiguousarray(np.asarray(data).astype(np.int8, copy=False)).tobytes()


def compress_indices(coords: Array, n_tokens: int, use_delta: bool = True, level: int = 22,
                     compressor: Optional[str] = None) -> bytes:
    """Compressed container of int8 lattice coordinates (temporal_codec.py:76-106).

    compressor: None or "zlib" writes zlib at min(level, 9) (what the
    reference writes without the `zstandard` package); "zstd" writes a zstd
    frame at min(level, 22) through libzstd.
    """
    n_total = _length(coords)
    if torch.is_tensor(coords):
        _lib.require_device(coords, "coords")
    data: Array = coords
    if use_delta:
        data = temporal_delta_encode(coords, n_tokens)
    raw = _host_bytes(data)
    if compressor in (None, "zlib"):
        payload = zlib.compress(raw, min(level, 9))
        kind = ZLIB
    elif compressor == "zstd":
        from .codec import Zstd
        payload = Zstd.get().compress(raw, min(level, 22))
        kind = ZSTD
    else:
        raise ValueError(f"compressor must be None, 'zlib' or 'zstd', got {compressor!r}")
    return HEADER.pack(n_total, n_tokens, int(use_delta), kind) + payload


def decompress_indices(data: bytes, device=None) -> Array:
    """int8 coordinates of a compress_indices container (temporal_codec.py:109-132).

    Returns a numpy array, as the reference does, or a device tensor when
    `device` is given (no copy back to the host).
    """
    n_elements, n_tokens, use_delta, kind = struct.unpack_from("<IIBB", data)
    payload = bytes(data[HEADER.size:])
    if kind == ZSTD:
        from .codec import Zstd
        raw = Zstd.get().decompress(payload, n_elements)
    else:
        raw = zlib.decompress(payload)
    host = np.frombuffer(raw, dtype=np.int8)
    if not use_delta:
        coords = torch.from_numpy(host.copy())
        return coords.to(device) if device is not None else coords.numpy()
    if device is None and not torch.cuda.is_available():
        raise _lib.NexusQuantError("nexusquant_amd runs on MI355X (ROCm) devices only; no GPU is visible")
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    x = torch.from_numpy(host.copy()).to(dev)
    out = temporal_delta_decode(x, n_tokens)
    return out if device is not None else out.cpu().numpy()


def measure_compression(coords: Array, n_tokens: int, fp16_bytes: int, scale_bytes: int) -> dict:
    """Container sizes and ratios with and without the delta (temporal_codec.py:135-157).

    Asserts that each container decodes back to coords, as the reference does.
    """
    results = {}
    on_device = torch.is_tensor(coords)
    for use_delta in (False, True):
        label = "delta" if use_delta else "raw"
        blob = compress_indices(coords, n_tokens, use_delta=use_delta)
        total = len(blob) + scale_bytes
        results[f"{label}_bytes"] = len(blob)
        results[f"{label}_total"] = total
        results[f"{label}_ratio"] = fp16_bytes / total
        if on_device:
            decoded = decompress_indices(blob, device=coords.device)
            same = decoded.shape == coords.shape and bool(torch.equal(decoded, coords.to(torch.int8)))
        else:
            decoded = decompress_indices(blob)
            same = np.array_equal(coords, decoded)
        assert same, f"Round-trip failed for {label}!"
    return results
