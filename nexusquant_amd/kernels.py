"""The compressed-attention primitive of nexusquant.kernels on gfx950.

Mirrors ``nexusquant.kernels.e8_dequant_matmul`` (nexusquant/kernels/e8_triton.py:613-660),
the fused decode + matrix product over the standalone E8 code format (int8
codes ``[K, H_pad]`` with one fp32 scale per row), on the library entry point
``nq_e8_dequant_matmul``.  Same arguments, same assertion messages, float32
``[K, Q_cols]`` result.  The product is exact per term and summed in fp32
(the query is split into three bf16 parts on the matrix cores); the
reference's ``tl.dot`` on fp32 operands may round them to TF32 on its GPUs.

``e8_nearest_point`` and ``e8_quantize_perhead`` (e8_triton.py:455-522, drop-ins
for E8Lattice.nearest_point / quantize_perhead, e8_lattice.py:27-69, 97-124) run
the reference's E8 rule on ``nq_e8_nearest_point`` / ``nq_e8_quantize_perhead``
in fp32 and return the input's dtype, as the reference's GPU versions do.  The
per-head path follows E8Lattice.quantize_perhead exactly (the reference's Triton
version goes through its int8 encoder, which truncates half-integer points).
``e8_encode`` / ``e8_decode`` are not provided.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib


def e8_dequant_matmul(codes: torch.Tensor, scales: torch.Tensor, query: torch.Tensor,
                      levels: int = 4) -> torch.Tensor:
    """out[k, j] = sum_h (codes[k, h] * scales[k]) * query[h, j] -> float32 [K, Q_cols].

    codes int8 [K, H_pad] (columns H .. H_pad-1 are padding), scales [K],
    query [H, Q_cols] with H <= H_pad <= 256.  ``levels`` is unused (kept for
    the reference's API symmetry).
    """
    assert codes.ndim == 2, "codes must be [K, H_pad]"
    assert query.ndim == 2, "query must be [H, Q_cols]"
    lib = _lib.load()
    for t, what in ((codes, "codes"), (scales, "scales"), (query, "query")):
        _lib.require_device(t, what)
    if codes.dtype != torch.int8:
        raise TypeError(f"codes must be int8, got {codes.dtype}")
    k_rows, h_pad = codes.shape
    h, q_cols = query.shape
    if h > h_pad:
        raise ValueError(f"query has {h} rows but codes only {h_pad} columns")
    if scales.numel() != k_rows:
        raise ValueError(f"scales must hold one value per code row ({k_rows}), got {scales.numel()}")
    codes_c = codes.contiguous()
    if codes_c.data_ptr() % 8:
        codes_c = codes_c.clone()
    scales_c = scales.contiguous().float()
    query_c = query.contiguous().float()
    out = torch.empty(k_rows, q_cols, dtype=torch.float32, device=codes.device)
    if k_rows and q_cols:
        dev = codes.device
        with torch.cuda.device(dev):
            st = lib.nq_e8_dequant_matmul(
                ctypes.c_void_p(codes_c.data_ptr()), ctypes.c_void_p(scales_c.data_ptr()),
                ctypes.c_void_p(query_c.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                k_rows, h_pad, h, q_cols, ctypes.c_void_p(_lib.current_stream_handle(dev)))
        _lib.check(st, "nq_e8_dequant_matmul")
    return out


def _call(lib, name, dev, *args):
    with torch.cuda.device(dev):
        st = getattr(lib, name)(*args, ctypes.c_void_p(_lib.current_stream_handle(dev)))
    _lib.check(st, name)


def e8_nearest_point(x: torch.Tensor) -> torch.Tensor:
    """Nearest relaxed-E8 point of every 8-group: (..., 8) -> same shape and dtype."""
    assert x.shape[-1] == 8, "last dim must be 8"
    lib = _lib.load()
    _lib.require_device(x, "x")
    shape = x.shape
    flat = x.contiguous().view(-1, 8).float()
    if flat.data_ptr() % 16:
        flat = flat.clone()
    out = torch.empty_like(flat)
    if flat.shape[0]:
        _call(lib, "nq_e8_nearest_point", x.device, ctypes.c_void_p(flat.data_ptr()),
              ctypes.c_void_p(out.data_ptr()), flat.shape[0])
    return out.view(shape).to(x.dtype)


def e8_quantize_perhead(x: torch.Tensor, levels: int = 4) -> torch.Tensor:
    """Per-row scale amax / (levels / 2), E8 rule on the padded 8-groups, clamp,
    rescale: (..., head_dim) -> same shape and dtype (computed in fp32)."""
    lib = _lib.load()
    _lib.require_device(x, "x")
    shape = x.shape
    d = shape[-1]
    flat = x.reshape(-1, d).contiguous().float()
    out = torch.empty_like(flat)
    if flat.numel():
        _call(lib, "nq_e8_quantize_perhead", x.device, ctypes.c_void_p(flat.data_ptr()),
              ctypes.c_void_p(out.data_ptr()), flat.shape[0], d, int(levels))
    return out.reshape(shape).to(x.dtype)
