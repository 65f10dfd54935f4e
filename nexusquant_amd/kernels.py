"""The compressed-attention primitive of nexusquant.kernels on gfx950.

Mirrors ``nexusquant.kernels.e8_dequant_matmul`` (nexusquant/kernels/e8_triton.py:613-660),
the fused decode + matrix product over the standalone E8 code format (int8
codes ``[K, H_pad]`` with one fp32 scale per row), on the library entry point
``nq_e8_dequant_matmul``.  Same arguments, same assertion messages, float32
``[K, Q_cols]`` result.  The product is exact per term and summed in fp32
(the query is split into three bf16 parts on the matrix cores); the
reference's ``tl.dot`` on fp32 operands may round them to TF32 on its GPUs.

The module's other exports are covered elsewhere: ``e8_nearest_point`` and
``e8_quantize_perhead`` are the E8 rule and per-head quantization fused into
the quantizer (``nq_quantize``).  ``e8_encode`` / ``e8_decode`` are not
provided.
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
