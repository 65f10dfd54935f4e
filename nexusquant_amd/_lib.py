"""ctypes binding of the gfx950 library (nexusquant_amd/lib/libnqamd.so).

The library is the only compute path: when it is missing, or the tensors are
not on a ROCm device, every entry point raises instead of falling back.
"""

from __future__ import annotations

import ctypes
import os
import threading

from .build import LIB_PATH, source_hash

NQ_F16, NQ_BF16, NQ_F32 = 0, 1, 2
NQ_KEEP_ZERO, NQ_KEEP_WRITE_KEPT, NQ_KEEP_WRITE_EVICTED = 0, 1, 2
ABI_VERSION = 8  # NQ_ABI_VERSION of the header these bindings mirror
_P = ctypes.c_void_p


class QuantDesc(ctypes.Structure):
    """Mirror of nq_quant_desc in include/nexusquant_amd.h."""
    _fields_ = [
        ("n_tensors", ctypes.c_int32),
        ("batch", ctypes.c_int32), ("heads", ctypes.c_int32), ("seq_in", ctypes.c_int32),
        ("seq_out", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("dtype", ctypes.c_int32), ("levels", ctypes.c_int32), ("is_key", ctypes.c_int32),
        ("keep_mode", ctypes.c_int32),
        ("src", _P), ("recon", _P), ("syms", _P), ("cosets", _P), ("scales", _P),
        ("gather", _P), ("keep", _P), ("rope_cos", _P), ("rope_sin", _P),
        ("rope_n_pos", ctypes.c_int64),
        ("hadamard_scale", ctypes.c_float), ("reserved_f", ctypes.c_float),
        ("rope_sin_minus_cos", _P), ("rope_cos_plus_sin", _P),
        ("order", _P), ("n_kept", _P),
    ]


class CodesDesc(ctypes.Structure):
    """Mirror of nq_codes_desc in include/nexusquant_amd.h."""
    _fields_ = [
        ("n_tensors", ctypes.c_int32),
        ("batch", ctypes.c_int32), ("heads", ctypes.c_int32), ("seq", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("levels", ctypes.c_int32), ("is_key", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("syms", _P), ("cosets", _P), ("scales", _P), ("out", _P),
        ("rope_cos", _P), ("rope_sin", _P), ("rope_n_pos", ctypes.c_int64),
        ("hadamard_scale", ctypes.c_float), ("reserved_f", ctypes.c_float),
        ("rope_sin_minus_cos", _P), ("rope_cos_plus_sin", _P),
    ]


class MergeDesc(ctypes.Structure):
    """Mirror of nq_merge_desc in include/nexusquant_amd.h."""
    _fields_ = [
        ("n_tensors", ctypes.c_int32), ("batch", ctypes.c_int32), ("heads", ctypes.c_int32),
        ("seq", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("dtype", ctypes.c_int32),
        ("src", _P), ("dst", _P), ("keep", _P), ("kept_idx", _P), ("n_kept", _P), ("importance", _P),
        ("centroids", _P), ("survivor", _P), ("workspace", _P), ("workspace_bytes", ctypes.c_int64),
    ]


class PageDesc(ctypes.Structure):
    """Mirror of nq_page_desc in include/nexusquant_amd.h."""
    _fields_ = [
        ("n_pages", ctypes.c_int32),
        ("heads", ctypes.c_int32), ("tokens", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("dtype", ctypes.c_int32), ("levels", ctypes.c_int32), ("is_key", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("src", _P), ("positions", _P), ("codes", _P), ("scales", _P), ("out", _P),
        ("rope_cos", _P), ("rope_sin", _P), ("rope_sin_minus_cos", _P), ("rope_cos_plus_sin", _P),
        ("rope_n_pos", ctypes.c_int64),
        ("hadamard_scale", ctypes.c_float), ("reserved_f", ctypes.c_float),
    ]


class AttnDesc(ctypes.Structure):
    """Mirror of nq_attn_desc in include/nexusquant_amd.h."""
    _fields_ = [
        ("batch", ctypes.c_int32), ("q_heads", ctypes.c_int32), ("kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("q_dtype", ctypes.c_int32), ("n_chunks", ctypes.c_int32),
        ("query", _P), ("out", _P), ("units", _P),
        ("chunk_units", _P), ("chunk_row", _P), ("chunk_tokens", _P), ("row_chunks", _P),
        ("rope_cos", _P), ("rope_sin", _P), ("rope_sin_minus_cos", _P), ("rope_cos_plus_sin", _P),
        ("rope_n_pos", ctypes.c_int64),
        ("hadamard_scale", ctypes.c_float), ("scale_divisor", ctypes.c_float),
        ("workspace", _P), ("workspace_bytes", ctypes.c_int64),
    ]


# Every exported symbol, with (argtypes, restype).  tests/test_abi.py checks
# that this list and include/nexusquant_amd.h agree and that the library
# exports all of them.
_I32, _I64, _F32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_float

SIGNATURES = {
    "nq_abi_version": ([], ctypes.c_int),
    "nq_last_error": ([], ctypes.c_char_p),
    "nq_source_hash": ([], ctypes.c_char_p),
    "nq_quantize": ([ctypes.POINTER(QuantDesc), _P], ctypes.c_int),
    "nq_score_keykey_workspace": ([_I32, _I32, _I32, _I32], _I64),
    "nq_score_keykey": ([_P, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _P, _P, _I64, _P], ctypes.c_int),
    "nq_score_keykey_noalloc": ([_P, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _P, _P], ctypes.c_int),
    "nq_keep_mask": ([_P, _I32, _I32, _I32, _I32, _I32, _P, _I32, _P, _P, _P, _P], ctypes.c_int),
    "nq_gather_rows": ([_P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _P, _P, _P], ctypes.c_int),
    "nq_dequantize": ([ctypes.POINTER(CodesDesc), _P], ctypes.c_int),
    "nq_codes_to_int8": ([ctypes.POINTER(CodesDesc), _I32, _P], ctypes.c_int),
    "nq_delta_encode": ([_P, _P, _I32, _I32, _I32, _I32, _P], ctypes.c_int),
    "nq_delta_decode": ([_P, _P, _I32, _I32, _I32, _I32, _P], ctypes.c_int),
    "nq_score_real_workspace": ([_I32, _I32, _I32], _I64),
    "nq_score_real": ([_P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _I32, _P, _P, _P, _I64, _P],
                      ctypes.c_int),
    "nq_attention_real_workspace": ([_I32, _I32, _I32, _I32, _I32], _I64),
    "nq_attention_real": ([_P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _I32, _P, _P, _P, _P, _I64, _P],
                          ctypes.c_int),
    "nq_rans_histogram": ([_P, _I64, _I32, _P, _P], ctypes.c_int),
    "nq_rans_scratch_words": ([_I64, _I32], _I64),
    "nq_rans_encode": ([_P, _I64, _I32, _I32, _P, _I32, _I32, _P, _P, _P, _P], ctypes.c_int),
    "nq_rans_compact": ([_P, _P, _P, _I64, _I32, _P, _P], ctypes.c_int),
    "nq_rans_decode": ([_P, _P, _I64, _I32, _I32, _P, _I32, _I32, _P, _P], ctypes.c_int),
    "nq_merge_workspace": ([_I32, _I32, _I32], _I64),
    "nq_merge_values": ([ctypes.POINTER(MergeDesc), _P], ctypes.c_int),
    "nq_page_encode": ([ctypes.POINTER(PageDesc), _P], ctypes.c_int),
    "nq_page_decode": ([ctypes.POINTER(PageDesc), _P], ctypes.c_int),
    "nq_page_logits": ([ctypes.POINTER(PageDesc), _P, _I32, _I32, _F32, _P, _P], ctypes.c_int),
    "nq_paged_attention_chunk_tokens": ([], ctypes.c_int32),
    "nq_paged_attention_workspace": ([_I32, _I32, _I32], _I64),
    "nq_paged_attention": ([ctypes.POINTER(AttnDesc), _P], ctypes.c_int),
    "nq_nibble_pack": ([_P, _I64, _I32, _P, _P], ctypes.c_int),
    "nq_nibble_unpack": ([_P, _I64, _I32, _I32, _P, _P], ctypes.c_int),
    "nq_e8_dequant_matmul": ([_P, _P, _P, _P, _I64, _I32, _I32, _I32, _P], ctypes.c_int),
    "nq_e8_nearest_point": ([_P, _P, _I64, _P], ctypes.c_int),
    "nq_e8_quantize_perhead": ([_P, _P, _I64, _I32, _I32, _P], ctypes.c_int),
    "nq_e8_stream_codes": ([_P, _P, _I64, _I64, _I32, _P, _P, _P], ctypes.c_int),
    "nq_e8_stream_values": ([_P, _P, _I64, _I64, _P, _P], ctypes.c_int),
}

_lock = threading.Lock()
_lib = None


class NexusQuantError(RuntimeError):
    pass


def load():
    """Load the library (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise NexusQuantError(
                    f"nexusquant_amd HIP library not found at {LIB_PATH}; build it with "
                    "`python -m nexusquant_amd.build` (hipcc, gfx950)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (args, res) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = res
            if lib.nq_abi_version() != ABI_VERSION:
                raise NexusQuantError(
                    f"{LIB_PATH} has ABI version {lib.nq_abi_version()}, the bindings expect "
                    f"{ABI_VERSION}; rebuild with `python -m nexusquant_amd.build`")
            built = lib.nq_source_hash().decode()
            want = source_hash()
            if built != want:
                raise NexusQuantError(
                    f"{LIB_PATH} was built from other sources (hash {built}, sources {want}); "
                    "rebuild with `python -m nexusquant_amd.build`")
            _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().nq_last_error().decode(errors="replace")
        if status == -1:
            raise ValueError(f"{what}: {msg}")
        raise NexusQuantError(f"{what} failed ({status}): {msg}")


def dtype_code(dtype) -> int:
    import torch
    if dtype == torch.float16:
        return NQ_F16
    if dtype == torch.bfloat16:
        return NQ_BF16
    if dtype == torch.float32:
        return NQ_F32
    raise TypeError(f"unsupported KV dtype {dtype}; expected float16, bfloat16 or float32")


def current_stream_handle(device) -> int:
    import torch
    return torch.cuda.current_stream(device).cuda_stream


def require_device(t, what: str = "tensor") -> None:
    if not t.is_cuda:
        raise NexusQuantError(
            f"nexusquant_amd runs on MI355X (ROCm) devices only; {what} is on {t.device}")
