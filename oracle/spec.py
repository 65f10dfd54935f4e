"""ctypes wrapper of the Tier-B C oracle (oracle/nq_spec.c).  Test infrastructure only."""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "libnq_spec.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile the C oracle with its Makefile (gcc, no FMA contraction)."""
    if force or not os.path.exists(_SO):
        subprocess.check_call(["make", "-B" if force else "-s", "-C", _HERE],
                              stdout=subprocess.DEVNULL)
    return _SO


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        P = ctypes.c_void_p
        L.nqs_quant_rows.argtypes = [ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_float, P, P, P, P, P, P, P, P, P, P, P, P]
        L.nqs_quant_rows.restype = None
        L.nqs_e8_group.argtypes = [P, ctypes.c_float, P, P, P]
        L.nqs_e8_group.restype = None
        L.nqs_page_decode.argtypes = [ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_float, P, P, P, P, P]
        L.nqs_page_decode.restype = None
        L.nqs_f32_to_f16.argtypes = [ctypes.c_float]
        L.nqs_f32_to_f16.restype = ctypes.c_uint16
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def hadamard_constant(D: int) -> float:
    """h_D = 1/sqrt(2) divided log2(D) times in fp32, as hadamard.py:37-43 builds it."""
    import math
    import torch
    h = torch.tensor([1.0])
    n = 1
    while n < D:
        h = h / math.sqrt(2)
        n *= 2
    return float(h.item())


def quant_rows(x: np.ndarray, L: int, D: int | None = None, cos_in=None, sin_in=None,
               cos_out=None, sin_out=None, margins: bool = False):
    """Run the C oracle on rows x [n, d] (fp32).  Returns a dict of numpy arrays."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, d = x.shape
    if D is None:
        D = 1
        while D < d:
            D <<= 1
    G = D // 8
    out = {
        "xn": np.empty((n, D), np.float32),
        "p": np.empty((n, D), np.float32),
        "sym": np.empty((n, D), np.uint8),
        "coset": np.empty((n, G), np.uint8),
        "scale": np.empty((n,), np.float32),
        "recon": np.empty((n, d), np.uint16),
    }
    if margins:
        out["margin"] = np.empty((n, G), np.float32)
    tabs = [None if t is None else np.ascontiguousarray(t, dtype=np.float32)
            for t in (cos_in, sin_in, cos_out, sin_out)]
    lib().nqs_quant_rows(n, d, D, L, hadamard_constant(D), _ptr(x),
                         *[_ptr(t) for t in tabs],
                         _ptr(out["xn"]), _ptr(out["p"]), _ptr(out["sym"]), _ptr(out["coset"]),
                         _ptr(out["scale"]), _ptr(out["recon"]), _ptr(out.get("margin")))
    out["recon"] = out["recon"].view(np.float16)
    return out


def e8_groups(x: np.ndarray, L: int):
    """Run the C E8 rule on [n, 8] normalised groups -> (p, coset, margin)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 8)
    n = x.shape[0]
    p = np.empty_like(x)
    cs = np.empty(n, np.int32)
    mg = np.empty(n, np.float32)
    f = lib().nqs_e8_group
    for i in range(n):
        f(_ptr(x[i]), float(L // 2), _ptr(p[i]), ctypes.c_void_p(cs[i:].ctypes.data),
          ctypes.c_void_p(mg[i:].ctypes.data))
    return p, cs, mg


def page_decode(codes: np.ndarray, scales16: np.ndarray, is_key: bool, cos_rows=None, sin_rows=None):
    """Run the C oracle's page decode on int8 codes [n, D] and fp16 scales [n]
    (keys: cos/sin rows [n, D/2] at each row's stored position) -> fp16 [n, D]."""
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    n, D = codes.shape
    sc = np.ascontiguousarray(scales16, dtype=np.float16).view(np.uint16)
    out = np.empty((n, D), np.uint16)
    tabs = [None if t is None else np.ascontiguousarray(t, dtype=np.float32) for t in (cos_rows, sin_rows)]
    lib().nqs_page_decode(n, D, int(is_key), hadamard_constant(D), _ptr(codes), _ptr(sc),
                          _ptr(tabs[0]), _ptr(tabs[1]), _ptr(out))
    return out.view(np.float16)


def page_encode(x: np.ndarray, L: int, cos_rows=None, sin_rows=None):
    """The page encoder's arithmetic (the row quantizer with keys rotated at
    each row's position): rows x [n, D] -> (int8 codes 2p [n, D], fp16 scales [n],
    margins [n, D/8])."""
    o = quant_rows(x, L, cos_in=cos_rows, sin_in=sin_rows, cos_out=cos_rows, sin_out=sin_rows, margins=True)
    return (2.0 * o["p"]).astype(np.int8), o["scale"].astype(np.float16), o["margin"]
