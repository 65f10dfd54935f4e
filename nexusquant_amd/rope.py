"""Host-built RoPE tables (nexusquant/core/rope_utils.py:34-249).

The reference builds cos/sin on the CPU in fp32 with torch on every call
(rope_utils.py:106-112).  Device cosf/sinf differ from torch's CPU kernels in
the last ulp for a few percent of angles, and at 128K positions one ulp of the
angle moves a rotated key by ~1e-2 relative, so the table is built the same way
on the host, once per (length, head_dim, base, scaling, device), and shared by
every layer and head.  Values for a position do not depend on the table length
(torch's CPU cos is elementwise and deterministic across sizes and threads).
"""

from __future__ import annotations

import json
import math
import threading
from typing import Optional, Tuple

import torch

_cache = {}
_lock = threading.Lock()
_ROUND = 4096


def scaled_inv_freq(inv_freq: torch.Tensor, rope_scaling: Optional[dict]) -> torch.Tensor:
    """linear / dynamic / llama3 frequency scaling (rope_utils.py:34-72)."""
    if rope_scaling is None:
        return inv_freq
    kind = rope_scaling.get("type", rope_scaling.get("rope_type", "linear"))
    factor = float(rope_scaling.get("factor", 1.0))
    if factor == 1.0:
        return inv_freq
    if kind in ("linear", "dynamic"):
        return inv_freq / factor
    if kind == "llama3":
        lo = float(rope_scaling.get("low_freq_factor", 1.0))
        hi = float(rope_scaling.get("high_freq_factor", 4.0))
        old = int(rope_scaling.get("original_max_position_embeddings", 8192))
        lo_wl, hi_wl = old / lo, old / hi
        out = []
        for f in inv_freq:
            wl = 2.0 * math.pi / f.item()
            if wl < hi_wl:
                out.append(f)
            elif wl > lo_wl:
                out.append(f / factor)
            else:
                t = (old / wl - lo) / (hi - lo)
                out.append((1.0 - t) * f / factor + t * f)
        return torch.stack(out)
    return inv_freq


def inv_freq(head_dim: int, base: float, rope_scaling: Optional[dict] = None) -> torch.Tensor:
    """1 / base**(arange(0, d, 2)/d) in fp32 on the CPU (rope_utils.py:106-108)."""
    f = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    return scaled_inv_freq(f, rope_scaling)


def host_table(n_pos: int, head_dim: int, base: float,
               rope_scaling: Optional[dict] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos/sin [n_pos, head_dim/2] for positions 0..n_pos-1 (CPU tensors)."""
    ang = torch.outer(torch.arange(n_pos, dtype=torch.float32), inv_freq(head_dim, base, rope_scaling))
    return ang.cos(), ang.sin()


def device_table(n_pos: int, head_dim: int, base: float, rope_scaling: Optional[dict],
                 device) -> Tuple[torch.Tensor, torch.Tensor]:
    """Cached device copy of host_table covering at least n_pos positions."""
    device = torch.device(device)
    key = (head_dim, float(base), json.dumps(rope_scaling, sort_keys=True, default=str), device)
    with _lock:
        hit = _cache.get(key)
        if hit is not None and hit[0].shape[0] >= n_pos:
            return hit
        n = max(_ROUND, -(-n_pos // _ROUND) * _ROUND)
        c, s = host_table(n, head_dim, base, rope_scaling)
        tab = (c.to(device), s.to(device))
        _cache[key] = tab
        return tab


def device_merged_table(n_pos: int, head_dim: int, base: float, rope_scaling: Optional[dict],
                        device) -> Tuple[torch.Tensor, torch.Tensor]:
    """Cached device fl(sin - cos), fl(cos + sin) [>= n_pos, head_dim/2] (fp32, built on the
    host from host_table).  The fused kernels fold RoPE into the top Hadamard stage
    with these; they are the same numbers the kernels would form from cos and sin."""
    device = torch.device(device)
    key = ("merged", head_dim, float(base), json.dumps(rope_scaling, sort_keys=True, default=str), device)
    with _lock:
        hit = _cache.get(key)
        if hit is not None and hit[0].shape[0] >= n_pos:
            return hit
        n = max(_ROUND, -(-n_pos // _ROUND) * _ROUND)
        c, s = host_table(n, head_dim, base, rope_scaling)
        tab = ((s - c).to(device), (c + s).to(device))
        _cache[key] = tab
        return tab


def clear_cache() -> None:
    with _lock:
        _cache.clear()
