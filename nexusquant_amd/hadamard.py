"""Hadamard helpers of the public API (nexusquant/core/hadamard.py:15-43).

The device kernels apply the transform as in-register butterflies; the host
only needs the normalisation constant, built with the same fp32 divisions as
the reference's Sylvester recursion so that the constant matches its entries.
"""

from __future__ import annotations

import functools
import math

import torch


def next_power_of_2(n: int) -> int:
    """Smallest power of two >= n (hadamard.py:15-20)."""
    p = 1
    while p < n:
        p <<= 1
    return p


def hadamard_matrix(n: int) -> torch.Tensor:
    """Orthonormal Sylvester matrix (hadamard.py:23-43); raises for n not a power of 2."""
    if n & (n - 1):
        raise ValueError(f"n must be power of 2, got {n}. Use pad_to_power_of_2() first.")
    m = torch.ones(1, 1)
    while m.shape[0] < n:
        m = torch.cat([torch.cat([m, m], 1), torch.cat([m, -m], 1)], 0) / math.sqrt(2)
    return m


@functools.lru_cache(maxsize=None)
def hadamard_constant(n: int) -> float:
    """|entry| of hadamard_matrix(n): 1.0 divided log2(n) times by sqrt(2) in fp32."""
    if n & (n - 1):
        raise ValueError(f"n must be power of 2, got {n}")
    h = torch.ones(1)
    size = 1
    while size < n:
        h = h / math.sqrt(2)
        size *= 2
    return float(h.item())
