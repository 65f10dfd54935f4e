"""Drop-in compression pipelines (nexusquant/pipeline.py), running on gfx950 kernels.

Same classes, constructor arguments, return conventions and error messages as
the reference; every tensor operation of the hot path is one fused HIP launch
per (role, layer group) instead of the reference's chain of torch operators.
"""

from __future__ import annotations

from typing import Any, Dict, List, Optional, Sequence, Tuple

import torch

from .ops import PackedCodes, quantize_tensors


# ---------------------------------------------------------------------------
# Cache access (pipeline.py:25-66): .key_cache/.value_cache lists or .layers[i]
# ---------------------------------------------------------------------------

def get_layer_kv(cache, layer: int):
    if hasattr(cache, "key_cache") and hasattr(cache, "value_cache"):
        return cache.key_cache[layer], cache.value_cache[layer]
    lay = cache.layers[layer]
    return getattr(lay, "keys"), getattr(lay, "values")


def set_layer_kv(cache, layer: int, keys, values) -> None:
    if hasattr(cache, "key_cache") and hasattr(cache, "value_cache"):
        cache.key_cache[layer] = keys
        cache.value_cache[layer] = values
        return
    lay = cache.layers[layer]
    setattr(lay, "keys", keys)
    setattr(lay, "values", values)


def num_layers(cache) -> int:
    if hasattr(cache, "key_cache"):
        return len(cache.key_cache)
    return len(cache.layers)


def _swa_layers_from_config(model_config) -> set:
    """Sliding-window layer detection for hybrid models (pipeline.py:193-221, 670-710)."""
    cfg = getattr(model_config, "text_config", model_config)
    swa = set()
    n = getattr(cfg, "num_hidden_layers", 32)
    pattern = getattr(cfg, "sliding_window_pattern", None)
    if pattern is not None:
        for i in range(n):
            if (i + 1) % pattern != 0:
                swa.add(i)
    types = getattr(cfg, "layer_types", None)
    if types is not None and not swa:
        for i, lt in enumerate(types):
            if lt in ("sliding_window", "local", "swa", "sliding_attention"):
                swa.add(i)
    shared = getattr(cfg, "num_kv_shared_layers", 0)
    if shared > 0 and not swa:
        for i in range(n - shared, n):
            swa.add(i)
    return swa


def _group_layers(cache, layers: Sequence[int]) -> List[List[int]]:
    """Split layers into runs that share shape/dtype/device (one launch each)."""
    groups: Dict[tuple, List[int]] = {}
    order = []
    for li in layers:
        k, v = get_layer_kv(cache, li)
        key = (tuple(k.shape), k.dtype, k.device, tuple(v.shape), v.dtype)
        if key not in groups:
            groups[key] = []
            order.append(key)
        groups[key].append(li)
    return [groups[k] for k in order]


def quantize_cache_layers(cache, layers: Sequence[int], key_levels: int, value_levels: int,
                          rope_base: float, rope_scaling: Optional[dict], *,
                          keep: Optional[torch.Tensor] = None, gather: Optional[torch.Tensor] = None,
                          return_codes: bool = False) -> Dict[int, Tuple[PackedCodes, PackedCodes]]:
    """Quantize the given layers in place (new fp16 tensors replace the old ones)."""
    codes: Dict[int, Tuple[PackedCodes, PackedCodes]] = {}
    for group in _group_layers(cache, layers):
        ks = [get_layer_kv(cache, li)[0] for li in group]
        vs = [get_layer_kv(cache, li)[1] for li in group]
        k_out, k_codes = quantize_tensors(ks, is_key=True, levels=key_levels, rope_base=rope_base,
                                          rope_scaling=rope_scaling, gather=gather, keep=keep,
                                          codes=return_codes)
        v_out, v_codes = quantize_tensors(vs, is_key=False, levels=value_levels, gather=gather,
                                          keep=keep, codes=return_codes)
        for i, li in enumerate(group):
            set_layer_kv(cache, li, k_out[i], v_out[i])
            if return_codes:
                codes[li] = (k_codes[i], v_codes[i])
    return codes


# ---------------------------------------------------------------------------
# Quantization only (pipeline.py:171-265)
# ---------------------------------------------------------------------------

class NexusQuantQuantOnly:
    """RoPE removal + Hadamard + relaxed E8 per-row quantization, no eviction.

    Mirrors NexusQuantQuantOnly (pipeline.py:171-265); `key_bits`/`value_bits`
    (default `bits`) select asymmetric levels, which the reference expresses
    only through NexusQuantEvict(eviction_rate=0).  After compress(),
    `last_codes` holds the packed codes per layer when `keep_codes=True`.
    """

    def __init__(self, bits: int = 3, rope_base: float = 10000.0, rope_scaling: dict = None,
                 compress_layers: str = "all", key_bits: Optional[int] = None,
                 value_bits: Optional[int] = None, keep_codes: bool = False):
        self.bits = bits
        self.levels = 2 ** bits
        self.key_bits = key_bits if key_bits is not None else bits
        self.value_bits = value_bits if value_bits is not None else bits
        self.key_levels = 2 ** self.key_bits
        self.value_levels = 2 ** self.value_bits
        self.rope_base = rope_base
        self.rope_scaling = rope_scaling
        self.compress_layers = compress_layers
        self.keep_codes = keep_codes
        self._swa_layer_indices = None
        self.last_codes: Dict[int, Tuple[PackedCodes, PackedCodes]] = {}

    def set_model_config(self, model_config):
        if self.compress_layers != "global_only":
            return
        self._swa_layer_indices = _swa_layers_from_config(model_config)

    def compress(self, past_key_values) -> Any:
        n = num_layers(past_key_values)
        skip = self._swa_layer_indices or set()
        layers = [li for li in range(n) if li not in skip]
        self.last_codes = quantize_cache_layers(
            past_key_values, layers, self.key_levels, self.value_levels, self.rope_base,
            self.rope_scaling, return_codes=self.keep_codes)
        return past_key_values


def compress_kv_cache(past_key_values, mode: str = "simple", head_dim: int = 128, **kwargs) -> Any:
    """Compress a KV cache in place (pipeline.py:1409-1468).

    mode "quant_only" (and "simple" without token merging, numerically the same
    path in the reference: pipeline.py:125-168 vs 232-265) run the fused gfx950
    quantizer.  Beyond the reference, `key_bits` / `value_bits` select
    asymmetric levels (K3V2); they default to `bits`.
    """
    if mode in ("quant_only", "simple"):
        if mode == "simple" and kwargs.get("merge_pct", 0.0):
            raise NotImplementedError("mode='simple' with merge_pct > 0 (token merging) is not "
                                      "part of the gfx950 hot path")
        nq = NexusQuantQuantOnly(
            bits=kwargs.get("bits", 3),
            rope_base=kwargs.get("rope_base", 10000.0),
            rope_scaling=kwargs.get("rope_scaling", None),
            key_bits=kwargs.get("key_bits"),
            value_bits=kwargs.get("value_bits"),
            keep_codes=kwargs.get("keep_codes", False),
        )
        out = nq.compress(past_key_values)
        if kwargs.get("keep_codes", False):
            past_key_values.nexusquant_codes = nq.last_codes
        return out
    if mode in ("fast", "max", "asymmetric"):
        raise NotImplementedError(
            f"mode={mode!r} is outside the gfx950 hot path (use 'quant_only' or 'simple')")
    raise ValueError(f"Unknown mode: {mode}. Use 'simple', 'fast', 'max', 'asymmetric', or 'quant_only'.")
