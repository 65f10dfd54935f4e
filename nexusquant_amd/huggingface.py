"""HuggingFace drop-in: the nexusquant_evict context manager (huggingface.py:505-807).

Same arguments, presets, errors, yielded compressor (.last_mask / .next_position)
and hook behaviour as the reference: DynamicLayer.update and
DynamicSlidingWindowLayer.update are patched for the duration of the context;
on each prefill-sized update of a layer the concatenated keys/values of that
layer are compressed on the GPU and returned to the attention call.  As in the
reference, compress() therefore sees one layer at a time, so key-key scoring
uses each layer's own keys and protect_boundary > 0 protects that single layer
(huggingface.py:736-752).

compat_reference_hook=False selects the full-cache semantics instead: prefill
updates pass through uncompressed and register their layer; the registered
layers are then compressed together by one NexusQuantEvict.compress call on the
whole cache (layer-0 or injected real-attention scores, boundary protection
across the model's layers, graduated bit profile, automatic boundary), as
compress_kv_cache does after a prefill.  That happens when the model's forward
returns, before the next update of a registered layer (a decode step or the
next prefill chunk) and, for what is still registered, when the context exits.
"""

from __future__ import annotations

import time
import warnings
from contextlib import contextmanager
from typing import Optional

import torch

from .pipeline import NexusQuantEvict, NexusQuantEvictTruncate

_EVICT_PRESETS = {
    "high": {"eviction_rate": 0.35, "bits": 2, "key_bits": 3},
    "balanced": {"eviction_rate": 0.60, "bits": 2},
    "max": {"eviction_rate": 0.80, "bits": 2},
    "asym": {"eviction_rate": 0.60, "bits": 2, "key_bits": 3},
}


class _CompressionStats:
    """Byte accounting of what the hook produced (the reference's _CompressionStats,
    huggingface.py:40-98, assumes 2 bits/element of scale overhead; this counts the
    packed code sizes of this build: per 8-group 8 symbols of ceil(log2(L+1)) bits,
    a coset bit and one fp32 scale per head vector)."""

    def __init__(self, key_bits: int, value_bits: int):
        self.key_bits, self.value_bits = key_bits, value_bits
        self.original = 0
        self.compressed = 0.0
        self.layers = 0
        self.start = time.time()

    def record(self, k: torch.Tensor, v: torch.Tensor) -> None:
        sym_bits = {1: 2, 2: 3, 3: 4, 4: 5}
        d = k.shape[-1]
        for t, bits in ((k, self.key_bits), (v, self.value_bits)):
            rows = t.numel() // d
            self.original += t.numel() * 2
            self.compressed += rows * (d / 8 * (sym_bits.get(bits, bits + 1) + 1 / 8) + 4)
        self.layers += 1

    def summary(self) -> str:
        ratio = self.original / self.compressed if self.compressed else 1.0
        return "\n".join([
            "", "--- NexusQuant Compression Stats (nexusquant_amd) ---",
            f"  Compression ratio:    {ratio:.1f}x (packed codes vs fp16)",
            f"  Layers compressed:    {self.layers}",
            f"  Wall time:            {time.time() - self.start:.2f}s",
            "------------------------------------"])


def _detect_model_config(model):
    """head_dim / layers / rope_theta / kv heads / rope_scaling (huggingface.py:105-133)."""
    cfg = model.config
    text = getattr(cfg, "text_config", cfg)
    head_dim = getattr(text, "head_dim", None)
    if head_dim is None:
        head_dim = getattr(text, "hidden_size", 4096) // getattr(text, "num_attention_heads", 32)
    rope_base = getattr(text, "rope_theta", None)
    rope_scaling = getattr(text, "rope_scaling", None)
    rp = getattr(text, "rope_parameters", None)
    if rope_base is None and isinstance(rp, dict):
        rope_base = rp.get("rope_theta")
        if rope_scaling is None and rp.get("rope_type", "default") != "default":
            rope_scaling = rp
    return {
        "head_dim": head_dim,
        "num_layers": getattr(text, "num_hidden_layers", 32),
        "rope_base": rope_base if rope_base is not None else 10000.0,
        "num_kv_heads": getattr(text, "num_key_value_heads", None) or getattr(text, "num_attention_heads", 32),
        "rope_scaling": rope_scaling,
    }


class _SingleLayerCache:
    def __init__(self, k, v):
        self.key_cache = [k]
        self.value_cache = [v]


class _LayerListCache:
    """Cache view over transformers cache-layer objects (reads and writes .keys/.values)."""

    def __init__(self, layers):
        self.layers = layers


@contextmanager
def nexusquant_evict(model, eviction_rate=0.6, quality: str = "balanced", sliding_window: int = 32,
                     obs_window: int = 32, bits: int = 2, key_bits: int = None, value_bits: int = None,
                     truncate: bool = False, scorer: str = "key-key", input_ids=None,
                     protected_layers: set = None, protect_boundary=0, min_context_for_compression: int = 0,
                     soft_eviction: bool = False, adaptive_context: bool = False,
                     protected_positions: Optional[torch.Tensor] = None, compress_layers: str = "all",
                     layer_bit_profile: str = "uniform", verbose: bool = True,
                     compat_reference_hook: bool = True):
    """Compress the KV cache with eviction + relaxed-E8 quantization on the first prefill.

    compat_reference_hook=True (default) compresses each layer alone inside its
    update, as the reference does; False compresses the whole cache at once
    after the prefill (see the module docstring)."""
    if quality in _EVICT_PRESETS:
        preset = _EVICT_PRESETS[quality]
        eviction_rate = preset["eviction_rate"]
        bits = preset["bits"]
        if key_bits is None and "key_bits" in preset:
            key_bits = preset["key_bits"]
        if value_bits is None and "value_bits" in preset:
            value_bits = preset["value_bits"]

    if scorer == "real":
        attn_impl = getattr(model.config, "_attn_implementation", None)
        if attn_impl != "eager":
            raise ValueError(
                f"scorer='real' requires attn_implementation='eager' but model reports "
                f"attn_implementation={attn_impl!r}. "
                "SDPA suppresses attention weights silently. "
                "Reload with: AutoModelForCausalLM.from_pretrained("
                "..., attn_implementation='eager')")
        if input_ids is None:
            raise ValueError(
                "scorer='real' requires input_ids to be passed to nexusquant_evict(). "
                "These are the (batch, seq) token ids for the prefix.")

    mc = _detect_model_config(model)
    if hasattr(model, "_offload_cache"):
        warnings.warn(
            "NexusQuantEvict detected KV cache offloading (_offload_cache). "
            "Compression hooks intercept DynamicCache layer updates and may not "
            "fire for offloaded cache writes. Results may be incorrect or "
            "compression may silently not apply. Disable KV cache offloading "
            "when using NexusQuant.", stacklevel=3)

    cls = NexusQuantEvictTruncate if truncate else NexusQuantEvict
    compressor = cls(head_dim=mc["head_dim"], bits=bits, key_bits=key_bits, value_bits=value_bits,
                     eviction_rate=eviction_rate, sliding_window=sliding_window, obs_window=obs_window,
                     rope_base=mc["rope_base"], rope_scaling=mc["rope_scaling"], scorer=scorer,
                     protected_layers=protected_layers, protect_boundary=protect_boundary,
                     min_context_for_compression=min_context_for_compression, soft_eviction=soft_eviction,
                     adaptive_context=adaptive_context, protected_positions=protected_positions,
                     compress_layers=compress_layers, layer_bit_profile=layer_bit_profile)
    if compress_layers == "global_only":
        compressor.set_model_config(model.config)
    compressor.last_mask = None
    compressor.next_position = None
    compressor._cached_real_importance = (
        compressor._score_importance_real(model, input_ids) if scorer == "real" else None)
    stats = _CompressionStats(compressor.key_bits, compressor.value_bits)

    from transformers.cache_utils import DynamicLayer, DynamicSlidingWindowLayer

    original_dl = DynamicLayer.update
    original_dsw = DynamicSlidingWindowLayer.update

    def run_compress(cache):
        if scorer == "real" and compressor._cached_real_importance is not None:
            cached = compressor._cached_real_importance
            compressor._score_importance = lambda k, _imp=cached: _imp
            try:
                result = compressor.compress(cache)
            finally:
                del compressor._score_importance
        else:
            result = compressor.compress(cache)
        if truncate:
            compressor.next_position = result[1]
        else:
            compressor.last_mask = result[1]

    # full-cache mode: cache-layer objects registered by prefill updates, in order
    pending = []

    def flush():
        if not pending:
            return
        layers = list(pending)
        pending.clear()
        run_compress(_LayerListCache(layers))
        for lay in layers:
            lay.keys._nq_compressed = True
            stats.record(lay.keys, lay.values)

    def make_hook(original):
        def hooked_update(self, key_states, value_states, *args, **kwargs):
            if not compat_reference_hook and any(lay is self for lay in pending):
                flush()
            keys, values = original(self, key_states, value_states, *args, **kwargs)
            if getattr(keys, "_nq_compressed", False):
                return keys, values
            incoming = key_states.shape[-2]
            existing = keys.shape[-2] - incoming
            if incoming < 2:
                return keys, values
            if existing > 0 and incoming < max(existing * 0.1, 8):
                return keys, values
            if not compat_reference_hook:
                pending.append(self)
                return keys, values
            single = _SingleLayerCache(keys, values)
            run_compress(single)
            new_k, new_v = single.key_cache[0], single.value_cache[0]
            new_k._nq_compressed = True
            self.keys = new_k
            self.values = new_v
            stats.record(new_k, new_v)
            return new_k, new_v
        return hooked_update

    DynamicLayer.update = make_hook(original_dl)
    DynamicSlidingWindowLayer.update = make_hook(original_dsw)
    forward_patched = False
    if not compat_reference_hook:
        # compress right after each forward of the model (a prefill), before
        # the caller or generate() sees the cache
        had_own_forward = "forward" in model.__dict__
        own_forward = model.__dict__.get("forward")
        inner_forward = model.forward

        def forward_then_compress(*args, **kwargs):
            out = inner_forward(*args, **kwargs)
            flush()
            return out

        model.forward = forward_then_compress
        forward_patched = True
    if verbose:
        kb, vb = compressor.key_bits, compressor.value_bits
        bits_label = f"K={kb}-bit/V={vb}-bit E8" if kb != vb else f"{kb}-bit E8"
        ev = "auto" if eviction_rate == "auto" else f"{eviction_rate:.0%}"
        name = getattr(model.config, "_name_or_path", model.__class__.__name__)
        print(f"NexusQuantEvict (gfx950): activating on {name} (eviction={ev}, {bits_label}, "
              f"sliding_window={sliding_window}, mode={'truncate' if truncate else 'mask'}, "
              f"scorer={scorer}, {'per-layer' if compat_reference_hook else 'full-cache'})", flush=True)
    try:
        yield compressor
        flush()
    finally:
        pending.clear()
        DynamicLayer.update = original_dl
        DynamicSlidingWindowLayer.update = original_dsw
        if forward_patched:
            if had_own_forward:
                model.forward = own_forward
            else:
                del model.forward
        if verbose:
            print(stats.summary(), flush=True)
