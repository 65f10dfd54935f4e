"""Drop-in compression pipelines (nexusquant/pipeline.py), running on gfx950 kernels.

Same classes, constructor arguments, return conventions and error messages as
the reference; every tensor operation of the hot path is one fused HIP launch
per (role, layer group) instead of the reference's chain of torch operators.
"""

from __future__ import annotations

import math
from typing import Any, Dict, List, Optional, Sequence, Tuple, Union

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


# ---------------------------------------------------------------------------
# Eviction + quantization (pipeline.py:535-1244) and truncation (:1247-1406)
# ---------------------------------------------------------------------------

class NexusQuantEvict:
    """Importance scoring, keep mask, eviction and relaxed-E8 quantization on gfx950.

    Constructor arguments, validation errors and the (cache, mask) return
    convention follow NexusQuantEvict (pipeline.py:535-668, 1050-1244).  Evicted
    rows are zeroed inside the fused quantizer (mask eviction).  soft_eviction
    quantizes evicted rows at levels 2 instead (two launches into the same
    outputs); merge_eviction folds evicted values into their nearest survivors first.
    """

    def __init__(self, head_dim: int = 128, bits: int = 2, key_bits: int = None, value_bits: int = None,
                 eviction_rate: Union[float, str] = 0.6, sliding_window: int = 32, obs_window: int = 32,
                 rope_base: float = 10000.0, rope_scaling: dict = None, scorer: str = "key-key",
                 protected_layers: set = None, protect_boundary: Union[int, str] = 0,
                 min_context_for_compression: int = 0, soft_eviction: bool = False,
                 adaptive_context: bool = False, protected_positions: Optional[torch.Tensor] = None,
                 compress_layers: str = "all", layer_bit_profile: str = "uniform",
                 distance_graduated: bool = False, merge_eviction: bool = False):
        if scorer not in ("key-key", "real"):
            raise ValueError(f"scorer must be 'key-key' or 'real', got {scorer!r}")
        if not (isinstance(eviction_rate, (int, float)) or eviction_rate == "auto"):
            raise ValueError(
                f"eviction_rate must be a float in [0, 1] or 'auto', got {eviction_rate!r}")
        if not (isinstance(protect_boundary, int) or protect_boundary == "auto"):
            raise ValueError(
                f"protect_boundary must be a non-negative int or 'auto', got {protect_boundary!r}")
        self.head_dim = head_dim
        self.bits = bits
        self.key_bits = key_bits if key_bits is not None else bits
        self.value_bits = value_bits if value_bits is not None else bits
        self.key_levels = 2 ** self.key_bits
        self.value_levels = 2 ** self.value_bits
        self.levels = 2 ** bits
        self.eviction_rate = eviction_rate
        self.sliding_window = sliding_window
        self.obs_window = obs_window
        self.rope_base = rope_base
        self.rope_scaling = rope_scaling
        self.scorer = scorer
        self.protected_layers = set(protected_layers) if protected_layers else set()
        self.protect_boundary = protect_boundary
        self.min_context_for_compression = min_context_for_compression
        self.soft_eviction = soft_eviction
        self.adaptive_context = adaptive_context
        self.protected_positions = protected_positions
        self.compress_layers = compress_layers
        self.layer_bit_profile = layer_bit_profile
        self.distance_graduated = distance_graduated
        self.merge_eviction = merge_eviction
        self._swa_layer_indices = None

    # -- configuration helpers (pipeline.py:670-754) --------------------------

    def set_model_config(self, model_config):
        if self.compress_layers != "global_only":
            return
        self._swa_layer_indices = _swa_layers_from_config(model_config)

    def _find_scoring_layer(self, past_key_values, n_layers: int) -> int:
        if self.compress_layers == "global_only" and self._swa_layer_indices:
            for li in range(n_layers):
                if li not in self._swa_layer_indices:
                    return li
        return 0

    def _resolve_layer_levels(self, layer_idx: int, n_layers: int):
        if self.layer_bit_profile == "graduated":
            edge = max(1, int(n_layers * 0.15))
            if layer_idx < edge or layer_idx >= n_layers - edge:
                return 8, 8
        return self.key_levels, self.value_levels

    # -- importance (pipeline.py:756-861) -------------------------------------

    def _score_importance(self, keys: torch.Tensor) -> torch.Tensor:
        """Key-key importance [batch, seq] (MFMA kernel, pipeline.py:756-782)."""
        from .ops import score_keykey
        return score_keykey(keys, self.obs_window)

    def _score_importance_real(self, model, input_ids: torch.Tensor) -> torch.Tensor:
        """Real-attention importance from one scoring forward pass (pipeline.py:784-836)."""
        from .scoring import real_importance
        return real_importance(model, input_ids)

    def _compute_adaptive_eviction_rate(self, importance: torch.Tensor, seq: int) -> float:
        """Entropy-driven rate (pipeline.py:838-861); a few device ops on a [seq] vector."""
        probs = importance[0] / (importance[0].sum() + 1e-8)
        ent = -(probs * (probs + 1e-8).log()).sum().item()
        norm = ent / math.log(max(seq, 2))
        return max(0.1, min(0.7, 0.7 - 0.5 * norm))

    def _auto_detect_boundary(self, past_key_values) -> int:
        """Boundary protection probe (pipeline.py:863-893), cached after the first call."""
        if hasattr(self, "_auto_boundary_cached"):
            return self._auto_boundary_cached
        n = num_layers(past_key_values)
        if n < 6:
            self._auto_boundary_cached = 0
            return 0
        k_first, _ = get_layer_kv(past_key_values, 0)
        k_last, _ = get_layer_kv(past_key_values, n - 1)
        k_mid, _ = get_layer_kv(past_key_values, n // 2)
        mb = (k_first.float().abs().mean() + k_last.float().abs().mean()) / 2
        mm = k_mid.float().abs().mean()
        self._auto_boundary_cached = 2 if (mb / (mm + 1e-8)).item() > 2.0 else 0
        return self._auto_boundary_cached

    def _resolve_rate(self, importance: torch.Tensor, seq: int) -> float:
        if self.eviction_rate == "auto":
            rate = self._compute_adaptive_eviction_rate(importance, seq)
        else:
            rate = float(self.eviction_rate)
        if self.adaptive_context:
            if seq < 256:
                rate = 0.0
            elif seq < 512:
                rate *= 0.5
            elif seq < 1024:
                rate *= 0.75
        return rate

    def _graduate(self, importance: torch.Tensor, seq: int) -> torch.Tensor:
        """Distance ramp on the prefix scores (pipeline.py:935-941)."""
        prefix = max(seq - self.sliding_window, 0)
        if not self.distance_graduated or prefix <= 1:
            return importance
        ramp = torch.linspace(0.0, 1.0, prefix - 1, device=importance.device)
        boost = ramp * importance[:, 1:prefix].max() * 0.25
        importance = importance.clone()
        importance[:, 1:prefix] = importance[:, 1:prefix] + boost
        return importance

    def _keep(self, importance: torch.Tensor, seq: int, rate: float):
        from .ops import keep_mask
        return keep_mask(self._graduate(importance, seq), rate, self.sliding_window,
                         self.protected_positions)

    def _skip_layers(self, past_key_values, n_layers: int) -> set:
        n_protect = (self._auto_detect_boundary(past_key_values) if self.protect_boundary == "auto"
                     else int(self.protect_boundary))
        skip = set(self.protected_layers)
        for i in range(min(max(n_protect, 0), n_layers)):
            skip.add(i)
            skip.add(n_layers - 1 - i)
        if self.compress_layers == "global_only" and self._swa_layer_indices:
            skip.update(self._swa_layer_indices)
        return skip

    def _importance(self, past_key_values, n_layers, model=None, input_ids=None, require_model=True):
        score_layer = self._find_scoring_layer(past_key_values, n_layers)
        k_score, _ = get_layer_kv(past_key_values, score_layer)
        # The nexusquant_evict hook injects precomputed real-attention scores by
        # shadowing _score_importance on the instance; use them.  (The reference
        # raises here in mask mode because model/input_ids are absent inside the
        # hook, pipeline.py:1077-1081 vs huggingface.py:743-752.)
        injected = "_score_importance" in self.__dict__
        if self.scorer == "real" and require_model and not injected:
            if model is None or input_ids is None:
                raise ValueError(
                    "scorer='real' requires model and input_ids to be passed to compress(). "
                    "Also ensure the model was loaded with attn_implementation='eager'.")
            return self._score_importance_real(model, input_ids), k_score
        return self._score_importance(k_score), k_score

    def _apply(self, past_key_values, n_layers: int, skip: set, *, keep=None, gather=None, soft=False,
               kept_idx=None, n_kept=None):
        """Quantize (or pass through at fp16) every layer with one mask / gather list.

        soft: kept rows at the layer's levels and evicted rows at levels 2, no row
        zeroed (pipeline.py:1129-1183); protected layers pass through unmasked.
        kept_idx / n_kept (keep_mask's row list): mask eviction reads and
        quantizes only the kept rows of layers as long as the mask; evicted rows
        get the zero-row outputs directly (the same results)."""
        todo: Dict[tuple, List[int]] = {}
        passthrough: Dict[tuple, List[int]] = {}
        for li in range(n_layers):
            k, v = get_layer_kv(past_key_values, li)
            key = (tuple(k.shape), k.dtype, tuple(v.shape), v.dtype)
            if li in skip:
                passthrough.setdefault(key, []).append(li)
            else:
                kl, vl = self._resolve_layer_levels(li, n_layers)
                todo.setdefault(key + (kl, vl), []).append(li)
        from .ops import gather_rows

        def layer_args(k_shape):
            s_l = k_shape[2]
            kp = None if keep is None else keep[:, :s_l]
            gp = None
            if gather is not None:
                gp = gather[gather < s_l].unsqueeze(0)
            return kp, gp

        for key, layers in passthrough.items():
            kp, gp = layer_args(key[0])
            if soft:
                kp = None
            ks = [get_layer_kv(past_key_values, li)[0] for li in layers]
            vs = [get_layer_kv(past_key_values, li)[1] for li in layers]
            k_out = gather_rows(ks, gather=gp, keep=kp)
            v_out = gather_rows(vs, gather=gp, keep=kp)
            for i, li in enumerate(layers):
                set_layer_kv(past_key_values, li, k_out[i], v_out[i])
        for key, layers in todo.items():
            kl, vl = key[4], key[5]
            kp, gp = layer_args(key[0])
            ks = [get_layer_kv(past_key_values, li)[0] for li in layers]
            vs = [get_layer_kv(past_key_values, li)[1] for li in layers]
            if soft:
                from ._lib import NQ_KEEP_WRITE_EVICTED, NQ_KEEP_WRITE_KEPT
                k_out, _ = quantize_tensors(ks, is_key=True, levels=kl, rope_base=self.rope_base,
                                            rope_scaling=self.rope_scaling, keep=kp, keep_mode=NQ_KEEP_WRITE_KEPT)
                quantize_tensors(ks, is_key=True, levels=2, rope_base=self.rope_base,
                                 rope_scaling=self.rope_scaling, keep=kp, keep_mode=NQ_KEEP_WRITE_EVICTED,
                                 recon_out=k_out)
                v_out, _ = quantize_tensors(vs, is_key=False, levels=vl, keep=kp, keep_mode=NQ_KEEP_WRITE_KEPT)
                quantize_tensors(vs, is_key=False, levels=2, keep=kp, keep_mode=NQ_KEEP_WRITE_EVICTED,
                                 recon_out=v_out)
            else:
                lst = {}
                if kp is not None and gp is None and kept_idx is not None and key[0][2] == keep.shape[1]:
                    lst = dict(order=kept_idx, n_kept=n_kept)
                k_out, _ = quantize_tensors(ks, is_key=True, levels=kl, rope_base=self.rope_base,
                                            rope_scaling=self.rope_scaling, gather=gp, keep=kp, **lst)
                v_out, _ = quantize_tensors(vs, is_key=False, levels=vl, gather=gp, keep=kp, **lst)
            for i, li in enumerate(layers):
                set_layer_kv(past_key_values, li, k_out[i], v_out[i])

    def _merge(self, past_key_values, n_layers: int, seq: int, keep, kept_idx, n_kept, importance) -> None:
        """Merge eviction (pipeline.py:961-1048): the values of every layer whose
        seq equals the mask's are replaced by nq_merge_values' merged copies."""
        from .ops import merge_values
        layers = [li for li in range(n_layers) if get_layer_kv(past_key_values, li)[1].shape[2] == seq]
        if not layers:
            return
        merged, _, _ = merge_values([get_layer_kv(past_key_values, li)[1] for li in layers], keep, kept_idx,
                                    n_kept, importance)
        for li, mv in zip(layers, merged):
            set_layer_kv(past_key_values, li, get_layer_kv(past_key_values, li)[0], mv)

    def compress(self, past_key_values, model=None, input_ids=None):
        """Evict + quantize in place; returns (cache, prefix_attention_mask [b, s] float)."""
        n = num_layers(past_key_values)
        importance, k_score = self._importance(past_key_values, n, model, input_ids)
        b, _, seq, _ = k_score.shape
        device = k_score.device
        rate = self._resolve_rate(importance, seq)
        keep, kept_idx, n_kept = self._keep(importance, seq, rate)
        prefix_attention_mask = keep.float()
        skip = self._skip_layers(past_key_values, n)
        if self.min_context_for_compression > 0 and seq < self.min_context_for_compression:
            return past_key_values, torch.ones(b, seq, device=device)
        if self.soft_eviction:
            # every position stays visible; evicted rows are only coarser (pipeline.py:1129-1183)
            self._apply(past_key_values, n, skip, keep=keep, soft=True)
            return past_key_values, torch.ones(b, seq, dtype=torch.float32, device=device)
        if self.merge_eviction:
            self._merge(past_key_values, n, seq, keep, kept_idx, n_kept, importance)
        self._apply(past_key_values, n, skip, keep=keep, kept_idx=kept_idx, n_kept=n_kept)
        return past_key_values, prefix_attention_mask


class NexusQuantEvictTruncate(NexusQuantEvict):
    """Physical truncation with RoPE re-encoded at contiguous positions (pipeline.py:1247-1406).

    Kept rows are gathered inside the fused quantizer: keys are de-rotated at
    their original positions and re-rotated at 0..n_kept-1.  Returns
    (cache, n_kept).
    """

    def compress(self, past_key_values):
        n = num_layers(past_key_values)
        score_layer = self._find_scoring_layer(past_key_values, n)
        k_score, _ = get_layer_kv(past_key_values, score_layer)
        b, _, seq, _ = k_score.shape
        if b > 1:
            raise ValueError(
                f"NexusQuantEvictTruncate does not support batch_size > 1 (got {b}). "
                "Physical truncation requires identical sequence lengths across batch elements. "
                "Use NexusQuantEvict (masking, not truncation) for batched inference.")
        importance = self._score_importance(k_score)
        rate = self._resolve_rate(importance, seq)
        _, kept, n_kept_t = self._keep(importance, seq, rate)
        skip = self._skip_layers(past_key_values, n)
        if self.min_context_for_compression > 0 and seq < self.min_context_for_compression:
            return past_key_values, seq
        n_kept = int(n_kept_t[0].item())
        self._apply(past_key_values, n, skip, gather=kept[0, :n_kept])
        if hasattr(past_key_values, "_seen_tokens"):
            past_key_values._seen_tokens = n_kept
        return past_key_values, n_kept


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
