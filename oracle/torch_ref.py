"""Tier-A oracle: op-for-op torch-CPU restatement of the reference KV-compression path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package (`nexusquant_amd/`)
may import this module; only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` use it, and only as the checker / CPU timing
baseline.

Every function repeats the reference's torch operator sequence (same ops, same
dtypes, same reduction shapes) so that on a given CPU its results equal the
reference's bit for bit; `tests/golden/` holds fixtures written by the real
reference that pin this claim.  Citations are `path:line` inside the reference
repository (jagmarques/nexusquant v0.5.0).

Pinning (see tests/test_oracle_*.py):
  e8_nearest_point        golden fixtures + Appendix-B known answers + invariants
  e8_quantize_perhead     golden fixtures + closed-form invariants
  hadamard_matrix         closed form (orthonormal, +-1/sqrt(n) entries)
  rope tables / rotation  golden fixtures + round-trip identities
  quant_only_compress     golden fixtures (reference NexusQuantEvict rate 0)
  score_keykey            golden fixtures + brute-force softmax on tiny inputs
  build_keep_mask         golden fixtures + reference test properties
  evict_mask_compress     golden fixtures
  evict_truncate_compress golden fixtures
  score_real_from_qk      golden fixtures written through transformers' eager
                          attention (third-party formula, transformers 5.15.0)
  delta_encode/decode     closed form + lossless round trip
  merge_eviction_values   golden fixture (reference NexusQuantEvict with
                          merge_eviction=True: survivors, merged values, outputs)
  vllm_* (page caller)    golden fixtures written by the reference's
                          integrations/vllm_backend.py (compress / decompress /
                          logits / nibble packing / paged forward)
  e8_dequant_matmul       brute-force loops on tiny inputs, identity query
                          (= codes * scales exactly), linearity in the query
                          (the reference's tests do not cover it)
"""

from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F


# ---------------------------------------------------------------------------
# Hadamard  (nexusquant/core/hadamard.py:15-43)
# ---------------------------------------------------------------------------

def next_power_of_2(n: int) -> int:
    """Smallest power of two >= n (hadamard.py:15-20)."""
    p = 1
    while p < n:
        p <<= 1
    return p


def hadamard_matrix(n: int) -> torch.Tensor:
    """Orthonormal Sylvester matrix built by recursive doubling (hadamard.py:23-43).

    Each doubling divides by the Python float sqrt(2) in fp32, exactly as the
    reference does, so the entries equal the reference's bit for bit.
    """
    if n & (n - 1):
        raise ValueError(f"n must be power of 2, got {n}. Use pad_to_power_of_2() first.")
    mat = torch.tensor([[1.0]])
    size = 1
    while size < n:
        top = torch.cat([mat, mat], dim=1)
        bottom = torch.cat([mat, -mat], dim=1)
        mat = torch.cat([top, bottom], dim=0) / math.sqrt(2)
        size *= 2
    return mat


# ---------------------------------------------------------------------------
# RoPE  (nexusquant/core/rope_utils.py:34-249)
# ---------------------------------------------------------------------------

def rope_scaled_inv_freq(inv_freq: torch.Tensor, rope_scaling: Optional[dict]) -> torch.Tensor:
    """Frequency scaling for linear / dynamic / llama3 configs (rope_utils.py:34-72)."""
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
        old_len = int(rope_scaling.get("original_max_position_embeddings", 8192))
        lo_wl = old_len / lo
        hi_wl = old_len / hi
        out = []
        for f in inv_freq:
            wl = 2.0 * math.pi / f.item()
            if wl < hi_wl:
                out.append(f)
            elif wl > lo_wl:
                out.append(f / factor)
            else:
                t = (old_len / wl - lo) / (hi - lo)
                out.append((1.0 - t) * f / factor + t * f)
        return torch.stack(out)
    return inv_freq


def rope_inv_freq(d: int, base: float, rope_scaling: Optional[dict] = None) -> torch.Tensor:
    """inv_freq = 1 / base**(arange(0,d,2)/d) in fp32 on the CPU (rope_utils.py:106-108)."""
    inv = 1.0 / (base ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    return rope_scaled_inv_freq(inv, rope_scaling)


def rope_cos_sin(positions: torch.Tensor, d: int, base: float,
                 rope_scaling: Optional[dict] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos/sin tables [len(positions), d/2] (rope_utils.py:109-112, 151-154)."""
    inv = rope_inv_freq(d, base, rope_scaling)
    ang = torch.outer(positions.to(torch.float32), inv)
    return ang.cos(), ang.sin()


def _rot_inverse(keys: torch.Tensor, cos_f: torch.Tensor, sin_f: torch.Tensor) -> torch.Tensor:
    half = keys.shape[-1] // 2
    lo = keys[..., :half]
    hi = keys[..., half:]
    out = keys.clone()
    out[..., :half] = lo * cos_f + hi * sin_f
    out[..., half:] = -lo * sin_f + hi * cos_f
    return out


def _rot_forward(keys: torch.Tensor, cos_f: torch.Tensor, sin_f: torch.Tensor) -> torch.Tensor:
    half = keys.shape[-1] // 2
    lo = keys[..., :half].clone()
    hi = keys[..., half:].clone()
    out = keys.clone()
    out[..., :half] = lo * cos_f - hi * sin_f
    out[..., half:] = lo * sin_f + hi * cos_f
    return out


def inverse_rope(keys: torch.Tensor, seq_offset: int = 0, base: float = 10000.0,
                 rope_scaling: Optional[dict] = None) -> torch.Tensor:
    """Split-half RoPE removal at positions offset..offset+s-1 (rope_utils.py:75-122)."""
    squeeze = keys.dim() == 3
    k4 = keys.unsqueeze(0) if squeeze else keys
    s, d = k4.shape[2], k4.shape[3]
    pos = torch.arange(s, dtype=torch.float32) + seq_offset
    c, sn = rope_cos_sin(pos, d, base, rope_scaling)
    out = _rot_inverse(k4, c.to(k4.device, k4.dtype), sn.to(k4.device, k4.dtype))
    return out.squeeze(0) if squeeze else out


def forward_rope(keys: torch.Tensor, seq_offset: int = 0, base: float = 10000.0,
                 rope_scaling: Optional[dict] = None) -> torch.Tensor:
    """Split-half RoPE application (rope_utils.py:203-249)."""
    squeeze = keys.dim() == 3
    k4 = keys.unsqueeze(0) if squeeze else keys
    s, d = k4.shape[2], k4.shape[3]
    pos = torch.arange(s, dtype=torch.float32) + seq_offset
    c, sn = rope_cos_sin(pos, d, base, rope_scaling)
    out = _rot_forward(k4, c.to(k4.device, k4.dtype), sn.to(k4.device, k4.dtype))
    return out.squeeze(0) if squeeze else out


def inverse_rope_at_positions(keys: torch.Tensor, positions: torch.Tensor, base: float = 10000.0,
                              rope_scaling: Optional[dict] = None) -> torch.Tensor:
    """RoPE removal at explicit positions, keys [h, s, d] (rope_utils.py:125-162)."""
    d = keys.shape[-1]
    c, sn = rope_cos_sin(positions.float(), d, base, rope_scaling)
    return _rot_inverse(keys, c.to(keys.dtype), sn.to(keys.dtype))


def forward_rope_at_positions(keys: torch.Tensor, positions: torch.Tensor, base: float = 10000.0,
                              rope_scaling: Optional[dict] = None) -> torch.Tensor:
    """RoPE application at explicit positions, keys [h, s, d] (rope_utils.py:165-200)."""
    d = keys.shape[-1]
    c, sn = rope_cos_sin(positions.float(), d, base, rope_scaling)
    return _rot_forward(keys, c.to(keys.dtype), sn.to(keys.dtype))


# ---------------------------------------------------------------------------
# Relaxed E8 lattice  (nexusquant/core/e8_lattice.py:27-124)
# ---------------------------------------------------------------------------

def e8_nearest_point(x: torch.Tensor) -> torch.Tensor:
    """Reference relaxed-E8 rule on (..., 8) fp32 (e8_lattice.py:27-69).

    Integer candidate: round-half-even, and when the coordinate sum is odd the
    FIRST smallest-gap coordinate steps one unit toward x (a zero gap steps +1).
    Half candidate: round(x - 0.5) + 0.5 with no parity repair (the reference's
    repair branch at :55-62 can never fire).  The half candidate wins only when
    its squared distance is strictly smaller.
    """
    r = x.round()
    odd = (r.sum(dim=-1) % 2) != 0
    if odd.any():
        gap = (x - r).abs()
        where = gap[odd].argmin(dim=-1, keepdim=True)
        step = torch.zeros_like(r[odd]).scatter_(-1, where, 1.0)
        direction = ((x[odd] - r[odd]).gather(-1, where) >= 0).float() * 2 - 1
        r[odd] = r[odd] + step * direction
    h = (x - 0.5).round() + 0.5
    d_int = ((x - r) ** 2).sum(dim=-1)
    d_half = ((x - h) ** 2).sum(dim=-1)
    out = r.clone()
    take = d_half < d_int
    out[take] = h[take]
    return out


def e8_quantize_perhead_parts(x: torch.Tensor, levels: int):
    """Per-row quantizer split into its parts (e8_lattice.py:97-124).

    Returns (lattice points p [rows, d] after clamp, scale [rows, 1]); the
    reference's output is `p * scale`.
    """
    d = x.shape[-1]
    flat = x.reshape(-1, d)
    amax = flat.abs().amax(dim=-1, keepdim=True).clamp(min=1e-8)
    scale = amax / (levels / 2)
    norm = flat / scale
    pad = (8 - d % 8) % 8
    if pad:
        norm = F.pad(norm, (0, pad))
    lp = e8_nearest_point(norm.reshape(-1, 8)).clamp(-levels / 2, levels / 2)
    p = lp.reshape(norm.shape)
    if pad:
        p = p[..., :d]
    return p, scale


def e8_quantize_perhead(x: torch.Tensor, levels: int = 8) -> torch.Tensor:
    """x -> p*scale, same shape (e8_lattice.py:97-124)."""
    p, scale = e8_quantize_perhead_parts(x, levels)
    return (p * scale).reshape(x.shape)


def lattice_codes_2p(p: torch.Tensor) -> torch.Tensor:
    """Stored int8 code = round(2p), the vLLM page format (vllm_backend.py:309-314)."""
    return (p * 2).round().clamp(-127, 127).to(torch.int8)


# ---------------------------------------------------------------------------
# Cache access  (nexusquant/pipeline.py:25-66)
# ---------------------------------------------------------------------------

def get_layer_kv(cache, i):
    if hasattr(cache, "key_cache") and hasattr(cache, "value_cache"):
        return cache.key_cache[i], cache.value_cache[i]
    layer = cache.layers[i]
    return layer.keys, layer.values


def set_layer_kv(cache, i, k, v):
    if hasattr(cache, "key_cache") and hasattr(cache, "value_cache"):
        cache.key_cache[i] = k
        cache.value_cache[i] = v
        return
    cache.layers[i].keys = k
    cache.layers[i].values = v


def num_layers(cache) -> int:
    if hasattr(cache, "key_cache"):
        return len(cache.key_cache)
    return len(cache.layers)


# ---------------------------------------------------------------------------
# Per-layer quantization bodies
# ---------------------------------------------------------------------------

def _quant_keys(k: torch.Tensor, H: torch.Tensor, levels: int, base: float,
                rope_scaling: Optional[dict]) -> torch.Tensor:
    """Keys of one layer, looped over batch (pipeline.py:245-255)."""
    b, h, s, d = k.shape
    outs = []
    for bi in range(b):
        k_nr = inverse_rope(k[bi], base=base, rope_scaling=rope_scaling)
        k_rot = torch.einsum('hsd,de->hse', k_nr, H)
        k_q = e8_quantize_perhead(k_rot.reshape(-1, d), levels=levels)
        k_back = torch.einsum('hsd,ed->hse', k_q.reshape(h, s, d), H)
        outs.append(forward_rope(k_back, base=base, rope_scaling=rope_scaling))
    return torch.stack(outs, dim=0)


def _quant_values(v: torch.Tensor, H: torch.Tensor, levels: int) -> torch.Tensor:
    """Values of one layer, batched (pipeline.py:257-261)."""
    b, h, s, d = v.shape
    v_rot = torch.einsum('bhsd,de->bhse', v, H)
    v_q = e8_quantize_perhead(v_rot.reshape(-1, d), levels=levels)
    return torch.einsum('bhsd,ed->bhse', v_q.reshape(b, h, s, d), H)


def quant_only_compress(cache, key_levels: int = 8, value_levels: int = 8,
                        rope_base: float = 10000.0, rope_scaling: Optional[dict] = None,
                        skip_layers: Sequence[int] = ()):
    """NexusQuantQuantOnly.compress with independent K/V levels (pipeline.py:232-265).

    With key_levels == value_levels this is the reference class exactly; with
    K8/V4 it equals NexusQuantEvict(key_bits=3, value_bits=2, eviction_rate=0)
    (every token kept, mask multiply by 1.0 is exact, pipeline.py:1190-1242).
    """
    for li in range(num_layers(cache)):
        if li in skip_layers:
            continue
        k, v = get_layer_kv(cache, li)
        k = k.float()
        v = v.float()
        d = k.shape[-1]
        H = hadamard_matrix(d).to(k.device).float()
        k_out = _quant_keys(k, H, key_levels, rope_base, rope_scaling).half()
        v_out = _quant_values(v, H, value_levels).half()
        set_layer_kv(cache, li, k_out, v_out)
    return cache


# ---------------------------------------------------------------------------
# Importance scoring  (pipeline.py:756-836)
# ---------------------------------------------------------------------------

def score_keykey(keys: torch.Tensor, obs_window: int = 32) -> torch.Tensor:
    """SnapKV-style key-key proxy (pipeline.py:756-782): [b,h,s,d] -> [b,s]."""
    b, h, s, d = keys.shape
    scale = d ** -0.5
    obs = min(obs_window, s)
    q = keys[:, :, -obs:, :]
    kk = keys[:, :, :s, :]
    att = torch.einsum('bhqd,bhkd->bhqk', q.float(), kk.float()) * scale
    att = torch.softmax(att, dim=-1)
    return att.sum(dim=2).mean(dim=1)


def eager_attention_probs(q: torch.Tensor, k: torch.Tensor, scaling: float, sliding_window=None,
                          softcap=None) -> torch.Tensor:
    """HF eager attention probabilities for one layer.

    transformers 5.15.0 models/llama/modeling_llama.py:179-213: repeat_kv for
    GQA, matmul(Q, K^T) * scaling in the model dtype, add the causal mask
    (dtype minimum above the diagonal), softmax in fp32, cast back.
    softcap: Gemma-2's w = tanh(w / softcap) * softcap before the mask
    (models/gemma2/modeling_gemma2.py:201-206); sliding_window: keys with
    key <= query - sliding_window are masked as well (masking_utils.py:92-101).
    q [b, hq, s, d], k [b, hkv, s, d] -> probs [b, hq, s, s] in q.dtype.
    """
    b, hq, s, d = q.shape
    rep = hq // k.shape[1]
    kr = k[:, :, None, :, :].expand(b, k.shape[1], rep, s, d).reshape(b, hq, s, d)
    w = torch.matmul(q, kr.transpose(2, 3)) * scaling
    if softcap is not None:
        w = w / softcap
        w = torch.tanh(w)
        w = w * softcap
    i = torch.arange(s, device=q.device)[:, None]
    j = torch.arange(s, device=q.device)[None, :]
    allowed = j <= i
    if sliding_window is not None:
        allowed = allowed & (j > i - sliding_window)
    mask = torch.zeros((s, s), dtype=q.dtype, device=q.device).masked_fill(~allowed, torch.finfo(q.dtype).min)
    w = w + mask
    return torch.softmax(w, dim=-1, dtype=torch.float32).to(q.dtype)


def score_real_from_qk(q_layers: Sequence[torch.Tensor], k_layers: Sequence[torch.Tensor],
                       scaling: Optional[float] = None, windows: Optional[Sequence] = None,
                       softcaps: Optional[Sequence] = None) -> torch.Tensor:
    """Importance from real attention (pipeline.py:822-836) given per-layer Q, K
    (and per-layer sliding windows / soft-caps, None for none)."""
    b, _, s, d = q_layers[0].shape
    if scaling is None:
        scaling = d ** -0.5
    n = len(q_layers)
    windows = windows if windows is not None else [None] * n
    softcaps = softcaps if softcaps is not None else [None] * n
    imp = torch.zeros(b, s, dtype=torch.float32)
    for q, k, w, cap in zip(q_layers, k_layers, windows, softcaps):
        probs = eager_attention_probs(q, k, scaling, sliding_window=w, softcap=cap).float()
        imp += probs.sum(dim=2).mean(dim=1)
    return imp / n


# ---------------------------------------------------------------------------
# Keep mask  (pipeline.py:895-959) and rate adjustments (:1083-1100)
# ---------------------------------------------------------------------------

def adaptive_context_rate(rate: float, seq: int) -> float:
    """Short-prefix rate scaling (pipeline.py:1093-1100)."""
    if seq < 256:
        return 0.0
    if seq < 512:
        return rate * 0.5
    if seq < 1024:
        return rate * 0.75
    return rate


def auto_eviction_rate(importance: torch.Tensor, seq: int) -> float:
    """Entropy-driven rate (pipeline.py:838-861)."""
    probs = importance[0] / (importance[0].sum() + 1e-8)
    ent = -(probs * (probs + 1e-8).log()).sum().item()
    norm = ent / math.log(max(seq, 2))
    return max(0.1, min(0.7, 0.7 - 0.5 * norm))


def build_keep_mask(importance: torch.Tensor, seq: int, rate: float, sliding_window: int = 32,
                    protected_positions=None, distance_graduated: bool = False) -> torch.Tensor:
    """BOS + recent window + top-k of the evictable prefix (pipeline.py:895-959)."""
    b = importance.shape[0]
    prefix = max(seq - sliding_window, 0)
    n_keep = max(1, int(prefix * (1.0 - rate)))
    keep = torch.zeros(b, seq, dtype=torch.bool, device=importance.device)
    keep[:, 0] = True
    if sliding_window > 0 and seq > 0:
        keep[:, max(0, seq - sliding_window):] = True
    if distance_graduated and prefix > 1:
        ramp = torch.linspace(0.0, 1.0, prefix - 1, device=importance.device)
        boost = ramp * importance[:, 1:prefix].max() * 0.25
        importance = importance.clone()
        importance[:, 1:prefix] = importance[:, 1:prefix] + boost
    if prefix > 1 and n_keep > 0:
        scores = importance[:, 1:prefix]
        k = min(n_keep, scores.shape[1])
        if k > 0:
            _, idx = torch.topk(scores, k=k, dim=1)
            keep.scatter_(1, idx + 1, True)
    if protected_positions is not None:
        for pos in protected_positions:
            i = int(pos)
            if 0 <= i < seq:
                keep[:, i] = True
    return keep


def boundary_skip_layers(n_layers: int, n_protect: int, protected_layers=()) -> set:
    """Boundary + explicit protected layers (pipeline.py:1110-1121)."""
    skip = set(protected_layers or ())
    for i in range(min(max(n_protect, 0), n_layers)):
        skip.add(i)
        skip.add(n_layers - 1 - i)
    return skip


def resolve_layer_levels(layer: int, n_layers: int, key_levels: int, value_levels: int,
                         profile: str = "uniform") -> Tuple[int, int]:
    """Graduated bit profile (pipeline.py:740-754)."""
    if profile == "graduated":
        edge = max(1, int(n_layers * 0.15))
        if layer < edge or layer >= n_layers - edge:
            return 8, 8
    return key_levels, value_levels


# ---------------------------------------------------------------------------
# Eviction pipelines
# ---------------------------------------------------------------------------

def _apply_keep_mask(cache, keep: torch.Tensor, key_levels: int, value_levels: int, rope_base: float,
                     rope_scaling: Optional[dict], skip_layers, layer_bit_profile: str) -> None:
    """Per-layer hard-eviction loop (pipeline.py:1190-1242): zero evicted rows,
    quantize (skip layers: fp16 cast only), zero them again."""
    n = num_layers(cache)
    for li in range(n):
        k, v = get_layer_kv(cache, li)
        k = k.float()
        v = v.float()
        _, h, s_l, d = k.shape
        m4 = keep[:, :s_l].unsqueeze(1).unsqueeze(-1).float()
        k = k * m4
        v = v * m4
        if li in skip_layers:
            set_layer_kv(cache, li, k.to(torch.float16), v.to(torch.float16))
            continue
        H = hadamard_matrix(d).to(k.device).float()
        kl, vl = resolve_layer_levels(li, n, key_levels, value_levels, layer_bit_profile)
        k_out = _quant_keys(k, H, kl, rope_base, rope_scaling).to(torch.float16)
        v_out = _quant_values(v, H, vl).to(torch.float16)
        k_out = k_out * m4.half()
        v_out = v_out * m4.half()
        set_layer_kv(cache, li, k_out, v_out)


def evict_mask_compress(cache, key_levels: int, value_levels: int, rate: float,
                        sliding_window: int = 32, obs_window: int = 32, rope_base: float = 10000.0,
                        rope_scaling: Optional[dict] = None, importance: Optional[torch.Tensor] = None,
                        skip_layers: Sequence[int] = (), protected_positions=None,
                        layer_bit_profile: str = "uniform"):
    """Hard-eviction mask path of NexusQuantEvict.compress (pipeline.py:1050-1244).

    Returns (cache, mask [b, s] float).  `importance` overrides the key-key
    scorer (used for the real-attention scorer).
    """
    k0, _ = get_layer_kv(cache, 0)
    b, _, seq, _ = k0.shape
    if importance is None:
        importance = score_keykey(k0.float(), obs_window)
    keep = build_keep_mask(importance, seq, rate, sliding_window, protected_positions)
    _apply_keep_mask(cache, keep, key_levels, value_levels, rope_base, rope_scaling, skip_layers, layer_bit_profile)
    return cache, keep.float()


def auto_detect_boundary(cache) -> int:
    """Boundary protection probe (pipeline.py:863-893): 2 when the mean |key| of
    the first and last layers is more than twice the middle layer's, else 0;
    0 below 6 layers."""
    n = num_layers(cache)
    if n < 6:
        return 0
    k_first, _ = get_layer_kv(cache, 0)
    k_last, _ = get_layer_kv(cache, n - 1)
    k_mid, _ = get_layer_kv(cache, n // 2)
    mag_boundary = (k_first.float().abs().mean() + k_last.float().abs().mean()) / 2
    mag_middle = k_mid.float().abs().mean()
    return 2 if (mag_boundary / (mag_middle + 1e-8)).item() > 2.0 else 0


def swa_layers_from_config(model_config) -> set:
    """Sliding-window layers of a hybrid model (pipeline.py:670-710): a
    sliding_window_pattern (every layer except each pattern-th), else
    layer_types naming local layers, else the last num_kv_shared_layers."""
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


def evict_compress(cache, key_levels: int, value_levels: int, eviction_rate, sliding_window: int = 32,
                   obs_window: int = 32, rope_base: float = 10000.0, rope_scaling: Optional[dict] = None,
                   protected_layers=(), protect_boundary=0, min_context_for_compression: int = 0,
                   adaptive_context: bool = False, distance_graduated: bool = False, swa_layers=None,
                   protected_positions=None, layer_bit_profile: str = "uniform", importance=None):
    """NexusQuantEvict.compress, hard-eviction mask mode, with every option
    (pipeline.py:1050-1127 then :1190-1244): the scoring layer is the first
    non-SWA layer when swa_layers is given ("global_only"), the rate is "auto"
    (entropy) or fixed, scaled by adaptive_context; the keep mask may carry the
    distance ramp; boundary protection is an int or "auto"; SWA layers are
    skipped; a prefix shorter than min_context_for_compression passes through.
    importance [b, s], when given, replaces the key-key scores, as the hook's
    injected real-attention scores do (huggingface.py:743-749).

    Returns (cache, mask [b, s] float, resolved rate, skipped layer set)."""
    n = num_layers(cache)
    score_layer = 0
    if swa_layers:
        score_layer = next((li for li in range(n) if li not in swa_layers), 0)
    k_score, _ = get_layer_kv(cache, score_layer)
    b, _, seq, _ = k_score.shape
    if importance is None:
        importance = score_keykey(k_score.float(), obs_window)
    rate = auto_eviction_rate(importance, seq) if eviction_rate == "auto" else float(eviction_rate)
    if adaptive_context:
        rate = adaptive_context_rate(rate, seq)
    keep = build_keep_mask(importance, seq, rate, sliding_window, protected_positions, distance_graduated)
    n_protect = auto_detect_boundary(cache) if protect_boundary == "auto" else int(protect_boundary)
    skip = boundary_skip_layers(n, n_protect, protected_layers)
    if swa_layers:
        skip |= set(swa_layers)
    if min_context_for_compression > 0 and seq < min_context_for_compression:
        return cache, torch.ones(b, seq), rate, skip
    _apply_keep_mask(cache, keep, key_levels, value_levels, rope_base, rope_scaling, skip, layer_bit_profile)
    return cache, keep.float(), rate, skip


def merge_centroids(value_layers: Sequence[torch.Tensor], bi: int) -> Optional[torch.Tensor]:
    """Mean over heads, averaged over layers, of batch row bi (pipeline.py:997-1013)."""
    centroid_sum = None
    count = 0
    for v_l in value_layers:
        v_mean = v_l[bi].float().mean(dim=0)
        centroid_sum = v_mean if centroid_sum is None else centroid_sum + v_mean
        count += 1
    return None if centroid_sum is None else centroid_sum / count


def merge_survivors(centroids: torch.Tensor, keep_row: torch.Tensor):
    """(evicted positions, kept positions, survivor kept-list index per evicted,
    cosine matrix) (pipeline.py:983-1024)."""
    evict_pos = (~keep_row).nonzero(as_tuple=True)[0]
    kept_pos = keep_row.nonzero(as_tuple=True)[0]
    e_n = F.normalize(centroids[evict_pos], dim=-1)
    k_n = F.normalize(centroids[kept_pos], dim=-1)
    cos = torch.mm(e_n, k_n.t())
    return evict_pos, kept_pos, cos.argmax(dim=1), cos


def merge_eviction_values(value_layers: Sequence[torch.Tensor], keep: torch.Tensor, importance: torch.Tensor,
                          survivors: Optional[Sequence[torch.Tensor]] = None) -> List[torch.Tensor]:
    """MergingPress-style value merging (pipeline.py:961-1048) over the layers
    whose seq equals the mask's; returns new value tensors.  `survivors[bi]`
    (kept-list index per evicted position) overrides the cosine argmax."""
    out = [v.clone() for v in value_layers]
    b = keep.shape[0]
    for bi in range(b):
        km = keep[bi]
        imp = importance[bi]
        evict_pos = (~km).nonzero(as_tuple=True)[0]
        kept_pos = km.nonzero(as_tuple=True)[0]
        if evict_pos.numel() == 0 or kept_pos.numel() == 0:
            continue
        cent = merge_centroids(out, bi)
        if survivors is None:
            _, _, nearest, _ = merge_survivors(cent, km)
        else:
            nearest = survivors[bi]
        for li, v_l in enumerate(out):
            v = v_l[bi].float()
            for ei, e_pos in enumerate(evict_pos):
                s_pos = kept_pos[nearest[ei].item()]
                imp_e = imp[e_pos].item()
                imp_s = imp[s_pos].item()
                w = imp_e / (imp_s + imp_e + 1e-8)
                v[:, s_pos, :] = v[:, s_pos, :] + w * v[:, e_pos, :]
            new_v = v_l.clone()
            new_v[bi] = v.to(dtype=v_l.dtype)
            out[li] = new_v
    return out


def evict_merge_compress(cache, key_levels: int, value_levels: int, rate: float, sliding_window: int = 32,
                         obs_window: int = 32, rope_base: float = 10000.0, importance=None,
                         skip_layers: Sequence[int] = ()):
    """NexusQuantEvict.compress with merge_eviction=True (pipeline.py:1184-1244)."""
    n = num_layers(cache)
    k0, _ = get_layer_kv(cache, 0)
    seq = k0.shape[2]
    if importance is None:
        importance = score_keykey(k0.float(), obs_window)
    keep = build_keep_mask(importance, seq, rate, sliding_window)
    layers = [li for li in range(n) if get_layer_kv(cache, li)[1].shape[2] == seq]
    merged = merge_eviction_values([get_layer_kv(cache, li)[1] for li in layers], keep, importance)
    for li, mv in zip(layers, merged):
        set_layer_kv(cache, li, get_layer_kv(cache, li)[0], mv)
    return evict_mask_compress(cache, key_levels, value_levels, rate, sliding_window, obs_window, rope_base,
                               importance=importance, skip_layers=skip_layers)


def evict_soft_compress(cache, key_levels: int, value_levels: int, rate: float,
                        sliding_window: int = 32, obs_window: int = 32, rope_base: float = 10000.0,
                        rope_scaling: Optional[dict] = None, skip_layers: Sequence[int] = (),
                        protected_positions=None, layer_bit_profile: str = "uniform"):
    """Soft-eviction path of NexusQuantEvict.compress (pipeline.py:1129-1183).

    Kept rows are quantized at the layer's levels, evicted rows at levels 2 (the
    reference computes both on every row and selects with the 0/1 mask);
    protected layers are cast to fp16 unmasked.  Returns (cache, all-ones mask).
    """
    n = num_layers(cache)
    k0, _ = get_layer_kv(cache, 0)
    b, _, seq, _ = k0.shape
    importance = score_keykey(k0.float(), obs_window)
    keep = build_keep_mask(importance, seq, rate, sliding_window, protected_positions)
    ones = torch.ones(b, seq, dtype=torch.float32)
    for li in range(n):
        k, v = get_layer_kv(cache, li)
        k = k.float()
        v = v.float()
        if li in skip_layers:
            set_layer_kv(cache, li, k.half(), v.half())
            continue
        _, h, s_l, d = k.shape
        H = hadamard_matrix(d).to(k.device).float()
        kl, vl = resolve_layer_levels(li, n, key_levels, value_levels, layer_bit_profile)
        m4 = keep[:, :s_l].unsqueeze(1).unsqueeze(-1).float()
        k_out = []
        for bi in range(b):
            k_nr = inverse_rope(k[bi], base=rope_base, rope_scaling=rope_scaling)
            k_flat = torch.einsum('hsd,de->hse', k_nr, H).reshape(-1, d)
            full = e8_quantize_perhead(k_flat, levels=kl)
            one_bit = e8_quantize_perhead(k_flat, levels=2)
            kf = m4[bi].expand(h, s_l, 1).reshape(h * s_l, 1)
            k_q = full * kf + one_bit * (1.0 - kf)
            k_back = torch.einsum('hsd,ed->hse', k_q.reshape(h, s_l, d), H)
            k_out.append(forward_rope(k_back, base=rope_base, rope_scaling=rope_scaling))
        k_out = torch.stack(k_out, dim=0).to(torch.float16)
        v_flat = torch.einsum('bhsd,de->bhse', v, H).reshape(-1, d)
        full = e8_quantize_perhead(v_flat, levels=vl)
        one_bit = e8_quantize_perhead(v_flat, levels=2)
        vf = m4.expand(b, h, s_l, 1).reshape(b * h * s_l, 1)
        v_q = full * vf + one_bit * (1.0 - vf)
        v_out = torch.einsum('bhsd,ed->bhse', v_q.reshape(b, h, s_l, d), H).to(torch.float16)
        set_layer_kv(cache, li, k_out, v_out)
    return cache, ones


def evict_truncate_compress(cache, key_levels: int, value_levels: int, rate: float,
                            sliding_window: int = 32, obs_window: int = 32,
                            rope_base: float = 10000.0, rope_scaling: Optional[dict] = None,
                            skip_layers: Sequence[int] = (), protected_positions=None,
                            layer_bit_profile: str = "uniform"):
    """NexusQuantEvictTruncate.compress (pipeline.py:1270-1406): returns (cache, n_kept)."""
    n = num_layers(cache)
    k0, _ = get_layer_kv(cache, 0)
    b, _, seq, _ = k0.shape
    if b > 1:
        raise ValueError(
            f"NexusQuantEvictTruncate does not support batch_size > 1 (got {b}).")
    importance = score_keykey(k0.float(), obs_window)
    keep = build_keep_mask(importance, seq, rate, sliding_window, protected_positions)
    kept = keep[0].nonzero(as_tuple=True)[0]
    n_kept = kept.shape[0]
    for li in range(n):
        k, v = get_layer_kv(cache, li)
        _, h, s_l, d = k.shape
        lk = kept[kept < s_l]
        nk = lk.shape[0]
        k_kept = k[:, :, lk, :].float()
        v_kept = v[:, :, lk, :].float()
        if li in skip_layers:
            set_layer_kv(cache, li, k_kept.to(torch.float16), v_kept.to(torch.float16))
            continue
        H = hadamard_matrix(d).to(k.device).float()
        kl, vl = resolve_layer_levels(li, n, key_levels, value_levels, layer_bit_profile)
        pos_in = lk.float()
        pos_out = torch.arange(nk, dtype=torch.float32)
        outs = []
        for bi in range(b):
            k_nr = inverse_rope_at_positions(k_kept[bi], pos_in, base=rope_base, rope_scaling=rope_scaling)
            k_rot = torch.einsum('hsd,de->hse', k_nr, H)
            k_q = e8_quantize_perhead(k_rot.reshape(-1, d), levels=kl)
            k_back = torch.einsum('hsd,ed->hse', k_q.reshape(h, nk, d), H)
            outs.append(forward_rope_at_positions(k_back, pos_out, base=rope_base, rope_scaling=rope_scaling))
        k_out = torch.stack(outs, dim=0).to(torch.float16)
        v_rot = torch.einsum('bhsd,de->bhse', v_kept, H)
        v_q = e8_quantize_perhead(v_rot.reshape(-1, d), levels=vl)
        v_out = torch.einsum('bhsd,ed->bhse', v_q.reshape(b, h, nk, d), H).to(torch.float16)
        set_layer_kv(cache, li, k_out, v_out)
    return cache, n_kept


# ---------------------------------------------------------------------------
# Temporal delta stream  (nexusquant/core/compression_accounting.py:49-77)
# ---------------------------------------------------------------------------

def delta_encode(codes: torch.Tensor) -> torch.Tensor:
    """int8 codes [streams, tokens, coords] -> deltas along tokens (int8 wrap)."""
    import numpy as np
    x = codes.numpy().astype(np.int8)
    out = np.zeros_like(x)
    out[:, 0, :] = x[:, 0, :]
    out[:, 1:, :] = x[:, 1:, :] - x[:, :-1, :]
    return torch.from_numpy(out.astype(np.int8))


def delta_decode(delta: torch.Tensor) -> torch.Tensor:
    """Inverse of delta_encode: cumulative sum along tokens, wrapped to int8."""
    import numpy as np
    x = delta.numpy()
    return torch.from_numpy(np.cumsum(x, axis=1).astype(np.int8))


# ---------------------------------------------------------------------------
# vLLM page caller  (nexusquant/integrations/vllm_backend.py)
# ---------------------------------------------------------------------------

def vllm_quantize_with_scales(x: torch.Tensor, levels: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """(h, s, d) fp32 -> int8 codes 2p (h, s, d), fp32 scales (h, s) (vllm_backend.py:267-314)."""
    h, s, d = x.shape
    flat = x.reshape(h * s, d)
    amax = flat.abs().amax(dim=-1, keepdim=True).clamp(min=1e-8)
    scale = amax / (levels / 2)
    normalized = flat / scale
    pad = (8 - d % 8) % 8
    if pad > 0:
        normalized = F.pad(normalized, (0, pad))
    lp = e8_nearest_point(normalized.reshape(-1, 8)).clamp(-levels / 2, levels / 2)
    codes_full = lp.reshape(h * s, d + pad)[..., :d]
    codes = (codes_full * 2).round().clamp(-127, 127).to(torch.int8).reshape(h, s, d)
    return codes, scale.squeeze(-1).reshape(h, s)


def vllm_dequantize(codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """(codes * 0.5) * scale in fp32 (vllm_backend.py:316-338)."""
    return (codes.float() * 0.5) * scales.float().unsqueeze(-1)


def _page_tables(positions: torch.Tensor, d: int, base: float):
    c, sn = rope_cos_sin(positions.to(torch.int32).float(), d, base)
    return c.unsqueeze(0), sn.unsqueeze(0)


def vllm_compress_page(key_page: torch.Tensor, value_page: torch.Tensor, positions: torch.Tensor,
                       bits: int, base: float):
    """-> (key_codes, value_codes, key_scales fp16, value_scales fp16) (vllm_backend.py:344-392, 187-224)."""
    levels = 2 ** bits
    d = key_page.shape[-1]
    H = hadamard_matrix(d)
    k = key_page.float()
    v = value_page.float()
    c, sn = _page_tables(positions, d, base)
    k_nr = _rot_inverse(k, c, sn)
    k_rot = torch.einsum('hsd,de->hse', k_nr, H.float())
    kc, ks = vllm_quantize_with_scales(k_rot, levels)
    v_rot = torch.einsum('hsd,de->hse', v, H.float())
    vc, vs = vllm_quantize_with_scales(v_rot, levels)
    return kc, vc, ks.to(torch.float16), vs.to(torch.float16)


def vllm_decompress_keys_fp32(key_codes, key_scales, positions, base: float) -> torch.Tensor:
    """Dequantize, inverse Hadamard, RoPE at the stored positions (vllm_backend.py:410-415, 226-265)."""
    d = key_codes.shape[-1]
    H = hadamard_matrix(d)
    k_rot = vllm_dequantize(key_codes, key_scales)
    k_nr = torch.einsum('hsd,ed->hse', k_rot, H.float())
    c, sn = _page_tables(positions, d, base)
    return _rot_forward(k_nr, c, sn)


def vllm_decompress_page(key_codes, value_codes, key_scales, value_scales, positions, base: float):
    """-> (keys, values) fp16 (vllm_backend.py:394-429)."""
    d = key_codes.shape[-1]
    H = hadamard_matrix(d)
    keys = vllm_decompress_keys_fp32(key_codes, key_scales, positions, base).to(torch.float16)
    v_rot = vllm_dequantize(value_codes, value_scales)
    values = torch.einsum('hsd,ed->hse', v_rot, H.float()).to(torch.float16)
    return keys, values


def vllm_decompress_for_attention(key_codes, key_scales, positions, query, base: float) -> torch.Tensor:
    """Logits (h, q_len, s) = q . k / sqrt(d) on fp32 keys (vllm_backend.py:431-467)."""
    scale = math.sqrt(key_codes.shape[-1])
    keys = vllm_decompress_keys_fp32(key_codes, key_scales, positions, base)
    return torch.einsum('hqd,hsd->hqs', query.float(), keys) / scale


def vllm_paged_forward(query: torch.Tensor, pages: dict, block_tables, context_lens, base: float) -> torch.Tensor:
    """Decode attention over pages {block_id: (kc, vc, ks, vs, positions)} (vllm_backend.py:692-765)."""
    batch_size, num_heads, head_dim = query.shape
    scale = math.sqrt(head_dim)
    output = torch.zeros_like(query)
    for b in range(batch_size):
        ctx_len = int(context_lens[b])
        if ctx_len == 0:
            continue
        ks, vs = [], []
        for block_id in block_tables[b]:
            if block_id not in pages:
                continue
            k_page, v_page = vllm_decompress_page(*pages[block_id], base)
            ks.append(k_page)
            vs.append(v_page)
        if not ks:
            continue
        keys = torch.cat(ks, dim=1)[:, :ctx_len, :]
        values = torch.cat(vs, dim=1)[:, :ctx_len, :]
        q3 = query[b].unsqueeze(1).float()
        logits = torch.einsum('hqd,hsd->hqs', q3, keys.float()) / scale
        w = torch.softmax(logits, dim=-1)
        att = torch.einsum('hqs,hsd->hqd', w, values.float())
        output[b] = att.squeeze(1).to(torch.float16)
    return output


def pack_codes_nibble(codes: torch.Tensor) -> torch.Tensor:
    """(..., d) int8 -> (..., ceil(d/2)) uint8 nibbles (vllm_backend.py:475-515)."""
    d = codes.shape[-1]
    c = (codes.to(torch.int32) + 8).clamp(0, 15)
    if d % 2 != 0:
        c = F.pad(c, (0, 1))
    return ((c[..., 0::2] & 0xF) | ((c[..., 1::2] & 0xF) << 4)).to(torch.uint8)


def unpack_codes_nibble(packed: torch.Tensor, original_d: int) -> torch.Tensor:
    """Inverse nibble unpacking (vllm_backend.py:517-536)."""
    p = packed.to(torch.int32)
    inter = torch.stack([p & 0xF, (p >> 4) & 0xF], dim=-1)
    shape = list(inter.shape)[:-2] + [-1]
    return (inter.reshape(shape)[..., :original_d] - 8).to(torch.int8)


def e8_dequant_matmul(codes: torch.Tensor, scales: torch.Tensor, query: torch.Tensor) -> torch.Tensor:
    """Fused decode + matrix product of the standalone E8 format
    (e8_triton.py:373-444, 613-660): vals = fp32(codes[:, :H]) * scales[:, None]
    rounded to fp32 as the reference forms them, then vals @ query accumulated in
    float64 (the exact value the GPU's fp32 sums approximate).  codes int8 [K, H_pad],
    query [H, Q_cols] -> float64 [K, Q_cols]."""
    h = query.shape[0]
    vals = codes[:, :h].to(torch.float32) * scales.to(torch.float32)[:, None]
    return vals.to(torch.float64) @ query.to(torch.float32).to(torch.float64)
