"""Real-attention importance through one scoring forward pass (pipeline.py:784-836).

The reference runs model(input_ids, output_attentions=True) under eager
attention and column-sums the returned [batch, heads, seq, seq] probabilities
of every layer.  Here the model runs with an attention wrapper registered in
transformers' AttentionInterface.  For fp16 / bf16 models with head_dim 64 or
128 each layer's attention goes to nq_attention_real, which computes the
layer output and accumulates the same column sums from its (post-RoPE)
queries, keys and values with eager's roundings and without materialising
the probabilities (causal, GQA).  Other models run their own attention for
the output, and nq_score_real adds the column sums.

Sliding-window layers (Mistral, Phi-3, Gemma-2's local layers) pass their
window to the kernels, and logit soft-capping (Gemma-2) a 65536-entry table of
the capped logit per model-dtype logit, built with torch's own ops.  The
model's attention mask is checked once per mask tensor against the causal
(+ window) pattern the kernels implement; any other mask (padding, chunked or
bidirectional attention) raises.
"""

from __future__ import annotations

import ctypes
import sys
import threading

import torch

from . import _lib
from .ops import _addr, workspace

_lock = threading.Lock()
_NAME = "nexusquant_real_scorer"
_maps = {}


def logit_map(dtype: torch.dtype, softcap: float, device) -> torch.Tensor:
    """Soft-capping as a table over the 65536 values of the model dtype.

    Entry x (the bits of a logit w in `dtype`) holds the bits of
    (tanh(w / softcap)) * softcap computed as transformers' Gemma-2 eager
    attention does (models/gemma2/modeling_gemma2.py:203-206): each op on a
    `dtype` tensor, on the CPU.  Cached per (dtype, softcap, device)."""
    if dtype not in (torch.float16, torch.bfloat16):
        raise NotImplementedError(f"logit soft-capping is implemented for fp16 and bf16 models, not {dtype}")
    key = (dtype, float(softcap), torch.device(device))
    t = _maps.get(key)
    if t is None:
        w = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(dtype)
        w = w / softcap
        w = torch.tanh(w)
        w = w * softcap
        t = w.view(torch.int16).to(device)
        _maps[key] = t
    return t


def _window(sliding_window, seq: int) -> int:
    """The kernels' window argument: 0 (plain causal) unless a window is shorter than seq."""
    if sliding_window is None or int(sliding_window) <= 0 or int(sliding_window) >= seq:
        return 0
    return int(sliding_window)


def mask_is_causal(attention_mask, q_len: int, kv_len: int, sliding_window: int = 0) -> bool:
    """True when an eager attention mask (4D additive float, 0 = attend, or bool,
    True = attend) admits exactly key j <= query i (and j > i - sliding_window
    for a window > 0), the pattern the real-scorer kernels implement."""
    if attention_mask is None or attention_mask.dim() != 4 or q_len != kv_len:
        return False
    m = attention_mask[..., :q_len, :kv_len]
    if tuple(m.shape[-2:]) != (q_len, kv_len):
        return False
    allowed = m if m.dtype == torch.bool else (m == 0)
    i = torch.arange(q_len, device=m.device)[:, None]
    j = torch.arange(kv_len, device=m.device)[None, :]
    want = j <= i
    if sliding_window > 0:
        want = want & (j > i - sliding_window)
    return bool(torch.equal(allowed, want.expand_as(allowed)))


def score_real_accumulate(query: torch.Tensor, key: torch.Tensor, importance: torch.Tensor,
                          scaling: float, sliding_window=None, softcap=None) -> None:
    """importance[b, s] += mean over query heads of causal column sums (one layer).

    sliding_window: query i sees keys i - window < j <= i (None: all j <= i);
    softcap: Gemma-2's logit soft-capping (fp16 / bf16 models)."""
    lib = _lib.load()
    _lib.require_device(query, "query")
    if query.dim() != 4 or key.dim() != 4:
        raise ValueError("expected query [b, hq, s, d] and key [b, hkv, s, d]")
    b, hq, s, d = query.shape
    hkv = key.shape[1]
    if key.shape[0] != b or key.shape[2] != s or key.shape[3] != d or hq % hkv:
        raise ValueError(f"incompatible query {tuple(query.shape)} / key {tuple(key.shape)}")
    if query.dtype != key.dtype:
        raise ValueError("query and key must share a dtype")
    q = query.contiguous()
    k = key.contiguous()
    dev = q.device
    ws_bytes = lib.nq_score_real_workspace(b, hq, s)
    ws = workspace(dev, ws_bytes)
    lm = None if softcap is None else logit_map(q.dtype, softcap, dev)
    with torch.cuda.device(dev):
        st = lib.nq_score_real(_addr(q), _addr(k), _lib.dtype_code(q.dtype), b, hq, hkv, s, d,
                               ctypes.c_float(scaling), _window(sliding_window, s), _addr(lm), _addr(importance),
                               _addr(ws), ws_bytes, ctypes.c_void_p(_lib.current_stream_handle(dev)))
    _lib.check(st, "nq_score_real")


def attention_real(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scaling: float,
                   importance: torch.Tensor = None, sliding_window=None, softcap=None) -> torch.Tensor:
    """Causal attention output [b, hq, s, d] with eager_attention_forward's roundings
    (nq_attention_real), and importance[b, s] += the layer's column sums when given;
    sliding_window and softcap as for score_real_accumulate."""
    lib = _lib.load()
    _lib.require_device(query, "query")
    if query.dim() != 4 or key.dim() != 4 or value.shape != key.shape:
        raise ValueError("expected query [b, hq, s, d] and key / value [b, hkv, s, d]")
    b, hq, s, d = query.shape
    hkv = key.shape[1]
    if key.shape[0] != b or key.shape[2] != s or key.shape[3] != d or hq % hkv:
        raise ValueError(f"incompatible query {tuple(query.shape)} / key {tuple(key.shape)}")
    if not (query.dtype == key.dtype == value.dtype) or query.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("query, key and value must share an fp16 or bf16 dtype")
    if d not in (64, 128):
        raise ValueError(f"head_dim {d} unsupported (64, 128)")
    q, k, v = (t.contiguous() for t in (query, key, value))
    q, k, v = (t if t.data_ptr() % 16 == 0 else t.clone() for t in (q, k, v))
    dev = q.device
    out = torch.empty_like(q)
    ws_bytes = lib.nq_attention_real_workspace(b, hq, hkv, s, d)
    ws = workspace(dev, ws_bytes)
    lm = None if softcap is None else logit_map(q.dtype, softcap, dev)
    with torch.cuda.device(dev):
        st = lib.nq_attention_real(_addr(q), _addr(k), _addr(v), _lib.dtype_code(q.dtype), b, hq, hkv, s, d,
                                   ctypes.c_float(scaling), _window(sliding_window, s), _addr(lm),
                                   _addr(importance), _addr(out), _addr(ws), ws_bytes,
                                   ctypes.c_void_p(_lib.current_stream_handle(dev)))
    _lib.check(st, "nq_attention_real")
    return out


def _model_eager(module):
    mod = sys.modules.get(type(module).__module__)
    fn = getattr(mod, "eager_attention_forward", None)
    if fn is None:
        raise RuntimeError(f"{type(module).__name__} has no eager_attention_forward to wrap")
    return fn


def real_importance(model, input_ids: torch.Tensor, fused_attention: bool = True) -> torch.Tensor:
    """importance [batch, seq] averaged over layers, from one scoring forward pass.

    fused_attention=False keeps the model's own attention for every layer's
    output (nq_score_real then adds the column sums), as for models the fused
    kernel does not cover."""
    from transformers import AttentionInterface
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    b, s = input_ids.shape
    imp = torch.zeros(b, s, dtype=torch.float32, device=input_ids.device)
    calls = [0]
    prev = model.config._attn_implementation

    checked = {}

    def wrapped(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
        s_q, s_k = query.shape[2], key.shape[2]
        window = _window(kwargs.get("sliding_window", getattr(module, "sliding_window", None)), s_k)
        softcap = kwargs.get("softcap")
        # Attention sinks (gpt-oss: an extra softmax column per head) change the
        # probabilities the reference column-sums; the kernels do not add them.
        if kwargs.get("s_aux") is not None or kwargs.get("sinks") is not None:
            raise NotImplementedError(
                "the real scorer kernel does not implement attention sinks (s_aux); "
                "use scorer='key-key' for this model")
        if softcap is not None and query.dtype not in (torch.float16, torch.bfloat16):
            raise NotImplementedError(
                f"the real scorer kernel implements logit soft-capping for fp16 / bf16 models (got {query.dtype})")
        # The kernels implement the causal mask with an optional sliding window.
        # The mask tensor is shared by the layers of one type, so each one is
        # checked once.
        mkey = (None if attention_mask is None else attention_mask.data_ptr(),
                None if attention_mask is None else tuple(attention_mask.shape), window)
        if mkey not in checked:
            checked[mkey] = mask_is_causal(attention_mask, s_q, s_k, window)
        if not checked[mkey]:
            raise NotImplementedError(
                "the real scorer kernels implement causal attention with an optional sliding window; this "
                "layer's attention mask is neither (padding, chunked or bidirectional attention); use "
                "scorer='key-key' for this model or input")
        sc = scaling if scaling is not None else query.shape[-1] ** -0.5
        eager = prev == "eager" or prev is None
        if (fused_attention and eager and dropout == 0.0 and not module.training
                and query.dtype in (torch.float16, torch.bfloat16)
                and query.shape[-1] in (64, 128) and s_k == s_q):
            # the layer output comes from the same kernels as the column sums,
            # with eager's roundings and mask, and P is never stored
            out = attention_real(query, key, value, float(sc), imp, sliding_window=window or None, softcap=softcap)
            calls[0] += 1
            return out.transpose(1, 2).contiguous(), None
        base = _model_eager(module) if eager else ALL_ATTENTION_FUNCTIONS[prev]
        out, _ = base(module, query, key, value, attention_mask, scaling=scaling, dropout=dropout, **kwargs)
        score_real_accumulate(query, key, imp, float(sc), sliding_window=window or None, softcap=softcap)
        calls[0] += 1
        return out, None

    with _lock:
        AttentionInterface.register(_NAME, wrapped)
        # transformers builds the attention mask per implementation name; give the
        # wrapper the mask format of the implementation it wraps (eager: the 4D
        # additive causal mask), or the scoring pass would run unmasked.
        from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS
        ALL_MASK_ATTENTION_FUNCTIONS.register(_NAME, ALL_MASK_ATTENTION_FUNCTIONS[prev or "eager"])
        model.config._attn_implementation = _NAME
        try:
            with torch.no_grad():
                model(input_ids, use_cache=False)
        finally:
            model.config._attn_implementation = prev
    if calls[0] == 0:
        raise RuntimeError(
            "the scoring forward pass ran no attention layer through the wrapper; "
            "the model does not dispatch attention through transformers' AttentionInterface")
    return imp / calls[0]
