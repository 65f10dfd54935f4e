"""Real-attention importance through one scoring forward pass (pipeline.py:784-836).

The reference runs model(input_ids, output_attentions=True) under eager
attention and column-sums the returned [batch, heads, seq, seq] probabilities
of every layer.  Here the model runs with an attention wrapper registered in
transformers' AttentionInterface: each layer's attention is computed by the
model's own implementation, and its (post-RoPE) queries and keys go to the
nq_score_real kernel, which accumulates the same column sums without
materialising the probabilities (causal, GQA, HF eager dtype roundings).
"""

from __future__ import annotations

import ctypes
import sys
import threading

import torch

from . import _lib
from .ops import _addr

_lock = threading.Lock()
_NAME = "nexusquant_real_scorer"


def score_real_accumulate(query: torch.Tensor, key: torch.Tensor, importance: torch.Tensor,
                          scaling: float) -> None:
    """importance[b, s] += mean over query heads of causal column sums (one layer)."""
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
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        st = lib.nq_score_real(_addr(q), _addr(k), _lib.dtype_code(q.dtype), b, hq, hkv, s, d,
                               ctypes.c_float(scaling), _addr(importance), _addr(ws), ws_bytes,
                               ctypes.c_void_p(_lib.current_stream_handle(dev)))
    _lib.check(st, "nq_score_real")


def _model_eager(module):
    mod = sys.modules.get(type(module).__module__)
    fn = getattr(mod, "eager_attention_forward", None)
    if fn is None:
        raise RuntimeError(f"{type(module).__name__} has no eager_attention_forward to wrap")
    return fn


def real_importance(model, input_ids: torch.Tensor) -> torch.Tensor:
    """importance [batch, seq] averaged over layers, from one scoring forward pass."""
    from transformers import AttentionInterface
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    b, s = input_ids.shape
    imp = torch.zeros(b, s, dtype=torch.float32, device=input_ids.device)
    calls = [0]
    prev = model.config._attn_implementation

    def wrapped(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
        window = kwargs.get("sliding_window", getattr(module, "sliding_window", None))
        if window is not None and window < query.shape[2]:
            raise NotImplementedError("the real scorer kernel implements full causal attention only")
        # Logit soft-capping (Gemma-2: tanh(x / cap) * cap) and attention sinks
        # (gpt-oss: an extra softmax column per head) change the probabilities
        # the reference column-sums; the kernel computes plain causal softmax.
        if kwargs.get("softcap") is not None:
            raise NotImplementedError(
                "the real scorer kernel does not implement attention logit soft-capping "
                f"(softcap={kwargs['softcap']}); use scorer='key-key' for this model")
        if kwargs.get("s_aux") is not None or kwargs.get("sinks") is not None:
            raise NotImplementedError(
                "the real scorer kernel does not implement attention sinks (s_aux); "
                "use scorer='key-key' for this model")
        if prev == "eager" or prev is None:
            base = _model_eager(module)
        else:
            base = ALL_ATTENTION_FUNCTIONS[prev]
        sc = scaling if scaling is not None else query.shape[-1] ** -0.5
        out, _ = base(module, query, key, value, attention_mask, scaling=scaling, dropout=dropout, **kwargs)
        score_real_accumulate(query, key, imp, float(sc))
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
