"""Host side of the real scorer (CPU): the soft-cap logit table and the check
that a layer's attention mask is the causal (+ sliding window) pattern the
kernels implement, against transformers' own mask builders."""

import pytest
import torch

from nexusquant_amd.scoring import logit_map, mask_is_causal


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("cap", [50.0, 30.0])
def test_logit_map_is_the_eager_softcap_chain_and_monotone(dtype, cap):
    t = logit_map(dtype, cap, "cpu")
    assert t.dtype == torch.int16 and t.numel() == 65536
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    w = bits.view(dtype)
    got = t.view(dtype)
    finite = torch.isfinite(w)
    # Gemma-2's eager attention (modeling_gemma2.py:203-206), one op at a time in the model dtype
    want = torch.tanh(w / cap) * cap
    assert torch.equal(got[finite], want[finite])
    # monotone non-decreasing over the finite values in increasing order: the
    # kernels take a row's maximum before the map
    order = torch.argsort(w[finite].float())
    vals = got[finite][order].float()
    assert bool((vals[1:] >= vals[:-1]).all())
    assert float(vals.abs().max()) <= cap


def _masks(window, pad=False, s=40):
    from transformers import MistralConfig
    from transformers.masking_utils import create_causal_mask, create_sliding_window_causal_mask
    cfg = MistralConfig(hidden_size=64, num_attention_heads=4, num_key_value_heads=2, num_hidden_layers=1,
                        sliding_window=window)
    cfg._attn_implementation = "eager"
    emb = torch.zeros(2, s, 64, dtype=torch.float16)
    am = torch.ones(2, s, dtype=torch.long)
    if pad:
        am[1, :5] = 0
    pos = torch.arange(s)[None].expand(2, -1)
    kw = dict(config=cfg, inputs_embeds=emb, attention_mask=am, past_key_values=None, position_ids=pos)
    build = create_sliding_window_causal_mask if window else create_causal_mask
    return build(**kw)


def test_mask_check_accepts_transformers_causal_and_sliding_masks():
    s = 40
    assert mask_is_causal(_masks(None), s, s, 0)
    assert mask_is_causal(_masks(12), s, s, 12)
    assert not mask_is_causal(_masks(12), s, s, 0)       # a window the caller did not name
    assert not mask_is_causal(_masks(12), s, s, 13)
    assert not mask_is_causal(_masks(None), s, s, 12)
    # boolean masks (True = attend) are read as such
    i, j = torch.arange(s)[:, None], torch.arange(s)[None, :]
    assert mask_is_causal((j <= i)[None, None], s, s, 0)


def test_mask_check_refuses_padding_bidirectional_and_missing_masks():
    s = 40
    assert not mask_is_causal(_masks(None, pad=True), s, s, 0)
    assert not mask_is_causal(_masks(12, pad=True), s, s, 12)
    assert not mask_is_causal(torch.zeros(1, 1, s, s), s, s, 0)   # everything attends
    assert not mask_is_causal(None, s, s, 0)
    assert not mask_is_causal(_masks(None), s, s + 1, 0)           # cached prefix: not the scoring pass


def test_real_scorer_refuses_softcapping_for_fp32_models():
    # the soft-cap table covers the 65536 values of an fp16 / bf16 logit; an
    # fp32 model is refused before any score is accumulated (no GPU reached)
    from transformers import Gemma2Config, Gemma2ForCausalLM
    from nexusquant_amd.scoring import real_importance
    cfg = Gemma2Config(vocab_size=128, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=16, max_position_embeddings=256,
                       attn_logit_softcapping=50.0, sliding_window=64)
    cfg._attn_implementation = "eager"
    torch.manual_seed(0)
    model = Gemma2ForCausalLM(cfg).eval()
    with pytest.raises(NotImplementedError, match="soft-capping"):
        real_importance(model, torch.randint(0, 128, (1, 20)))
    assert model.config._attn_implementation == "eager"
