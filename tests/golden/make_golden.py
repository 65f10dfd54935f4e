"""Write golden fixtures from the real reference (run in the build container only).

The reference (jagmarques/nexusquant v0.5.0, mounted read-only at
/root/reference) is imported here, on the CPU, to record input/output vectors
for the functions whose exact results no closed form pins: the end-to-end
pipelines (dense-GEMM Hadamard and torch reduction order), the key-key scorer,
torch.topk keep masks, and the real-attention scorer through transformers'
eager attention.  Nothing under /root/reference is copied; only the numbers it
produces are stored, as small .npz files next to this script.

Usage:  python tests/golden/make_golden.py [/root/reference [evict_soft | vllm_pages | evict_merge | rans |
                                                              temporal_codec | e8stream |
                                                              real_scorer_window]]
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
sys.path.insert(0, REF)

from nexusquant.pipeline import (NexusQuantEvict, NexusQuantEvictTruncate,  # noqa: E402
                                 NexusQuantQuantOnly, compress_kv_cache)
from nexusquant.core.e8_lattice import E8Lattice  # noqa: E402
from nexusquant.core.rope_utils import inverse_rope, forward_rope  # noqa: E402

from make_golden_cases import e8_entropy_input, e8stream_cases, temporal_cases  # noqa: E402


class ListCache:
    def __init__(self, ks, vs):
        self.key_cache = list(ks)
        self.value_cache = list(vs)


def synth_kv(seed, n_layers, b, h, s, d, base, sink=False, dtype=torch.float16):
    """Keys: N(0,1) with 4 outlier channels x8 per head, then RoPE; values N(0, 0.5^2)."""
    g = torch.Generator().manual_seed(seed)
    ks, vs = [], []
    for _ in range(n_layers):
        kp = torch.randn(b, h, s, d, generator=g)
        for hi in range(h):
            ch = torch.randperm(d, generator=g)[:4]
            kp[:, hi, :, ch] *= 8
        if sink:
            kp[:, :, 0, :] *= 4
        k = forward_rope(kp, base=base)
        v = torch.randn(b, h, s, d, generator=g) * 0.5
        ks.append(k.to(dtype))
        vs.append(v.to(dtype))
    return ks, vs


def save(name, **arrays):
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **{k: (v.numpy() if torch.is_tensor(v) else np.asarray(v))
                                 for k, v in arrays.items()})
    print("wrote", path, os.path.getsize(path), "bytes")


def stack(ts):
    return torch.stack([t for t in ts])


def main():
    torch.manual_seed(0)

    # 1. E8 nearest point and per-row quantizer.
    g = torch.Generator().manual_seed(11)
    x = torch.randn(16384, 8, generator=g) * 1.7
    x[:64] = torch.round(x[:64] * 2) / 2          # exact half/integer ties
    x[64:128] = torch.round(x[64:128])           # integer points
    save("e8_nearest", x=x, p=E8Lattice.nearest_point(x.clone()))
    rows = torch.randn(512, 128, generator=g)
    rows[0] = 0.0
    save("e8_perhead", x=rows, q8=E8Lattice.quantize_perhead(rows.clone(), levels=8),
         q4=E8Lattice.quantize_perhead(rows.clone(), levels=4),
         q2=E8Lattice.quantize_perhead(rows.clone(), levels=2),
         q16=E8Lattice.quantize_perhead(rows.clone(), levels=16))

    # 2. RoPE at large positions (pins the host cos/sin table construction).
    kk = torch.randn(2, 64, 128, generator=g)
    save("rope_far", x=kk,
         inv=inverse_rope(kk, seq_offset=131008, base=500000.0),
         fwd=forward_rope(kk, seq_offset=131008, base=500000.0),
         inv_scaled=inverse_rope(kk, seq_offset=40000, base=500000.0,
                                 rope_scaling={"rope_type": "llama3", "factor": 8.0,
                                               "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                                               "original_max_position_embeddings": 8192}))

    # 3. Quant-only K3V2 (== NexusQuantEvict rate 0) and symmetric QuantOnly.
    for base, tag in ((10000.0, "b1e4"), (500000.0, "b5e5")):
        ks, vs = synth_kv(21, 2, 1, 2, 256, 128, base)
        c = ListCache([k.clone() for k in ks], [v.clone() for v in vs])
        nq = NexusQuantEvict(key_bits=3, value_bits=2, eviction_rate=0.0, rope_base=base)
        _, mask = nq.compress(c)
        c3 = ListCache([k.clone() for k in ks], [v.clone() for v in vs])
        compress_kv_cache(c3, mode="quant_only", rope_base=base)
        save(f"quant_only_{tag}", k_in=stack(ks), v_in=stack(vs),
             k_k3v2=stack(c.key_cache), v_k3v2=stack(c.value_cache), mask=mask,
             k_k3v3=stack(c3.key_cache), v_k3v3=stack(c3.value_cache), base=base)

    # 4. d = 256 quant-only K2V2; bf16 input K3V2.
    ks, vs = synth_kv(31, 1, 1, 2, 128, 256, 10000.0)
    c = ListCache([k.clone() for k in ks], [v.clone() for v in vs])
    NexusQuantEvict(bits=2, eviction_rate=0.0, rope_base=10000.0).compress(c)
    save("quant_only_d256", k_in=stack(ks), v_in=stack(vs), k_out=stack(c.key_cache),
         v_out=stack(c.value_cache))
    ks, vs = synth_kv(32, 1, 1, 2, 256, 128, 500000.0, dtype=torch.bfloat16)
    c = ListCache([k.clone() for k in ks], [v.clone() for v in vs])
    NexusQuantEvict(key_bits=3, value_bits=2, eviction_rate=0.0, rope_base=500000.0).compress(c)
    save("quant_only_bf16", k_in=stack(ks).float(), v_in=stack(vs).float(),
         k_out=stack(c.key_cache), v_out=stack(c.value_cache))

    # 5. Key-key scorer and keep masks, mask-mode eviction, b = 4 with a sink.
    ks, vs = synth_kv(41, 2, 4, 2, 256, 128, 10000.0, sink=True)
    nq = NexusQuantEvict(key_bits=3, value_bits=2, eviction_rate=0.25, sliding_window=32,
                         obs_window=32, rope_base=10000.0)
    imp = nq._score_importance(ks[0].float())
    c = ListCache([k.clone() for k in ks], [v.clone() for v in vs])
    _, mask = nq.compress(c)
    save("evict_mask_b4", k_in=stack(ks), v_in=stack(vs), importance=imp, mask=mask,
         k_out=stack(c.key_cache), v_out=stack(c.value_cache))

    # 6. Rate 0.6 K2V2, b = 1, plus boundary protection on 6 layers.
    ks, vs = synth_kv(51, 6, 1, 2, 128, 128, 10000.0, sink=True)
    nq = NexusQuantEvict(bits=2, eviction_rate=0.6, sliding_window=16, rope_base=10000.0,
                         protect_boundary=2)
    c = ListCache([k.clone() for k in ks], [v.clone() for v in vs])
    _, mask = nq.compress(c)
    save("evict_mask_boundary", k_in=stack(ks), v_in=stack(vs), mask=mask,
         k_out=stack(c.key_cache), v_out=stack(c.value_cache))

    # 7. Truncation (b = 1) at two rates.
    for rate in (0.25, 0.6):
        ks, vs = synth_kv(61, 2, 1, 2, 256, 128, 10000.0, sink=True)
        nq = NexusQuantEvictTruncate(key_bits=3, value_bits=2, eviction_rate=rate,
                                     sliding_window=32, rope_base=10000.0)
        c = ListCache([k.clone() for k in ks], [v.clone() for v in vs])
        _, n_kept = nq.compress(c)
        save(f"evict_truncate_r{int(rate * 100)}", k_in=stack(ks), v_in=stack(vs),
             n_kept=n_kept, k_out=stack(c.key_cache), v_out=stack(c.value_cache))

    # 8. Real-attention scorer through transformers' eager attention (tiny Llama).
    real_scorer_fixture()


def real_scorer_fixture():
    from transformers import LlamaConfig, LlamaForCausalLM
    import transformers.models.llama.modeling_llama as ml

    torch.manual_seed(71)
    cfg = LlamaConfig(vocab_size=128, hidden_size=256, intermediate_size=512,
                      num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                      max_position_embeddings=512, rope_theta=10000.0)
    cfg._attn_implementation = "eager"
    model = LlamaForCausalLM(cfg).eval()
    captured = []
    orig = ml.eager_attention_forward

    def spy(module, query, key, value, attention_mask, scaling, dropout=0.0, **kw):
        captured.append((query.detach().clone(), key.detach().clone(), float(scaling)))
        return orig(module, query, key, value, attention_mask, scaling, dropout, **kw)

    ml.eager_attention_forward = spy
    try:
        ids = torch.randint(0, 128, (1, 96), generator=torch.Generator().manual_seed(72))
        nq = NexusQuantEvict(scorer="real")
        imp = nq._score_importance_real(model, ids)
    finally:
        ml.eager_attention_forward = orig
    qs = torch.stack([q for q, _, _ in captured])
    kss = torch.stack([k for _, k, _ in captured])
    save("real_scorer", q=qs, k=kss, scaling=captured[0][2], importance=imp)


def real_scorer_window_fixtures():
    """The real scorer through transformers' eager attention on models whose
    masks or logits differ from plain causal softmax: a tiny Mistral with a
    sliding window shorter than the sequence, and a tiny Gemma-2 with logit
    soft-capping and alternating sliding-window / full layers.  fp16 weights
    on the CPU; per layer the post-RoPE q, k, scaling, window and soft-cap the
    eager attention received, and the reference's importance."""
    from transformers import Gemma2Config, Gemma2ForCausalLM, MistralConfig, MistralForCausalLM
    import transformers.models.gemma2.modeling_gemma2 as mg
    import transformers.models.mistral.modeling_mistral as mm

    seq = 160
    cases = {
        "real_scorer_mistral": (mm, MistralForCausalLM, MistralConfig(
            vocab_size=128, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
            num_attention_heads=4, num_key_value_heads=2, head_dim=64, max_position_embeddings=512,
            rope_theta=10000.0, sliding_window=48)),
        "real_scorer_gemma2": (mg, Gemma2ForCausalLM, Gemma2Config(
            vocab_size=128, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
            num_attention_heads=4, num_key_value_heads=2, head_dim=64, max_position_embeddings=512,
            rope_theta=10000.0, sliding_window=40, attn_logit_softcapping=50.0, final_logit_softcapping=30.0,
            query_pre_attn_scalar=64)),
    }
    for name, (mod, cls, cfg) in cases.items():
        torch.manual_seed(73)
        cfg._attn_implementation = "eager"
        model = cls(cfg).to(torch.float16).eval()
        captured = []
        orig = mod.eager_attention_forward

        def spy(module, query, key, value, attention_mask, *args, _orig=orig, **kw):
            captured.append((query.detach().clone(), key.detach().clone(), float(kw.get("scaling", args[0] if args
                                                                                       else module.scaling)),
                             kw.get("sliding_window"), kw.get("softcap")))
            return _orig(module, query, key, value, attention_mask, *args, **kw)

        mod.eager_attention_forward = spy
        try:
            ids = torch.randint(0, 128, (1, seq), generator=torch.Generator().manual_seed(74))
            nq = NexusQuantEvict(scorer="real")
            imp = nq._score_importance_real(model, ids)
        finally:
            mod.eager_attention_forward = orig
        save(name, q=torch.stack([c[0] for c in captured]), k=torch.stack([c[1] for c in captured]),
             scaling=np.array([c[2] for c in captured], np.float64),
             window=np.array([0 if c[3] is None else int(c[3]) for c in captured], np.int64),
             softcap=np.array([0.0 if c[4] is None else float(c[4]) for c in captured], np.float64),
             importance=imp)


def make_soft():
    """8. Soft eviction (pipeline.py:1129-1183): b = 2, K3V2 at rate 0.5, evicted
    rows at levels 2, first and last layer protected (cast to fp16 unmasked)."""
    ks, vs = synth_kv(81, 4, 2, 2, 128, 128, 10000.0, sink=True)
    nq = NexusQuantEvict(key_bits=3, value_bits=2, eviction_rate=0.5, sliding_window=16,
                         rope_base=10000.0, soft_eviction=True, protect_boundary=1)
    imp = nq._score_importance(ks[0].float())
    c = ListCache([k.clone() for k in ks], [v.clone() for v in vs])
    _, mask = nq.compress(c)
    save("evict_soft", k_in=torch.stack(ks), v_in=torch.stack(vs), importance=imp, mask=mask,
         k_out=torch.stack(c.key_cache), v_out=torch.stack(c.value_cache))


def make_merge():
    """10. Merge eviction (pipeline.py:961-1048): b = 2, 3 layers fp16, K3V2 at rate
    0.5, first/last layer protected; the merged values, survivors and outputs."""
    import torch.nn.functional as F
    ks, vs = synth_kv(101, 3, 2, 2, 96, 64, 10000.0, sink=True)
    nq = NexusQuantEvict(key_bits=3, value_bits=2, eviction_rate=0.5, sliding_window=8, rope_base=10000.0,
                         merge_eviction=True, protect_boundary=1)
    imp = nq._score_importance(ks[0].float())
    keep = nq._build_keep_mask(imp, 96, eviction_rate=0.5)
    survivors = []
    cent_all = []
    for bi in range(2):
        cs = None
        for v in vs:
            m = v[bi].float().mean(dim=0)
            cs = m if cs is None else cs + m
        cent = cs / len(vs)
        cent_all.append(cent)
        ev = (~keep[bi]).nonzero(as_tuple=True)[0]
        kp = keep[bi].nonzero(as_tuple=True)[0]
        cos = torch.mm(F.normalize(cent[ev], dim=-1), F.normalize(cent[kp], dim=-1).t())
        sv = torch.full((96,), -1, dtype=torch.int32)
        sv[ev] = kp[cos.argmax(dim=1)].to(torch.int32)
        survivors.append(sv)
    c = ListCache([k.clone() for k in ks], [v.clone() for v in vs])
    nq._apply_merge_eviction(c, keep, imp, 3)
    merged = torch.stack(c.value_cache)
    c2 = ListCache([k.clone() for k in ks], [v.clone() for v in vs])
    _, mask = nq.compress(c2)
    save("evict_merge", k_in=torch.stack(ks), v_in=torch.stack(vs), importance=imp, keep=keep,
         centroids=torch.stack(cent_all), survivor=torch.stack(survivors), v_merged=merged, mask=mask,
         k_out=torch.stack(c2.key_cache), v_out=torch.stack(c2.value_cache))


def make_rans():
    """11. rANS entropy coder (core/entropy_coder.py): symbol mapping, frequency
    table and the encoder's 16-bit word stream for E8 code streams at levels
    4, 8, 16, an integer-only stream, a skewed stream and a one-symbol stream."""
    from nexusquant.core import entropy_coder as ec
    from nexusquant.core.e8_lattice import E8Lattice
    g = torch.Generator().manual_seed(111)
    out = {}
    cases = []
    for L, n_rows in ((8, 96), (4, 64), (16, 48)):
        x = torch.randn(n_rows, 128, generator=g)
        amax = x.abs().amax(dim=-1, keepdim=True).clamp(min=1e-8)
        p = E8Lattice.nearest_point((x / (amax / (L / 2))).reshape(-1, 8)).clamp(-L / 2, L / 2)
        cases.append((f"l{L}", L, p.reshape(-1).numpy()))
    ints = torch.randint(-3, 4, (5000,), generator=g).float()
    cases.append(("int", 8, ints.numpy()))
    skew = torch.zeros(20000)
    skew[torch.randint(0, 20000, (37,), generator=g)] = 2.5
    skew[torch.randint(0, 20000, (5,), generator=g)] = -3.5
    cases.append(("skew", 8, skew.numpy()))
    cases.append(("one", 4, np.array([1.5], np.float32)))
    for tag, L, pts in cases:
        sym, has_half, alpha = ec._lattice_to_symbols(pts.astype(np.float32), L)
        freqs, cum = ec._build_freq_table(sym, alpha)
        words = ec._rans_encode(sym, freqs, cum)
        back = ec._rans_decode(words, len(sym), freqs, cum, alpha)
        assert np.array_equal(back, sym)
        out.update({f"{tag}_points": pts.astype(np.float32), f"{tag}_levels": L, f"{tag}_symbols": sym,
                    f"{tag}_has_half": int(has_half), f"{tag}_alphabet": alpha, f"{tag}_freqs": freqs,
                    f"{tag}_words": np.array(words, dtype=np.uint16)})
    save("rans", **out)


def make_vllm():
    """9. vLLM page caller and decode consumer (integrations/vllm_backend.py):
    compress_page / decompress_page / decompress_for_attention at bits 2, 3, 4
    (head_dim 128, 128, 64; fp16 and fp32 inputs; non-contiguous absolute
    positions), nibble packing, and NexusQuantPagedAttention.forward over 16-token
    pages with a missing block, a partial context, an empty row and a negative
    context length (Python slice semantics)."""
    from nexusquant.integrations.vllm_backend import NexusQuantKVCompressor, NexusQuantPagedAttention
    g = torch.Generator().manual_seed(91)
    out = {}
    cases = [("b2", 2, 128, torch.float16, torch.arange(16, dtype=torch.int32) * 3 + 5000),
             ("b3", 3, 128, torch.float32, torch.randint(0, 131072, (16,), generator=g, dtype=torch.int32)),
             ("b4", 4, 64, torch.float16, torch.arange(24, dtype=torch.int32) + 777)]
    for tag, bits, d, dt, pos in cases:
        n = pos.numel()
        comp = NexusQuantKVCompressor(head_dim=d, bits=bits, rope_base=500000.0 if tag == "b3" else 10000.0)
        k = (torch.randn(4, n, d, generator=g) * 2).to(dt)
        k[:, :, :3] *= 6
        v = (torch.randn(4, n, d, generator=g) * 0.5).to(dt)
        page = comp.compress_page(k, v, pos)
        kd, vd = comp.decompress_page(page)
        qry = torch.randn(4, 3, d, generator=g).to(torch.float16)
        logits = comp.decompress_for_attention(page, qry)
        out.update({f"{tag}_k": k, f"{tag}_v": v, f"{tag}_pos": pos,
                    f"{tag}_kc": page.key_codes, f"{tag}_vc": page.value_codes,
                    f"{tag}_ks": page.key_scales, f"{tag}_vs": page.value_scales,
                    f"{tag}_kdec": kd, f"{tag}_vdec": vd, f"{tag}_q": qry, f"{tag}_logits": logits})
    codes = torch.randint(-12, 13, (5, 3, 33), generator=g, dtype=torch.int8)
    out["nib_codes"] = codes
    out["nib_packed"] = NexusQuantKVCompressor.pack_codes_nibble(codes)
    out["nib_unpacked"] = NexusQuantKVCompressor.unpack_codes_nibble(out["nib_packed"], 33)
    # paged decode attention
    comp = NexusQuantKVCompressor(head_dim=128, bits=2, rope_base=10000.0)
    attn = NexusQuantPagedAttention(comp)
    cache = {}
    pk, pv, pp = [], [], []
    for bid in range(6):
        pos = torch.arange(16, dtype=torch.int32) + 16 * bid
        k = (torch.randn(4, 16, 128, generator=g) * 2).to(torch.float16)
        v = (torch.randn(4, 16, 128, generator=g) * 0.5).to(torch.float16)
        cache[bid] = comp.compress_page(k, v, pos)
        pk.append(k)
        pv.append(v)
        pp.append(pos)
    tables = [[0, 1, 2], [3, 99, 4], [5], [2, 0]]
    ctx = torch.tensor([40, 20, 0, -5], dtype=torch.int32)
    query = torch.randn(4, 4, 128, generator=g).to(torch.float16)
    fwd = attn.forward(query, cache, cache, tables, ctx)
    out.update({"fwd_k": torch.stack(pk), "fwd_v": torch.stack(pv), "fwd_pos": torch.stack(pp),
                "fwd_kc": torch.stack([cache[i].key_codes for i in range(6)]),
                "fwd_vc": torch.stack([cache[i].value_codes for i in range(6)]),
                "fwd_ks": torch.stack([cache[i].key_scales for i in range(6)]),
                "fwd_vs": torch.stack([cache[i].value_scales for i in range(6)]),
                "fwd_query": query, "fwd_ctx": ctx, "fwd_out": fwd})
    save("vllm_pages", **out)


def make_temporal():
    """compress_indices / decompress_indices bytes and outputs (temporal_codec.py:76-132)."""
    from nexusquant.core import temporal_codec as tc
    assert not tc._HAS_ZSTD, "fixture is for the zlib branch"
    out = {}
    for name, coords, n_tokens, use_delta, level in temporal_cases():
        blob = tc.compress_indices(coords, n_tokens, use_delta=use_delta, level=level)
        out[f"{name}_coords"] = coords
        out[f"{name}_meta"] = np.array([n_tokens, int(use_delta), level], np.int64)
        out[f"{name}_blob"] = np.frombuffer(blob, np.uint8)
        out[f"{name}_decoded"] = tc.decompress_indices(blob)
        if use_delta:
            out[f"{name}_delta"] = tc.temporal_delta_encode(coords.astype(np.int8), n_tokens)
    m = tc.measure_compression(out["delta_coords"], 48, fp16_bytes=48 * 64 * 2, scale_bytes=48 * 8 * 2)
    keys = sorted(m)
    out["measure_keys"] = np.array(keys)
    out["measure_values"] = np.array([float(m[k]) for k in keys])
    save("temporal_codec", **out)


def make_e8stream():
    """encode_e8 / decode_e8 containers and e8_quantize_with_entropy (entropy_coder.py:360-570)."""
    from nexusquant.core import entropy_coder as ec
    out = {}
    for name, q, s, levels in e8stream_cases():
        blob = ec.encode_e8(torch.from_numpy(q), torch.from_numpy(s), levels=levels)
        dq, ds = ec.decode_e8(blob)
        out.update({f"{name}_quantized": q, f"{name}_scales": s, f"{name}_levels": levels,
                    f"{name}_blob": np.frombuffer(blob, np.uint8), f"{name}_decoded": dq, f"{name}_dscales": ds})
    x = torch.from_numpy(e8_entropy_input())
    r = ec.e8_quantize_with_entropy(x, levels=8)
    keys = ["n_bytes_compressed", "n_bytes_uniform", "n_bytes_original", "rans_compression_ratio",
            "e8_base_ratio", "total_compression_ratio"]
    stats = sorted(r["entropy_stats"])
    out.update({"e2e_blob": np.frombuffer(r["compressed_bytes"], np.uint8), "e2e_reconstructed": r["reconstructed"],
                "e2e_scale_factors": r["scale_factors"], "e2e_keys": np.array(keys),
                "e2e_values": np.array([float(r[k]) for k in keys]), "e2e_stat_keys": np.array(stats),
                "e2e_stat_values": np.array([float(r["entropy_stats"][k]) for k in stats])})
    save("e8stream", **out)


if __name__ == "__main__":
    if sys.argv[2:] == ["evict_soft"]:
        make_soft()
    elif sys.argv[2:] == ["vllm_pages"]:
        make_vllm()
    elif sys.argv[2:] == ["evict_merge"]:
        make_merge()
    elif sys.argv[2:] == ["rans"]:
        make_rans()
    elif sys.argv[2:] == ["temporal_codec"]:
        make_temporal()
    elif sys.argv[2:] == ["e8stream"]:
        make_e8stream()
    elif sys.argv[2:] == ["real_scorer_window"]:
        real_scorer_window_fixtures()
    else:
        main()
        make_soft()
        make_vllm()
        make_merge()
        make_rans()
        make_temporal()
        make_e8stream()
        real_scorer_window_fixtures()
