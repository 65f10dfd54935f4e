"""GPU parity of the vLLM page caller and the paged decode-attention consumer.

- nq_page_encode / nq_page_decode: bit for bit against the Tier-B spec
  (oracle/nq_spec.c), within tolerance of the reference's fixture.
- nq_page_logits and nq_paged_attention: within tolerance of the Tier-A
  restatement / the reference's fixture (fp32 sums in another order; the
  fused attention also skips the per-token fp16 rounding of decoded values).
- nibble packing: exact.
"""

import math

import numpy as np
import pytest
import torch

from oracle import spec as S
from oracle import torch_ref as T

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
BASE = {"b2": 10000.0, "b3": 500000.0, "b4": 10000.0}


def _np16(t):
    return t.detach().cpu().numpy()


def _same_fp16(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    return bool(np.all((a.view(np.uint16) == b.view(np.uint16)) | ((a == 0) & (b == 0))))


def _tables(pos, d, base, h):
    c, s = T.rope_cos_sin(torch.as_tensor(pos).float(), d, base)
    return np.tile(c.numpy(), (h, 1)), np.tile(s.numpy(), (h, 1))


def _page(h, n, d, dtype, seed, pos_hi=200000):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(h, n, d, generator=g) * 2
    k[:, :, :3] *= 6
    v = torch.randn(h, n, d, generator=g) * 0.5
    pos = torch.randint(0, pos_hi, (n,), generator=g, dtype=torch.int32)
    return k.to(dtype), v.to(dtype), pos


@pytest.mark.parametrize("bits,d,dtype", [(2, 128, torch.float16), (3, 128, torch.float32), (4, 64, torch.float16),
                                          (2, 256, torch.bfloat16), (3, 128, torch.float16), (4, 128, torch.float32)])
def test_page_encode_decode_bitexact_vs_spec(bits, d, dtype):
    from nexusquant_amd.vllm_backend import NexusQuantKVCompressor
    print(f"[gpu] page codec bits={bits} d={d} {dtype}", flush=True)
    h, n = 4, 40
    base = 500000.0
    comp = NexusQuantKVCompressor(head_dim=d, bits=bits, rope_base=base)
    k, v, pos = _page(h, n, d, dtype, seed=bits * 100 + d)
    page = comp.compress_page(k.to(DEV), v.to(DEV), pos.to(DEV))
    kd, vd = comp.decompress_page(page)
    torch.cuda.synchronize()
    c, s = _tables(pos, d, base, h)
    L = 2 ** bits
    for x, key, codes, scales, dec in ((k, True, page.key_codes, page.key_scales, kd),
                                       (v, False, page.value_codes, page.value_scales, vd)):
        rows = x.float().numpy().reshape(-1, d)
        want_c, want_s, _ = S.page_encode(rows, L, c if key else None, s if key else None)
        assert np.array_equal(_np16(codes).reshape(-1, d), want_c)
        assert np.array_equal(_np16(scales).reshape(-1).view(np.uint16), want_s.view(np.uint16))
        want_d = S.page_decode(want_c, want_s, key, c if key else None, s if key else None)
        assert _same_fp16(_np16(dec).reshape(-1, d), want_d)
    assert page.num_valid == n and page.positions.dtype == torch.int32


@pytest.mark.parametrize("tag,bits", [("b2", 2), ("b3", 3), ("b4", 4)])
def test_pages_within_tolerance_of_reference_fixture(golden, tag, bits):
    from nexusquant_amd.vllm_backend import CompressedPage, NexusQuantKVCompressor
    print(f"[gpu] page fixture {tag}", flush=True)
    g = golden("vllm_pages")
    base = BASE[tag]
    k, v, pos = (torch.from_numpy(g[f"{tag}_{n}"]) for n in ("k", "v", "pos"))
    h, n, d = k.shape
    comp = NexusQuantKVCompressor(head_dim=d, bits=bits, rope_base=base)
    page = comp.compress_page(k.to(DEV), v.to(DEV), pos.to(DEV))
    c, s = _tables(pos, d, base, h)
    for role, key, codes in (("k", True, page.key_codes), ("v", False, page.value_codes)):
        got = _np16(codes).reshape(-1, 8)
        ref = g[f"{tag}_{role}c"].reshape(-1, 8)
        _, _, margin = S.page_encode(g[f"{tag}_{role}"].astype(np.float32).reshape(-1, d), 2 ** bits,
                                     c if key else None, s if key else None)
        mism = (got != ref).any(1)
        assert mism.mean() <= 1e-2 and np.all(margin.reshape(-1)[mism] < 1e-5)
    # decode and logits of the reference's own page
    ref_page = CompressedPage(*(torch.from_numpy(g[f"{tag}_{n}"]).to(DEV) for n in ("kc", "vc", "ks", "vs", "pos")),
                              num_valid=n)
    kd, vd = comp.decompress_page(ref_page)
    for got, name in ((kd, "kdec"), (vd, "vdec")):
        a = _np16(got).astype(np.float32).reshape(-1, d)
        r = g[f"{tag}_{name}"].astype(np.float32).reshape(-1, d)
        tol = np.spacing(np.maximum(np.abs(a), np.abs(r)).astype(np.float16)).astype(np.float32)
        assert np.all(np.abs(a - r) <= tol + 1e-6 * np.abs(r).max(1, keepdims=True))
    q = torch.from_numpy(g[f"{tag}_q"])
    lg = comp.decompress_for_attention(ref_page, q.to(DEV)).cpu().numpy()
    ref = g[f"{tag}_logits"]
    keys32 = T.vllm_decompress_keys_fp32(*(torch.from_numpy(g[f"{tag}_{n}"]) for n in ("kc", "ks", "pos")), base)
    bound = (q.float().norm(dim=-1)[:, :, None] * keys32.norm(dim=-1)[:, None, :]).numpy() / math.sqrt(d)
    assert np.all(np.abs(lg - ref) <= 1e-5 * bound + 1e-6)


def test_decompress_for_attention_fp32_and_bf16_queries():
    from nexusquant_amd.vllm_backend import NexusQuantKVCompressor
    print("[gpu] page logits dtypes", flush=True)
    comp = NexusQuantKVCompressor(head_dim=128, bits=3, rope_base=10000.0)
    k, v, pos = _page(8, 33, 128, torch.float16, seed=4)
    page = comp.compress_page(k.to(DEV), v.to(DEV), pos.to(DEV))
    for qdt in (torch.float32, torch.bfloat16, torch.float16):
        q = torch.randn(8, 5, 128, generator=torch.Generator().manual_seed(5)).to(qdt)
        lg = comp.decompress_for_attention(page, q.to(DEV)).cpu()
        ref = T.vllm_decompress_for_attention(page.key_codes.cpu(), page.key_scales.cpu(), pos, q, 10000.0)
        assert torch.allclose(lg, ref, rtol=1e-4, atol=1e-4)


def test_nibble_pack_unpack_match_reference(golden):
    from nexusquant_amd.vllm_backend import NexusQuantKVCompressor as C
    print("[gpu] nibbles", flush=True)
    g = golden("vllm_pages")
    codes = torch.from_numpy(g["nib_codes"]).to(DEV)
    packed = C.pack_codes_nibble(codes)
    assert np.array_equal(packed.cpu().numpy(), g["nib_packed"])
    assert np.array_equal(C.unpack_codes_nibble(packed, 33).cpu().numpy(), g["nib_unpacked"])
    even = torch.randint(-4, 5, (7, 128), dtype=torch.int8).to(DEV)
    assert torch.equal(C.unpack_codes_nibble(C.pack_codes_nibble(even), 128), even)


def _fixture_cache(g):
    from nexusquant_amd.vllm_backend import CompressedPage
    cache = {}
    for i in range(6):
        cache[i] = CompressedPage(*(torch.from_numpy(g[n][i]).to(DEV)
                                    for n in ("fwd_kc", "fwd_vc", "fwd_ks", "fwd_vs", "fwd_pos")), num_valid=16)
    return cache


def _close_fp16(got, ref, rel_l2=1e-3, bf16=False):
    """Attended outputs: within 2^-9 of the row's largest entry (a few fp16 ulps
    of it), plus one bf16 ulp of the entry for bf16 outputs, which round the fp16
    result once more; and 1e-3 relative L2 overall -- 2^-9, bf16's rounding
    bound, for bf16 outputs: an fp16 result one ulp off the reference's moves
    the bf16 rounding by a whole bf16 ulp (2^-8) in about 8 % of the entries."""
    a = np.asarray(got, np.float32)
    r = np.asarray(ref, np.float32)
    if bf16:
        rel_l2 = max(rel_l2, 2.0 ** -9)
    assert np.linalg.norm(a - r) <= rel_l2 * max(np.linalg.norm(r), 1e-30)
    scale = np.abs(r).max(axis=-1, keepdims=True)
    tol = 2.0 ** -9 * scale + 1e-6 + (2.0 ** -7 * np.abs(r) if bf16 else 0.0)
    assert np.all(np.abs(a - r) <= tol)


def test_paged_forward_matches_reference_fixture(golden):
    from nexusquant_amd.vllm_backend import NexusQuantKVCompressor, NexusQuantPagedAttention
    print("[gpu] paged forward fixture", flush=True)
    g = golden("vllm_pages")
    attn = NexusQuantPagedAttention(NexusQuantKVCompressor(head_dim=128, bits=2, rope_base=10000.0))
    cache = _fixture_cache(g)
    query = torch.from_numpy(g["fwd_query"]).to(DEV)
    out = attn.forward(query, cache, cache, [[0, 1, 2], [3, 99, 4], [5], [2, 0]],
                       torch.from_numpy(g["fwd_ctx"]))
    torch.cuda.synchronize()
    ref = g["fwd_out"]
    got = out.cpu().numpy()
    assert np.all(got[2] == 0) and np.all(ref[2] == 0)  # empty row
    _close_fp16(got, ref)


def _oracle_forward(cache, query, tables, ctx, base, group):
    pages = {}
    for bid, p in cache.items():
        kc, vc, ks, vs, pos = (t.cpu() for t in (p.key_codes, p.value_codes, p.key_scales, p.value_scales,
                                                  p.positions))
        if group > 1:
            kc, vc, ks, vs = (t.repeat_interleave(group, dim=0) for t in (kc, vc, ks, vs))
        pages[bid] = (kc, vc, ks, vs, pos)
    return T.vllm_paged_forward(query.cpu(), pages, tables, ctx, base)


@pytest.mark.parametrize("group,qdt", [(1, torch.float16), (2, torch.float16), (4, torch.float16),
                                       (8, torch.float16), (1, torch.float32), (2, torch.bfloat16)])
def test_paged_forward_long_context_gqa_and_dtypes(group, qdt):
    from nexusquant_amd.vllm_backend import NexusQuantKVCompressor, NexusQuantPagedAttention
    print(f"[gpu] paged forward group={group} {qdt}", flush=True)
    kv, d, base = 2, 128, 500000.0
    comp = NexusQuantKVCompressor(head_dim=d, bits=3, rope_base=base)
    attn = NexusQuantPagedAttention(comp)
    gen = torch.Generator().manual_seed(group * 7 + 1)
    cache = {}
    work = []
    sizes = [16] * 70 + [5, 600, 16, 1]  # many 16-token pages, a partial page, one page larger than a chunk
    for bid, n in enumerate(sizes):
        k = (torch.randn(kv, n, d, generator=gen) * 2).to(torch.float16)
        v = (torch.randn(kv, n, d, generator=gen) * 0.5).to(torch.float16)
        pos = torch.arange(n, dtype=torch.int32) + 16 * bid
        work.append((k.to(DEV), v.to(DEV), pos))
    for bid, page in enumerate(comp.compress_pages(work)):
        cache[bid] = page
    tables = [list(range(74)), [71, 5, 3, 200, 72, 73], [9], [0, 1, 2]]
    ctx = [70 * 16 + 5 + 600 + 10, 10 ** 6, 0, -7]
    query = torch.randn(4, kv * group, d, generator=gen).to(qdt)
    out = attn.forward(query.to(DEV), cache, cache, tables, torch.tensor(ctx))
    torch.cuda.synchronize()
    assert out.dtype == qdt
    ref = _oracle_forward(cache, query, tables, ctx, base, group)
    _close_fp16(out.float().cpu().numpy(), ref.float().numpy(), bf16=qdt == torch.bfloat16)


@pytest.mark.parametrize("d,group,qdt,vmul", [(64, 8, torch.float16, 1.0), (256, 8, torch.float16, 1.0),
                                              (256, 4, torch.bfloat16, 1.0), (64, 2, torch.float32, 1.0),
                                              (128, 8, torch.float16, 1e-4), (128, 1, torch.float16, 2e3)])
def test_paged_forward_head_dims_and_value_ranges(d, group, qdt, vmul):
    """Every head_dim with 8 and fewer query heads per kv head; values scaled
    down (row scales near fp16's subnormals) and up (scales near 2^6) so the
    value weights' fp16 hi/lo split is exercised at both ends of its range."""
    from nexusquant_amd.vllm_backend import NexusQuantKVCompressor, NexusQuantPagedAttention
    print(f"[gpu] paged forward d={d} group={group} {qdt} vmul={vmul}", flush=True)
    kv, base = 2, 10000.0
    comp = NexusQuantKVCompressor(head_dim=d, bits=2, rope_base=base)
    attn = NexusQuantPagedAttention(comp)
    gen = torch.Generator().manual_seed(d + group)
    work = []
    sizes = [16] * 40 + [3, 40, 16]
    for bid, n in enumerate(sizes):
        k = (torch.randn(kv, n, d, generator=gen) * 2).to(torch.float16)
        v = (torch.randn(kv, n, d, generator=gen) * vmul).to(torch.float16)
        pos = torch.arange(n, dtype=torch.int32) + 16 * bid
        work.append((k.to(DEV), v.to(DEV), pos))
    cache = dict(enumerate(comp.compress_pages(work)))
    tables = [list(range(43)), [41, 7, 42], [40]]
    ctx = [40 * 16 + 3 + 40 + 16, 10 ** 6, 2]
    query = torch.randn(3, kv * group, d, generator=gen).to(qdt)
    out = attn.forward(query.to(DEV), cache, cache, tables, torch.tensor(ctx))
    torch.cuda.synchronize()
    ref = _oracle_forward(cache, query, tables, ctx, base, group)
    _close_fp16(out.float().cpu().numpy(), ref.float().numpy(), bf16=qdt == torch.bfloat16)


@pytest.mark.parametrize("d,group,qdt", [(128, 8, torch.float16), (64, 2, torch.bfloat16), (256, 4, torch.float32)])
def test_paged_forward_rows_of_many_chunks(d, group, qdt):
    """Rows of 66 chunks (33.6K tokens): each of the combine's 32 thread groups
    sums more than one chunk (rows of fewer than 32 chunks, the case of the
    tests above, give each group at most one)."""
    from nexusquant_amd.vllm_backend import NexusQuantKVCompressor, NexusQuantPagedAttention
    print(f"[gpu] paged forward, 66 chunks per row, d={d} group={group} {qdt}", flush=True)
    kv, base = 1, 500000.0
    comp = NexusQuantKVCompressor(head_dim=d, bits=2, rope_base=base)
    attn = NexusQuantPagedAttention(comp)
    gen = torch.Generator().manual_seed(3 * d + group)
    n_pages = 2100  # x 16 tokens = 33600 = 65.6 chunks of 512
    k = (torch.randn(n_pages, kv, 16, d, generator=gen) * 2).to(torch.float16)
    v = (torch.randn(n_pages, kv, 16, d, generator=gen) * 0.5).to(torch.float16)
    work = [(k[i].to(DEV), v[i].to(DEV), torch.arange(16, dtype=torch.int32) + 16 * i) for i in range(n_pages)]
    cache = dict(enumerate(comp.compress_pages(work)))
    tables = [list(range(n_pages)), list(range(n_pages))[::-1]]
    ctx = [16 * n_pages, 16 * n_pages - 9]
    query = torch.randn(2, kv * group, d, generator=gen).to(qdt)
    out = attn.forward(query.to(DEV), cache, cache, tables, torch.tensor(ctx))
    torch.cuda.synchronize()
    ref = _oracle_forward(cache, query, tables, ctx, base, group)
    _close_fp16(out.float().cpu().numpy(), ref.float().numpy(), bf16=qdt == torch.bfloat16)


def test_paged_forward_at_a_1m_token_context():
    """One row of 1,048,573 tokens in 1024-token pages (2048 chunks, pages larger
    than a chunk): the combine's groups each sum 64 chunks."""
    from nexusquant_amd.vllm_backend import NexusQuantKVCompressor, NexusQuantPagedAttention
    print("[gpu] paged forward, 1M-token context", flush=True)
    kv, d, base, group, size, n_pages = 1, 128, 500000.0, 8, 1024, 1024
    comp = NexusQuantKVCompressor(head_dim=d, bits=2, rope_base=base)
    attn = NexusQuantPagedAttention(comp)
    gen = torch.Generator().manual_seed(5)
    work = []
    for i in range(n_pages):
        k = (torch.randn(kv, size, d, generator=gen) * 2).to(torch.float16)
        v = (torch.randn(kv, size, d, generator=gen) * 0.5).to(torch.float16)
        work.append((k.to(DEV), v.to(DEV), torch.arange(size, dtype=torch.int32) + size * i))
    cache = dict(enumerate(comp.compress_pages(work)))
    del work
    tables = [list(range(n_pages))]
    ctx = [size * n_pages - 3]
    query = torch.randn(1, kv * group, d, generator=gen).half()
    out = attn.forward(query.to(DEV), cache, cache, tables, torch.tensor(ctx))
    torch.cuda.synchronize()
    ref = _oracle_forward(cache, query, tables, ctx, base, group)
    _close_fp16(out.float().cpu().numpy(), ref.float().numpy())


def test_paged_plan_reuse_across_queries():
    from nexusquant_amd.vllm_backend import NexusQuantKVCompressor, NexusQuantPagedAttention
    print("[gpu] paged plan reuse", flush=True)
    comp = NexusQuantKVCompressor(head_dim=64, bits=4, rope_base=10000.0)
    attn = NexusQuantPagedAttention(comp)
    gen = torch.Generator().manual_seed(3)
    work = [(torch.randn(4, 16, 64, generator=gen).half().to(DEV), torch.randn(4, 16, 64, generator=gen).half().to(DEV),
             torch.arange(16, dtype=torch.int32) + 16 * i) for i in range(40)]
    cache = dict(enumerate(comp.compress_pages(work)))
    tables = [list(range(40)), list(range(20, 40))]
    plan = attn.plan(cache, tables, [640, 300])
    for step in range(3):
        q = torch.randn(2, 4, 64, generator=gen).half()
        out = attn.run(plan, q.to(DEV))
        ref = _oracle_forward(cache, q, tables, [640, 300], 10000.0, 1)
        _close_fp16(out.cpu().numpy(), ref.numpy())


def test_compress_and_cache_follows_reference_semantics():
    from nexusquant_amd.vllm_backend import NexusQuantKVCompressor, NexusQuantPagedAttention
    print("[gpu] compress_and_cache", flush=True)
    comp = NexusQuantKVCompressor(head_dim=128, bits=2, rope_base=10000.0)
    attn = NexusQuantPagedAttention(comp)
    gen = torch.Generator().manual_seed(8)
    key = torch.randn(10, 4, 128, generator=gen).half()
    value = torch.randn(10, 4, 128, generator=gen).half()
    slots = torch.tensor([32, 33, 34, 35, 36, 37, 64, 65, 66, 9])
    kcache, vcache = {}, {}
    attn.compress_and_cache(key.to(DEV), value.to(DEV), kcache, vcache, slots.to(DEV))
    # the reference's block-size heuristic returns 4: blocks slot // 4, positions slot % 4
    assert attn._infer_block_size(slots) == 4
    assert sorted(kcache) == [2, 8, 9, 16] and kcache is not vcache and kcache[8] is vcache[8]
    for bid, page in kcache.items():
        idx = [i for i, sl in enumerate(slots.tolist()) if sl // 4 == bid]
        pos = torch.tensor([slots[i].item() % 4 for i in idx], dtype=torch.int32)
        kc, vc, ks, vs = T.vllm_compress_page(key[idx].permute(1, 0, 2), value[idx].permute(1, 0, 2), pos, 2, 10000.0)
        assert torch.equal(page.positions.cpu(), pos)
        mism = (page.key_codes.cpu().reshape(-1, 8) != kc.reshape(-1, 8)).any(1).float().mean().item()
        assert mism <= 2e-2
