"""GPU parity of the code kernels: dequantize, int8 2p codes, temporal deltas."""

import numpy as np
import pytest
import torch

from oracle import codes as C
from oracle import spec as S
from oracle import torch_ref as T

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _quant(D, L, key, dtype=torch.float16, shape=(2, 3, 150), seed=0):
    from nexusquant_amd.ops import quantize_tensors
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, D, generator=g)
    x[..., ::16] *= 6
    x = x.to(dtype).to(DEV)
    rec, cd = quantize_tensors([x], is_key=key, levels=L, rope_base=10000.0, codes=True)
    return x, rec[0], cd[0]


def _same_fp16(a, b):
    a = a.cpu().numpy()
    b = b.cpu().numpy()
    diff = a.view(np.uint16) != b.view(np.uint16)
    return bool(np.all(~diff | ((a == 0) & (b == 0))))


@pytest.mark.parametrize("D,L,key", [(128, 8, True), (128, 4, False), (128, 2, True), (128, 16, False),
                                     (64, 8, True), (256, 4, False), (256, 16, True), (96, 4, True),
                                     (96, 8, False)])
def test_dequantize_reproduces_fused_reconstruction(D, L, key):
    from nexusquant_amd.codec import dequantize
    print(f"[gpu] dequant D={D} L={L} key={key}", flush=True)
    _, rec, cd = _quant(D, L, key, seed=D + L)
    out = dequantize([cd], rope_base=10000.0)[0]
    torch.cuda.synchronize()
    assert _same_fp16(out, rec)


@pytest.mark.parametrize("D,L", [(128, 8), (128, 4), (128, 2), (256, 16), (64, 4)])
def test_int8_codes_and_deltas_match_oracle(D, L):
    from nexusquant_amd.codec import codes_int8, delta_decode
    print(f"[gpu] int8 codes D={D} L={L}", flush=True)
    x, rec, cd = _quant(D, L, False, seed=7 * D + L)
    ref = S.quant_rows(x.float().cpu().numpy().reshape(-1, D), L)
    two_p = C.codes_2p(ref["sym"], ref["coset"], L)
    got = codes_int8([cd])[0].cpu().numpy().reshape(-1, D)
    assert np.array_equal(got, two_p)
    assert np.array_equal(got, T.lattice_codes_2p(torch.from_numpy(ref["p"])).numpy())
    b, h, s = cd.scales.shape
    d = codes_int8([cd], delta=True)[0]
    want = C.delta_tokens(two_p.reshape(b * h, s, D))
    assert np.array_equal(d.cpu().numpy().reshape(b * h, s, D), want)
    back = delta_decode([d])[0].cpu().numpy().reshape(-1, D)
    assert np.array_equal(back, two_p)
    # vLLM dequant convention (code * 0.5) * scale equals the lattice point times the scale
    sc = cd.scales.cpu().numpy().reshape(-1, 1)
    assert np.array_equal((got.astype(np.float32) * 0.5) * sc, ref["p"] * sc)


@pytest.mark.parametrize("D,L,seq", [(128, 8, 64), (128, 4, 65), (128, 2, 1), (128, 16, 130), (64, 16, 37),
                                     (64, 2, 130), (64, 4, 200), (64, 8, 63), (256, 16, 63), (256, 4, 129),
                                     (128, 8, 300), (64, 4, 513), (256, 2, 257)])
def test_int8_codes_of_any_symbol_bytes_match_oracle(D, L, seq):
    """Random symbol and coset bytes, so every symbol value the packed format can
    hold appears (also those above L, which the quantizer never writes); three
    tensors per launch; tiles cut by seq (one row, exactly one tile, one past)
    and streams longer than one block's run of tiles."""
    from nexusquant_amd.codec import codes_int8
    from nexusquant_amd.ops import PackedCodes
    print(f"[gpu] int8 codes of random bytes D={D} L={L} seq={seq}", flush=True)
    rng = np.random.default_rng(1000 * D + 10 * L + seq)
    b, h, n_t = 2, 3, 3
    n = b * h * seq
    raw, codes = [], []
    for _ in range(n_t):
        syms = rng.integers(0, 256, (b, h, seq, D // 8 * C.bits_for(L)), dtype=np.uint8)
        cos = rng.integers(0, 256, (b, h, seq, D // 64), dtype=np.uint8)
        sc = rng.random((b, h, seq), dtype=np.float32)
        raw.append((syms, cos))
        codes.append(PackedCodes(syms=torch.from_numpy(syms).to(DEV), cosets=torch.from_numpy(cos).to(DEV),
                                 scales=torch.from_numpy(sc).to(DEV), levels=L, head_dim=D, padded_dim=D,
                                 is_key=False))
    got = codes_int8(codes)
    deltas = codes_int8(codes, delta=True)
    torch.cuda.synchronize()
    for i, (syms, cos) in enumerate(raw):
        want = C.codes_2p(C.unpack_symbols(syms.reshape(n, -1), L, D), C.unpack_cosets(cos.reshape(n, -1), D // 8), L)
        assert np.array_equal(got[i].cpu().numpy().reshape(n, D), want), i
        d = deltas[i].cpu().numpy().reshape(b * h, seq, D)
        assert np.array_equal(d, C.delta_tokens(want.reshape(b * h, seq, D))), i


def test_nqc1_container_roundtrip_and_ratio():
    from nexusquant_amd.codec import codes_int8, pack_nqc1, unpack_nqc1
    print("[gpu] nqc1", flush=True)
    layers = {}
    for li in range(3):
        _, _, ck = _quant(128, 8, True, shape=(1, 2, 300), seed=li)
        _, _, cv = _quant(128, 4, False, shape=(1, 2, 300), seed=10 + li)
        layers[li] = (ck, cv)
    packed = pack_nqc1(layers, zstd_level=3)
    assert packed["ratio"] > 3.0
    out = unpack_nqc1(packed["blob"])
    assert out["key_bits"] == 3 and out["value_bits"] == 2
    for li in range(3):
        for r in range(2):
            want = codes_int8([layers[li][r]])[0]
            assert torch.equal(out["codes"][2 * li + r].reshape(want.shape), want)
            assert np.array_equal(out["scales"][2 * li + r].reshape(-1),
                                  layers[li][r].scales.cpu().numpy().reshape(-1))


def test_c2_shaped_layer_properties_over_every_row():
    """One Llama-3-70B layer at full length (bf16 [1, 8, 131072, 128], K3 keys and K2
    values): checks that hold for every row, independent of size.  The codes dequantize
    to the fused reconstruction bit for bit; every int8 code 2p is within +-L; scales
    are finite and non-negative; token deltas and the rANS stream round-trip exactly."""
    from nexusquant_amd.codec import codes_int8, delta_decode, dequantize
    from nexusquant_amd.entropy import rans_decode, rans_encode
    from nexusquant_amd.ops import quantize_tensors
    print("[gpu] C2-shaped layer, whole-tensor properties", flush=True)
    g = torch.Generator(device=DEV).manual_seed(21)
    for key, L, scale in ((True, 8, 1.0), (False, 4, 0.5)):
        x = (torch.randn(1, 8, 131072, 128, device=DEV, generator=g) * scale).to(torch.bfloat16)
        rec, cd = quantize_tensors([x], is_key=key, levels=L, rope_base=500000.0, codes=True)
        rec, cd = rec[0], cd[0]
        back = dequantize([cd], rope_base=500000.0)[0]
        torch.cuda.synchronize()
        same = (back.view(torch.int16) == rec.view(torch.int16)) | ((back == 0) & (rec == 0))
        assert bool(same.all()), "dequantized codes differ from the fused reconstruction"
        c = codes_int8([cd])[0]
        assert int(c.abs().max()) <= L
        assert bool(torch.isfinite(cd.scales).all() & (cd.scales >= 0).all())
        d = codes_int8([cd], delta=True)[0]
        assert torch.equal(delta_decode([d])[0].reshape(c.shape), c)
        st = rans_encode(c, L)
        assert torch.equal(rans_decode(st), c)
        del x, rec, cd, back, c, d, st
        torch.cuda.empty_cache()
