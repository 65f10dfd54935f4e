"""GPU parity of the reference's single-stream E8 container (encode_e8 /
decode_e8 / e8_quantize_with_entropy) against the bytes the reference wrote
and against the oracle."""

import numpy as np
import pytest
import torch

from conftest import load_golden
from golden.make_golden_cases import E8STREAM_NAMES, e8_entropy_input
from oracle import rans_ref as R

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("name", E8STREAM_NAMES)
def test_container_bytes_match_the_reference(name):
    from nexusquant_amd.entropy import decode_e8, encode_e8
    print(f"[gpu] encode_e8 fixture {name}", flush=True)
    f = load_golden("e8stream")
    blob = f[f"{name}_blob"].tobytes()
    q = torch.from_numpy(f[f"{name}_quantized"]).to(DEV)
    s = torch.from_numpy(f[f"{name}_scales"])
    assert encode_e8(q, s, levels=int(f[f"{name}_levels"])) == blob
    vals, sc = decode_e8(blob)
    assert not vals.is_cuda and vals.dtype == torch.float32
    assert np.array_equal(vals.numpy(), f[f"{name}_decoded"]) and np.array_equal(sc.numpy(), f[f"{name}_dscales"])
    dv, ds = decode_e8(blob, original_shape=(-1,), device=DEV)
    assert dv.is_cuda and np.array_equal(dv.cpu().numpy(), f[f"{name}_decoded"].reshape(-1))


def test_quantize_with_entropy_matches_the_reference():
    from nexusquant_amd.entropy import e8_quantize_with_entropy
    print("[gpu] e8_quantize_with_entropy", flush=True)
    f = load_golden("e8stream")
    x = torch.from_numpy(e8_entropy_input()).to(DEV)
    r = e8_quantize_with_entropy(x, levels=8)
    assert r["compressed_bytes"] == f["e2e_blob"].tobytes()
    assert np.array_equal(r["reconstructed"].cpu().numpy(), f["e2e_reconstructed"])
    assert np.array_equal(r["scale_factors"].cpu().numpy(), f["e2e_scale_factors"])
    for k, v in zip(f["e2e_keys"], f["e2e_values"]):
        assert float(r[str(k)]) == v, k
    for k, v in zip(f["e2e_stat_keys"], f["e2e_stat_values"]):
        assert float(r["entropy_stats"][str(k)]) == v, k


@pytest.mark.parametrize("levels,groups,half", [(8, 20000, True), (4, 12000, False), (16, 5000, True)])
def test_container_against_oracle_at_larger_sizes(levels, groups, half):
    from nexusquant_amd.entropy import decode_e8, encode_e8
    print(f"[gpu] encode_e8 vs oracle levels={levels} groups={groups}", flush=True)
    rng = np.random.default_rng(levels * groups)
    # center-heavy points, as the E8 quantizer's output is
    p = np.clip(np.round(rng.standard_normal((groups, 8)) * levels / 6 * (2 if half else 1)),
                -levels if half else -levels // 2, levels if half else levels // 2)
    p = p / 2 if half else p
    s = rng.uniform(0.01, 3.0, groups).astype(np.float32)
    q = (p * s[:, None]).astype(np.float32)
    blob = encode_e8(torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV), levels=levels)
    assert blob == R.encode_e8(q, s, levels)
    vals, sc = decode_e8(blob, device=DEV)
    want, want_sc = R.decode_e8(blob)
    assert np.array_equal(vals.cpu().numpy(), want) and np.array_equal(sc.cpu().numpy(), want_sc)


def test_million_symbol_roundtrip():
    # one chain over 2^20 symbols: decode(encode(x)) gives back the points
    # times the fp16-rounded scales
    from nexusquant_amd.entropy import decode_e8, encode_e8
    print("[gpu] encode_e8 2^20 symbols", flush=True)
    g = torch.Generator(device=DEV).manual_seed(9)
    p = torch.clamp(torch.round(torch.randn(1 << 17, 8, device=DEV, generator=g) * 2), -8, 8) / 2
    s = torch.rand(1 << 17, device=DEV, generator=g) + 0.1
    blob = encode_e8(p * s[:, None], s, levels=8)
    vals, sc = decode_e8(blob, device=DEV)
    assert torch.equal(vals, p * s.half().float()[:, None])


def test_roundtrip_above_2_24_symbols():
    # one chain over 2^24 + 64 symbols, above the chunk bound of earlier builds
    # (a whole [1, 8, 16384, 128] layer is 2^24 symbols)
    from nexusquant_amd.entropy import decode_e8, encode_e8
    print("[gpu] encode_e8 2^24 + 64 symbols", flush=True)
    g = torch.Generator(device=DEV).manual_seed(11)
    n_groups = (1 << 21) + 8
    p = torch.clamp(torch.round(torch.randn(n_groups, 8, device=DEV, generator=g) * 2), -8, 8) / 2
    s = torch.rand(n_groups, device=DEV, generator=g) + 0.1
    blob = encode_e8(p * s[:, None], s, levels=8)
    vals, _ = decode_e8(blob, device=DEV)
    assert torch.equal(vals, p * s.half().float()[:, None])
