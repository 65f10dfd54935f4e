"""Host-side logic of the drop-in API (no GPU needed)."""

import math

import pytest
import torch

import nexusquant_amd as nq
from nexusquant_amd import rope
from nexusquant_amd.hadamard import hadamard_constant
from oracle import torch_ref as T


class Cache:
    def __init__(self, ks, vs):
        self.key_cache, self.value_cache = list(ks), list(vs)


def test_cpu_tensors_are_refused_not_silently_computed():
    c = Cache([torch.randn(1, 2, 16, 128).half()], [torch.randn(1, 2, 16, 128).half()])
    with pytest.raises(RuntimeError, match=r"ROCm\) devices only"):
        nq.compress_kv_cache(c, mode="quant_only")


def test_unknown_mode_raises_value_error():
    with pytest.raises(ValueError, match="Unknown mode"):
        nq.compress_kv_cache(Cache([], []), mode="nope")


def test_hadamard_helpers_match_reference_restatement():
    for n in (2, 8, 64, 128, 256):
        assert torch.equal(nq.hadamard_matrix(n), T.hadamard_matrix(n))
        assert hadamard_constant(n) == T.hadamard_matrix(n)[0, 0].item()
    with pytest.raises(ValueError):
        nq.hadamard_matrix(96)
    assert [nq.next_power_of_2(x) for x in (1, 2, 3, 96, 128, 129)] == [1, 2, 4, 128, 128, 256]


@pytest.mark.parametrize("base,scaling", [
    (10000.0, None), (500000.0, None), (10000.0, {"type": "linear", "factor": 4.0}),
    (500000.0, {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                "high_freq_factor": 4.0, "original_max_position_embeddings": 8192})])
def test_host_rope_table_equals_reference_tables(base, scaling):
    c, s = rope.host_table(5000, 128, base, scaling)
    rc, rs = T.rope_cos_sin(torch.arange(5000, dtype=torch.float32), 128, base, scaling)
    assert torch.equal(c, rc) and torch.equal(s, rs)
    # a position's entry does not depend on the table length
    c2, s2 = rope.host_table(131072, 128, base, scaling)
    assert torch.equal(c2[:5000], c) and torch.equal(s2[:5000], s)


def test_quant_only_level_resolution():
    q = nq.NexusQuantQuantOnly(bits=3, key_bits=3, value_bits=2)
    assert (q.key_levels, q.value_levels) == (8, 4)
    q = nq.NexusQuantQuantOnly(bits=2)
    assert (q.key_levels, q.value_levels) == (4, 4)
