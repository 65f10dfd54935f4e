"""The C-ABI library builds, loads and exports every symbol include/nexusquant_amd.h declares.

No compute call is made here (no GPU in the build container).
"""

import ctypes
import os
import re
import subprocess

import pytest

from nexusquant_amd import _lib
from nexusquant_amd.build import LIB_PATH

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nexusquant_amd.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nq_[a-z0-9_]+)\s*\(", text)))


def test_library_is_built_in_tree():
    assert os.path.exists(LIB_PATH), "run python -m nexusquant_amd.build"


def test_every_declared_symbol_is_exported_and_bound():
    lib = ctypes.CDLL(LIB_PATH)
    names = declared_functions()
    assert names, "header declares no functions"
    for name in names:
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
    assert sorted(_lib.SIGNATURES) == names, "ctypes signature table out of sync with the header"


@pytest.mark.parametrize("cname,pystruct", [("nq_quant_desc", _lib.QuantDesc), ("nq_codes_desc", _lib.CodesDesc),
                                            ("nq_page_desc", _lib.PageDesc), ("nq_attn_desc", _lib.AttnDesc),
                                            ("nq_merge_desc", _lib.MergeDesc)])
def test_struct_layout_matches_the_c_compiler(tmp_path, cname, pystruct):
    """ctypes offsets of every descriptor field equal gcc's offsetof on the header."""
    fields = [f[0] for f in pystruct._fields_]
    prog = ["#include <stddef.h>", "#include <stdio.h>", f'#include "{HEADER}"', "int main(void){",
            f'printf("%zu\\n", sizeof({cname}));']
    prog += [f'printf("%zu\\n", offsetof({cname}, {f}));' for f in fields]
    prog += ["return 0;}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(prog))
    exe = tmp_path / "layout"
    subprocess.check_call(["gcc", "-o", str(exe), str(src)])
    out = [int(x) for x in subprocess.check_output([str(exe)]).split()]
    assert out[0] == ctypes.sizeof(pystruct)
    assert out[1:] == [getattr(pystruct, f).offset for f in fields]


def test_abi_version_and_error_calls_need_no_gpu():
    lib = _lib.load()
    assert lib.nq_abi_version() == _lib.ABI_VERSION == 8
    assert isinstance(lib.nq_last_error(), bytes)


def test_library_was_built_from_these_sources():
    # the loader refuses a stale library; this names the mismatch directly
    from nexusquant_amd.build import source_hash
    lib = ctypes.CDLL(LIB_PATH)
    lib.nq_source_hash.restype = ctypes.c_char_p
    assert lib.nq_source_hash().decode() == source_hash(), "stale libnqamd.so: rebuild"


def test_loader_refuses_a_stale_library(monkeypatch):
    # a library whose embedded hash differs from the sources must not load
    from nexusquant_amd import build as nqbuild
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "source_hash", lambda: "0" * 16)
    with pytest.raises(_lib.NexusQuantError, match="other sources"):
        _lib.load()
    monkeypatch.setattr(_lib, "source_hash", nqbuild.source_hash)
    monkeypatch.setattr(_lib, "_lib", None)
    assert _lib.load().nq_abi_version() == _lib.ABI_VERSION


def test_noalloc_keykey_rejects_shapes_beyond_its_scratch_without_a_gpu():
    # the size check runs on the host before any HIP call or pointer use, so
    # dummy pointers are never dereferenced
    lib = _lib.load()
    b, h, s, obs = 1, 64, 131072, 96          # 12 MiB of row statistics > 8 MiB
    assert lib.nq_score_keykey_workspace(b, h, s, obs) > (8 << 20)
    assert lib.nq_score_keykey_workspace(1, 64, 131072, 64) == (8 << 20)
    dummy = ctypes.c_void_p(256)
    st = lib.nq_score_keykey_noalloc(dummy, _lib.NQ_F16, b, h, s, 128, obs, ctypes.c_float(128 ** -0.5),
                                     dummy, None)
    assert st == -1 and b"scratch" in lib.nq_last_error()
    st = lib.nq_score_keykey_noalloc(dummy, _lib.NQ_F16, 0, h, s, 128, obs, ctypes.c_float(1.0), dummy, None)
    assert st == -1


def test_grid_limits_are_checked_on_the_host_without_a_gpu():
    # A dispatch's grid is at most 2^32 - 1 work-items per dimension; shapes
    # beyond what a launch can cover are refused before any HIP call, and the
    # dummy pointers are never dereferenced.
    lib = _lib.load()
    dummy = ctypes.c_void_p(256)
    d = _lib.CodesDesc()
    d.n_tensors, d.batch, d.heads, d.seq = 65535, 1, 8, 1 << 27   # 2^30 rows per tensor
    d.head_dim, d.levels, d.is_key = 128, 8, 0
    d.syms = d.cosets = d.scales = d.out = dummy
    d.hadamard_scale = 1.0
    assert lib.nq_dequantize(ctypes.byref(d), None) == -1
    assert b"grid too large" in lib.nq_last_error()
    # the nibble kernels stride over a capped grid; only absurd row counts are refused
    assert lib.nq_nibble_pack(dummy, 1 << 41, 128, dummy, None) == -1
    assert b"bad geometry" in lib.nq_last_error()
    assert lib.nq_nibble_unpack(dummy, 1 << 41, 64, 128, dummy, None) == -1
    assert b"bad geometry" in lib.nq_last_error()
    # the rANS histogram's bins are uint32: one call takes at most 2^32 - 1 codes
    assert lib.nq_rans_histogram(ctypes.c_void_p(4096), 1 << 32, 4, dummy, None) == -1
    assert b"2^32 - 1" in lib.nq_last_error()
    # the rANS compaction stores word pairs: words must be 4-byte aligned
    odd = ctypes.c_void_p(4098)
    assert lib.nq_rans_compact(dummy, dummy, dummy, 4096, 2048, odd, None) == -1
    assert b"4-byte aligned" in lib.nq_last_error()
