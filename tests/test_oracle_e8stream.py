"""The encode_e8 container restated in oracle/rans_ref.py against the bytes
the reference wrote (tests/golden/e8stream.npz), on the CPU."""

import struct

import numpy as np
import pytest

from conftest import load_golden
from golden.make_golden_cases import E8STREAM_NAMES
from oracle import rans_ref as R


@pytest.mark.parametrize("name", E8STREAM_NAMES)
def test_oracle_container_equals_the_reference_bytes(name):
    f = load_golden("e8stream")
    blob = f[f"{name}_blob"].tobytes()
    q = f[f"{name}_quantized"].astype(np.float32)
    assert R.encode_e8(q, f[f"{name}_scales"], int(f[f"{name}_levels"])) == blob
    vals, sc = R.decode_e8(blob)
    assert vals.dtype == np.float32 and np.array_equal(vals, f[f"{name}_decoded"])
    assert np.array_equal(sc, f[f"{name}_dscales"])


def test_container_layout():
    f = load_golden("e8stream")
    blob = f["half8_blob"].tobytes()
    n_groups, levels, has_half, n_sym = struct.unpack_from("<IBBI", blob, 0)
    assert (n_groups, levels, has_half, n_sym) == (600, 8, 1, 4800)
    f_len, s_len, r_len = struct.unpack_from("<III", blob, 10)
    assert f_len == 2 + 2 * 17 and s_len == 2 * 600 and 22 + f_len + s_len + r_len == len(blob)
    # integer-only points use the L + 1 alphabet; one scale broadcasts
    assert struct.unpack_from("<IBBI", f["int4_blob"].tobytes(), 0)[2] == 0
    assert struct.unpack_from("<III", f["scalar16_blob"].tobytes(), 10)[1] == 2
    # the empty stream flushes the initial state 2^16 as the words (1, 0)
    e = f["empty_blob"].tobytes()
    assert e[-4:] == struct.pack("<HH", 1, 0) and len(e) == 46


def test_freq_table_against_the_reference_tables():
    g = load_golden("rans")
    for tag in ("l8", "l4", "l16", "int", "skew", "one"):
        assert np.array_equal(R.freq_table(g[f"{tag}_symbols"], int(g[f"{tag}_alphabet"])), g[f"{tag}_freqs"])
    # the empty-histogram rule: M // alphabet each, the remainder on symbol 0
    f = R.freq_table(np.zeros(0, np.int64), 9)
    assert f.sum() == R.M and f[0] == R.M // 9 + R.M % 9 and np.all(f[1:] == R.M // 9)
