"""Inputs of the temporal codec fixture (shared by make_golden.py and the tests)."""

import numpy as np


def temporal_cases():
    """(name, coords, n_tokens, use_delta, level) of the temporal codec fixture."""
    rng = np.random.default_rng(1234)
    walk = np.clip(np.cumsum(rng.integers(-1, 2, size=(48, 64)), axis=0), -8, 8).astype(np.int8).ravel()
    wide = np.clip(np.cumsum(rng.integers(-2, 3, size=(4, 1000)), axis=0), -16, 16).astype(np.int8).ravel()
    return [
        ("delta", walk, 48, True, 22),          # rows of 64: 16-byte words on the GPU
        ("raw", walk, 48, False, 22),
        ("level1", walk, 48, True, 1),
        ("ragged", walk[:3000], 48, True, 22),  # 48 does not divide 3000: no delta either way
        ("width12", rng.integers(-8, 9, 480).astype(np.int8), 40, True, 22),  # delta skipped, undone anyway
        ("width6", rng.integers(-8, 9, 60).astype(np.int8), 10, True, 22),    # 1-byte words
        ("wide", wide, 4, True, 6),             # rows of 1000: 4-byte words
        ("wrap", rng.integers(-300, 300, 256).astype(np.int32), 16, True, 22),  # astype(int8) wraps
        ("empty", np.zeros(0, np.int8), 1, True, 22),
    ]


CASE_NAMES = [c[0] for c in temporal_cases()]
