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


def e8stream_cases():
    """(name, quantized [n, 8], scales, levels) of the encode_e8 container fixture:
    scaled half- and integer-coordinate points, per-group or single scales."""
    rng = np.random.default_rng(77)

    def scaled(p, s):
        return (p * s.reshape(-1, 1)).astype(np.float32)

    p8 = rng.integers(-8, 9, (600, 8)) / 2
    s8 = rng.uniform(0.01, 2.0, 600).astype(np.float32)
    p4 = rng.integers(-2, 3, (500, 8)).astype(np.float64)
    s4 = rng.uniform(0.05, 1.0, 500).astype(np.float32)
    p16 = rng.integers(-16, 17, (300, 8)) / 2
    s16 = np.array([0.37], np.float32)
    p2 = rng.integers(-6, 7, (200, 8)) / 2           # beyond +-1: clipped at levels 2
    s2 = rng.uniform(0.5, 1.5, 200).astype(np.float32)
    pt = rng.integers(-4, 5, (64, 8)).astype(np.float64)
    st = np.full(64, 1e-9, np.float32)                # clamped to 1e-8, zero in fp16
    return [
        ("half8", scaled(p8, s8), s8, 8),
        ("int4", scaled(p4, s4), s4, 4),
        ("scalar16", scaled(p16, np.full(300, 0.37, np.float32)), s16, 16),
        ("clip2", scaled(p2, s2), s2, 2),
        ("tiny", scaled(pt, st), st, 8),
        ("fp16in", scaled(p8[:128], s8[:128]).astype(np.float16), s8[:128], 8),
        ("empty", np.zeros((0, 8), np.float32), np.zeros(0, np.float32), 8),
    ]


E8STREAM_NAMES = [c[0] for c in e8stream_cases()]


def e8_entropy_input():
    """x of the e8_quantize_with_entropy case: last dim 60 (padded to 64)."""
    return (np.random.default_rng(78).standard_normal((2, 3, 40, 60)) * 0.5).astype(np.float32)
