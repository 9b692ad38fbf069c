"""Test data generators restating the reference's own test helpers
(src/native/tests.rs:24-103) plus tolerance checks."""

import numpy as np

Q4_0 = 2
Q8_0 = 8
Q2_K = 10
Q3_K = 11
Q4_K = 12
Q5_K = 13
Q6_K = 14
IQ4_NL = 20
IQ4_XS = 23
IQ2_XXS = 16
IQ2_XS = 17
IQ3_XXS = 18
IQ3_S = 21
IQ2_S = 22
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18, IQ4_NL: 18, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210, IQ4_XS: 136,
               IQ2_XXS: 66, IQ2_XS: 74, IQ2_S: 82, IQ3_XXS: 98, IQ3_S: 110}
BLOCK_ELEMENTS = {Q8_0: 32, Q4_0: 32, IQ4_NL: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256,
                  IQ4_XS: 256, IQ2_XXS: 256, IQ2_XS: 256, IQ2_S: 256, IQ3_XXS: 256, IQ3_S: 256}
# the formats of the generic (planes) GPU path
PLANE_FORMATS = [Q8_0, Q4_0, IQ4_NL, Q2_K, Q3_K, Q5_K, Q6_K]
# the IQ2 / IQ3 formats, whose decode reads the grid tables
GRID_FORMATS = [IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S]


def synthetic_iq_grids(seed=1):
    """Stand-in grid tables (the real ones live in the external
    magnetar-provider-api crate, absent here), as the bench uses them."""
    from magnetar_gpu.workloads import synthetic_iq_grids as tables

    return tables(seed)


class Rng:
    """xorshift32 (src/native/tests.rs:34-43)."""

    def __init__(self, state):
        self.state = state & 0xFFFFFFFF

    def next(self):
        x = self.state
        x ^= (x << 13) & 0xFFFFFFFF
        x ^= x >> 17
        x ^= (x << 5) & 0xFFFFFFFF
        self.state = x
        return x


def half_offsets(fmt):
    """Byte offsets of each block's f16 scale fields (src/native/tests.rs:24-32)."""
    if fmt in (Q4_K, Q5_K):
        return [0, 2]
    return {Q6_K: [208], Q2_K: [80, 82], Q3_K: [108]}.get(fmt, [0])


def packed(fmt, rows, cols, seed):
    """A random packed matrix: random bytes, small positive f16 scales with
    exponent 3..7 (src/native/tests.rs:45-67). uint8 [rows, row_bytes]."""
    rng = Rng((seed * 2654435761 + 1) & 0xFFFFFFFF)
    bb, be = BLOCK_BYTES[fmt], BLOCK_ELEMENTS[fmt]
    blocks = rows * cols // be
    out = np.empty(blocks * bb, np.uint8)
    for i in range(blocks):
        blk = [rng.next() % 256 for _ in range(bb)]
        for at in half_offsets(fmt):
            exponent = 3 + rng.next() % 5
            bits = (exponent << 10) | (rng.next() % 1024)
            blk[at] = bits & 0xFF
            blk[at + 1] = bits >> 8
        out[i * bb:(i + 1) * bb] = blk
    return out.reshape(rows, cols // be * bb)


def activations(rows, cols, seed):
    """Uniform in [-1, 1] in 0.001 steps (src/native/tests.rs:69-75)."""
    rng = Rng(seed + 7)
    v = np.array([rng.next() % 2001 for _ in range(rows * cols)], dtype=np.float32)
    return (v / np.float32(1000.0) - np.float32(1.0)).astype(np.float32).reshape(rows, cols)


def assert_close_reference(actual, expected, what=""):
    """`assert_close` (src/native/tests.rs:91-103): |a - e| <= 2e-5 max(1, max|e|)."""
    scale = max(1.0, float(np.max(np.abs(expected)))) if expected.size else 1.0
    err = np.abs(actual.astype(np.float64) - expected.astype(np.float64))
    assert err.max(initial=0.0) <= 2e-5 * scale, f"{what}: max err {err.max()} vs {2e-5 * scale}"


def row_tolerance_violation(actual, expected):
    """Largest max|d| / (1e-3 ||row||_inf) over rows: <= 1 passes the
    stated output tolerance (max |d| <= 1e-3 ||row||_inf, f32 accumulate)."""
    a = actual.astype(np.float64)
    e = expected.astype(np.float64)
    norm = np.max(np.abs(e), axis=1)
    err = np.max(np.abs(a - e), axis=1)
    ratio = err / np.maximum(1e-3 * norm, 1e-30)
    return float(ratio.max(initial=0.0))


def assert_row_tolerance(actual, expected, what=""):
    assert actual.shape == expected.shape, f"{what}: shape {actual.shape} vs {expected.shape}"
    assert np.isfinite(actual).all() == np.isfinite(expected).all(), f"{what}: non-finite mismatch"
    r = row_tolerance_violation(actual, expected)
    assert r <= 1.0, f"{what}: max|d| is {r:.3f} x the 1e-3 ||row||_inf tolerance"
