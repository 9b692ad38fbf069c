"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each test checks an oracle function against something other than its own
formula: host F16C, the reference's known-answer vectors and test
invariants, exact arithmetic on hand-built blocks, numpy's IEEE
arithmetic, brute force, or a structural property of the format."""

import struct

import numpy as np
import pytest

import oracle
from helpers import IQ4_XS, Q4_K, activations, assert_close_reference, packed


def f32_bits(v):
    return struct.unpack("<I", struct.pack("<f", v))[0]


# ---- f16 ----------------------------------------------------------------

def test_f16_to_f32_exhaustive_against_f16c_and_numpy():
    """All 65,536 patterns: bit-identical to the F16C conversion the AVX2
    kernels use (src/native/quant.rs:1494-1502), and to numpy's."""
    ref = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    for bits in range(65536):
        a = oracle.f16_to_f32(bits)
        f = oracle.half_f16c(bits)
        assert f32_bits(a) == f32_bits(f), hex(bits)
        if not np.isnan(ref[bits]):
            assert f32_bits(a) == f32_bits(float(ref[bits])), hex(bits)


# ---- scale_min_k4 ---------------------------------------------------------

def _all_scale_mins(twelve):
    return [oracle.scale_min_k4(j, twelve) for j in range(8)]


def test_scale_min_k4_is_a_bijection_of_the_96_bits():
    """The 12 scale bytes hold eight 6-bit scales and eight 6-bit mins: every
    one of the 96 input bits must move exactly one output bit, and all 96
    output bits must be reached (a wrong shift or byte index breaks this)."""
    base = np.zeros(12, np.uint8)
    zero = _all_scale_mins(base)
    assert zero == [(0, 0)] * 8
    reached = set()
    for byte in range(12):
        for bit in range(8):
            t = base.copy()
            t[byte] = 1 << bit
            out = _all_scale_mins(t)
            changed = []
            for j, (sc, m) in enumerate(out):
                for which, v in (("sc", sc), ("m", m)):
                    for ob in range(6):
                        if (v >> ob) & 1:
                            changed.append((j, which, ob))
            assert len(changed) == 1, (byte, bit, changed)
            reached.add(changed[0])
    assert len(reached) == 96


@pytest.mark.parametrize("twelve,expected", [
    # all ones: every scale and min is 63
    ([0xFF] * 12, [(63, 63)] * 8),
    # low 6 bits of bytes 0..3 are the scales of sub-blocks 0..3
    ([0x3F] * 4 + [0] * 8, [(63, 0)] * 4 + [(0, 0)] * 4),
    # low 6 bits of bytes 4..7 are the mins of sub-blocks 0..3
    ([0] * 4 + [0x3F] * 4 + [0] * 4, [(0, 63)] * 4 + [(0, 0)] * 4),
    # bytes 8..11: low nibble = low 4 bits of scales 4..7, high nibble = mins 4..7
    ([0] * 8 + [0x0F] * 4, [(0, 0)] * 4 + [(15, 0)] * 4),
    ([0] * 8 + [0xF0] * 4, [(0, 0)] * 4 + [(0, 15)] * 4),
    # top 2 bits of bytes 0..3 / 4..7 are the high bits of scales / mins 4..7
    ([0xC0] * 4 + [0] * 8, [(0, 0)] * 4 + [(48, 0)] * 4),
    ([0] * 4 + [0xC0] * 4 + [0] * 4, [(0, 0)] * 4 + [(0, 48)] * 4),
    # distinct values per sub-block
    ([1, 2, 3, 4, 5, 6, 7, 8, 0x21, 0x43, 0x65, 0x87],
     [(1, 5), (2, 6), (3, 7), (4, 8), (1, 2), (3, 4), (5, 6), (7, 8)]),
])
def test_scale_min_k4_known_answers(twelve, expected):
    """Known answers from the GGUF Q4_K scale packing (ggml get_scale_min_k4,
    restated at src/native/quant.rs:46-57)."""
    assert _all_scale_mins(np.array(twelve, np.uint8)) == expected


# ---- Q4_K / IQ4_XS dequantization ----------------------------------------

def _f16(v):
    return int(np.array([v], np.float16).view(np.uint16)[0])


def _q4k_block(d, dmin, sc, mn, q):
    """A Q4_K block from its fields: the inverse of the GGUF layout (12
    scale bytes per the packing pinned above, q[j][i] in chunk j//2, low
    nibble for even j)."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([_f16(d)], np.uint16).view(np.uint8)
    blk[2:4] = np.array([_f16(dmin)], np.uint16).view(np.uint8)
    s = np.zeros(12, np.int64)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    blk[4:16] = s.astype(np.uint8)
    for j in range(8):
        for i in range(32):
            blk[16 + 32 * (j // 2) + i] |= np.uint8(q[j][i] << (4 * (j % 2)))
    assert [oracle.scale_min_k4(j, blk[4:16]) for j in range(8)] == list(zip(sc, mn))
    return blk


def test_q4k_dequant_identity_block():
    """d = 1, dmin = 0, every scale 1: each value is its 4-bit quant."""
    rng = np.random.default_rng(1)
    q = rng.integers(0, 16, (8, 32))
    blk = _q4k_block(1.0, 0.0, [1] * 8, [0] * 8, q)
    out = oracle.dequantize(Q4_K, blk, 1, 256)
    np.testing.assert_array_equal(out.reshape(8, 32), q.astype(np.float32))


def test_q4k_dequant_scales_and_mins_exact():
    """value = (d sc_j) q - dmin m_j. Every product of an f16, a 6-bit and a
    4-bit integer is exact in f32 (at most 21 significant bits), so the only
    rounding is the final difference: float64 arithmetic rounded once to f32
    gives the exact f32 answer."""
    rng = np.random.default_rng(2)
    for trial in range(50):
        d = float(np.float16(rng.uniform(1e-4, 0.05)))
        dmin = float(np.float16(rng.uniform(1e-4, 0.05)))
        sc = [int(v) for v in rng.integers(0, 64, 8)]
        mn = [int(v) for v in rng.integers(0, 64, 8)]
        q = rng.integers(0, 16, (8, 32))
        blk = _q4k_block(d, dmin, sc, mn, q)
        out = oracle.dequantize(Q4_K, blk, 1, 256).reshape(8, 32)
        exp = (np.array(sc, np.float64)[:, None] * d * q - (np.array(mn, np.float64) * dmin)[:, None])
        np.testing.assert_array_equal(out, exp.astype(np.float32))


def _iq4nl():
    import json
    import os

    with open(os.path.join(os.path.dirname(__file__), "golden", "gguf_iq4nl_codebook.json")) as f:
        return json.load(f)["kvalues_iq4nl"]


def test_iq4_codebook_matches_gguf_spec_fixture():
    """The IQ4_NL codebook lives in the external provider-api crate; it is
    pinned to the GGUF specification's kvalues_iq4nl (committed fixture)."""
    T = _iq4nl()
    blk = np.zeros(136, np.uint8)
    blk[0:2] = np.array([_f16(1.0)], np.uint16).view(np.uint8)
    # every run scale ls = 33 -> 1
    blk[2:4] = np.array([0xAAAA], np.uint16).view(np.uint8)  # high bits 2 -> 32
    blk[4:8] = 0x11  # low nibbles 1 -> 33 - 32 = 1
    for j in range(8):
        for l in range(16):
            blk[8 + 16 * j + l] = (l & 15) | (((15 - l) & 15) << 4)
    out = oracle.dequantize(IQ4_XS, blk, 1, 256).reshape(8, 32)
    for j in range(8):
        assert list(out[j, :16]) == [float(T[l]) for l in range(16)]
        assert list(out[j, 16:]) == [float(T[15 - l]) for l in range(16)]


def test_iq4xs_scale_layout_known_answers():
    """IQ4_XS per-run scales: 6-bit ls_j = low nibble j of scales_l | 2 bits
    j of scales_h << 4, value ls_j - 32 (GGUF IQ4_XS layout)."""
    six = np.array([0b11100100, 0b00011011, 0x10, 0x32, 0x54, 0x76], np.uint8)
    # scales_h = 0x1BE4: bit pairs j=0..7: 0,1,2,3,3,2,1,0
    high = [0, 1, 2, 3, 3, 2, 1, 0]
    low = [0, 1, 2, 3, 4, 5, 6, 7]
    exp = [(lo | (hi << 4)) - 32 for lo, hi in zip(low, high)]
    assert list(oracle.iq4_xs_scales(six)) == exp
    # each run's scale multiplies its codebook values exactly (11+6+7 bits)
    blk = np.zeros(136, np.uint8)
    blk[0:2] = np.array([_f16(0.25)], np.uint16).view(np.uint8)
    blk[2:8] = six
    blk[8:] = 0xF0  # low nibble 0 -> -127, high nibble 15 -> 113
    T = _iq4nl()
    out = oracle.dequantize(IQ4_XS, blk, 1, 256).reshape(8, 32)
    for j in range(8):
        assert np.all(out[j, :16] == np.float32(0.25 * exp[j] * T[0]))
        assert np.all(out[j, 16:] == np.float32(0.25 * exp[j] * T[15]))


@pytest.mark.parametrize("fmt", [Q4_K, IQ4_XS])
def test_dequant_random_blocks_match_spec_decoder(fmt):
    """Reference-style random blocks (src/native/tests.rs:45-67) through a
    vectorized float64 decoder written from the GGUF layouts: exact."""
    rows, cols = 3, 512
    w = packed(fmt, rows, cols, 11)
    got = oracle.dequantize(fmt, w, rows, cols)
    blocks = w.reshape(-1, 144 if fmt == Q4_K else 136)
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    if fmt == Q4_K:
        dmin = blocks[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
        s = blocks[:, 4:16].astype(np.int64)
        sc = np.concatenate([s[:, 0:4] & 63, (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)], axis=1)
        mn = np.concatenate([s[:, 4:8] & 63, (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)], axis=1)
        qs = blocks[:, 16:].astype(np.int64).reshape(-1, 4, 32)
        q = np.stack([qs & 15, qs >> 4], axis=2).reshape(-1, 8, 32)
        val = (d[:, None, None] * sc[:, :, None]) * q - (dmin[:, None] * mn)[:, :, None]
    else:
        T = np.array(_iq4nl(), np.int64)
        h = blocks[:, 2].astype(np.int64) | (blocks[:, 3].astype(np.int64) << 8)
        lo = blocks[:, 4:8].astype(np.int64)
        ls = np.stack([((lo[:, j // 2] >> (4 * (j % 2))) & 15) | (((h >> (2 * j)) & 3) << 4)
                       for j in range(8)], axis=1) - 32
        qs = blocks[:, 8:].astype(np.int64).reshape(-1, 8, 16)
        idx = np.concatenate([qs & 15, qs >> 4], axis=2)
        val = (d[:, None, None] * ls[:, :, None]) * T[idx]
    np.testing.assert_array_equal(got, val.reshape(rows, cols).astype(np.float32))


def test_decode_run_matches_dequant_definition():
    """`dequantize_row` (quant.rs:1702-1711) is scale[p] q - min[p] per run."""
    w = packed(Q4_K, 1, 256, 5)
    full = oracle.dequantize(Q4_K, w, 1, 256)[0]
    for run in range(8):
        q, scale, mn = oracle.decode_run(Q4_K, w[0], run)
        exp = (scale[np.arange(32) // 16] * q.astype(np.float32) - mn[np.arange(32) // 16]).astype(np.float32)
        np.testing.assert_array_equal(full[32 * run:32 * run + 32], exp)


# ---- int8 activation quantization ----------------------------------------

def _quantize_numpy(x):
    """quantize_rows by numpy's IEEE float32 arithmetic."""
    x = x.astype(np.float32).reshape(-1, 32)
    ax = np.abs(x)
    ax = np.where(np.isnan(ax), np.float32(0), ax)
    amax = ax.max(axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.rint(x / d[:, None])
    r = np.where(np.isnan(r), 0, np.clip(r, -128, 127))
    r = np.where(amax[:, None] == 0, 0, r).astype(np.int8)
    sums = np.stack([r[:, :16].astype(np.int32).sum(1), r[:, 16:].astype(np.int32).sum(1)], axis=1)
    return r.reshape(-1), d, sums


def test_quantize_rows_matches_numpy_ieee():
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(32 * 200), rng.uniform(-1e-30, 1e-30, 32 * 4),
                        rng.standard_normal(32 * 4) * 1e30]).astype(np.float32)
    v, s, h = oracle.quantize_rows(x)
    ev, es, eh = _quantize_numpy(x)
    np.testing.assert_array_equal(v, ev)
    np.testing.assert_array_equal(s.view(np.uint32), es.view(np.uint32))
    np.testing.assert_array_equal(h, eh)


def test_quantize_rows_special_cases():
    blocks = []
    blocks.append(np.zeros(32, np.float32))                                # amax 0 -> q 0
    blocks.append(np.arange(-127, 129, 8, dtype=np.float32)[:32].clip(-127, 127))  # amax 127 -> d 1
    t = np.zeros(32, np.float32); t[0] = 127; t[1] = 2.5; t[2] = 3.5; t[3] = -2.5; t[4] = 0.5
    blocks.append(t)                                                       # ties to even
    t = np.ones(32, np.float32); t[5] = np.nan
    blocks.append(t)                                                       # NaN ignored, q 0
    t = np.ones(32, np.float32); t[7] = np.inf; t[8] = -np.inf
    blocks.append(t)                                                       # amax inf
    blocks.append(np.full(32, np.nan, np.float32))                         # all NaN -> amax 0
    x = np.concatenate(blocks)
    v, s, h = oracle.quantize_rows(x)
    v = v.reshape(-1, 32)
    assert s[0] == 0 and not v[0].any() and list(h[0]) == [0, 0]
    assert s[1] == 1.0 and list(v[1]) == list(blocks[1].astype(np.int8))
    assert s[2] == 1.0 and list(v[2][:5]) == [127, 2, 4, -2, 0]
    assert s[3] == np.float32(1.0) / np.float32(127.0) and v[3][5] == 0 and v[3][0] == 127
    assert np.isinf(s[4]) and v[4][7] == 0 and v[4][8] == 0 and v[4][0] == 0
    assert s[5] == 0 and not v[5].any()
    assert list(h[1]) == [int(v[1][:16].astype(np.int32).sum()), int(v[1][16:].astype(np.int32).sum())]


def test_int8_rounded_is_q_times_d():
    x = activations(2, 64, 3)
    v, s, _ = oracle.quantize_rows(x)
    exp = (v.astype(np.float32).reshape(-1, 32) * s[:, None]).astype(np.float32).reshape(2, 64)
    np.testing.assert_array_equal(oracle.int8_rounded(x), exp)


def test_dot_halves_brute_force_including_minus_128():
    """`vector_dots_equal_scalar_dots` (src/native/tests.rs:212-232)."""
    rng = np.random.default_rng(5)
    for _ in range(1000):
        q = rng.integers(-128, 128, 32).astype(np.int8)
        a = rng.integers(-128, 128, 32).astype(np.int8)
        q[0] = -128
        got = oracle.dot_halves(q, a)
        p = q.astype(np.int64) * a.astype(np.int64)
        assert list(got) == [int(p[:16].sum()), int(p[16:].sum())]


# ---- dense matmul -----------------------------------------------------------

def test_dense_matmul_known_output():
    """Conformance known-answer check `matmul-known-output` (src/lib.rs:1882-1892)."""
    out = oracle.matmul_dense(np.array([[1, 2], [3, 4]], np.float32), np.array([[5, 6], [7, 8]], np.float32))
    assert out.tolist() == [[19, 22], [43, 50]]


class SplitMix:
    """splitmix64 values in [-10, 10] by 0.01 (src/tests.rs:14-33)."""

    def __init__(self, s):
        self.s = s

    def value(self):
        self.s = (self.s + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        z = self.s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        z ^= z >> 31
        return np.float32(z % 2001) / np.float32(100.0) - np.float32(10.0)

    def tensor(self, r, c):
        return np.array([[self.value() for _ in range(c)] for _ in range(r)], np.float32)


def test_dense_matmul_bit_identical_to_straightforward_form():
    """`matmul_is_bit_identical_to_the_straightforward_form` (src/tests.rs:83-113)."""
    rng = SplitMix(0x513D)
    for ta in (False, True):
        for tb in (False, True):
            for trial in range(40):
                m, k, n = 1 + trial % 7, 1 + (trial // 2) % 6, 1 + (trial // 3) % 5
                a = rng.tensor(k, m) if ta else rng.tensor(m, k)
                b = rng.tensor(n, k) if tb else rng.tensor(k, n)
                A = a.T if ta else a
                B = b.T if tb else b
                exp = np.zeros((m, n), np.float32)
                for r in range(m):
                    for c in range(n):
                        acc = np.float32(0)
                        for i in range(k):
                            acc = np.float32(acc + np.float32(A[r, i] * B[i, c]))
                        exp[r, c] = acc
                got = oracle.matmul_dense(a, b, ta, tb)
                np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_dense_matmul_propagates_non_finite():
    """0 * NaN and 0 * inf give NaN: no zero-skip (src/tests.rs:115-128)."""
    a = np.zeros((1, 2), np.float32)
    assert np.isnan(oracle.matmul_dense(a, np.array([[np.nan], [1]], np.float32))[0, 0])
    assert np.isnan(oracle.matmul_dense(a, np.array([[np.inf], [1]], np.float32))[0, 0])


# ---- packed column kernels ----------------------------------------------------

@pytest.mark.parametrize("fmt", [Q4_K, IQ4_XS])
def test_scalar_columns_match_reference_cpu(fmt):
    """`packed_matmuls_match_the_reference_cpu` (src/native/tests.rs:134-154)
    for the scalar kernel: int8 mode within the reference tolerance of
    matmul(int8_rounded(a), dequantize(W)); f32 mode bit-identical to the
    dense matmul (same products, same k order)."""
    k, n = 512, 37
    w = packed(fmt, n, k, 21)
    dense_t = oracle.dequantize(fmt, w, n, k)
    for m in (1, 3, 9):
        a = activations(m, k, m)
        exp8 = oracle.matmul_dense(oracle.int8_rounded(a), dense_t, False, True)
        assert_close_reference(oracle.columns_scalar(fmt, w, n, k, a, True), exp8, f"int8 m {m}")
        exp32 = oracle.matmul_dense(a, dense_t, False, True)
        got32 = oracle.columns_scalar(fmt, w, n, k, a, False)
        np.testing.assert_array_equal(got32.view(np.uint32), exp32.view(np.uint32))


@pytest.mark.parametrize("fmt", [Q4_K, IQ4_XS])
@pytest.mark.parametrize("threads", [1, 4])
def test_avx2_baseline_matches_reference_cpu(fmt, threads):
    """The timed CPU baseline agrees with the dense oracle on int8-rounded
    activations, reference tolerance, one and several threads."""
    k, n = 512, 37
    w = packed(fmt, n, k, 21)
    dense_t = oracle.dequantize(fmt, w, n, k)
    for m in (1, 3, 9):
        a = activations(m, k, m)
        exp = oracle.matmul_dense(oracle.int8_rounded(a), dense_t, False, True)
        assert_close_reference(oracle.baseline_packed_matmul(fmt, w, n, k, a, threads), exp, f"m {m}")


def test_q4k_reduces_to_integer_matmul():
    """d = 1, dmin = 0, scales 1: a Q4_K matmul of integer activations is an
    integer GEMM of the nibbles, exact in any summation order."""
    rng = np.random.default_rng(7)
    n, k = 9, 512
    q = rng.integers(0, 16, (n, k // 256, 8, 32))
    w = np.stack([np.stack([_q4k_block(1.0, 0.0, [1] * 8, [0] * 8, q[r, b]) for b in range(k // 256)])
                  for r in range(n)]).reshape(n, -1)
    x = rng.integers(-8, 9, (3, k)).astype(np.float32)
    exp = x.astype(np.int64) @ q.reshape(n, k).T.astype(np.int64)
    np.testing.assert_array_equal(oracle.columns_scalar(Q4_K, w, n, k, x, False), exp.astype(np.float32))
    # int8 mode is exact too once every block's amax is 127 (d = 1)
    x8 = x.copy()
    x8[:, ::32] = 127
    exp8 = x8.astype(np.int64) @ q.reshape(n, k).T.astype(np.int64)
    np.testing.assert_array_equal(oracle.columns_scalar(Q4_K, w, n, k, x8, True), exp8.astype(np.float32))
    np.testing.assert_array_equal(oracle.baseline_packed_matmul(Q4_K, w, n, k, x8, 2), exp8.astype(np.float32))


def test_int8_mode_power_of_two_scaling_is_exact():
    """y(2^e x) = 2^e y(x) bit-exactly in int8 mode: d scales by 2^e and the
    quantized values do not change."""
    k, n = 512, 16
    w = packed(Q4_K, n, k, 9)
    a = activations(2, k, 4)
    y = oracle.columns_scalar(Q4_K, w, n, k, a, True)
    for e in (-3, 5):
        y2 = oracle.columns_scalar(Q4_K, w, n, k, a * np.float32(2.0 ** e), True)
        np.testing.assert_array_equal(y2, (y * np.float32(2.0 ** e)).astype(np.float32))
