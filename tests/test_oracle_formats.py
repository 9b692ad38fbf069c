"""Pins of the oracle's Q8_0, Q4_0, IQ4_NL, Q2_K, Q3_K, Q5_K and Q6_K decode
(oracle/oracle.c `or_decode_run`, restating src/native/quant.rs:102-195).

The reference's own decode is run-based; the checks here are the public
GGUF dequantizers (ggml `dequantize_row_*`), which walk the blocks in a
different order (Q5_K by 64-value chunks with a moving high-bit mask, Q6_K
by 128-value halves producing four outputs per byte position), written in
vectorized float64 numpy. A transposed plane, a wrong shift or a wrong
scale index fails them. Hand-built blocks give exact known answers."""

import json
import os

import numpy as np
import pytest

import oracle
from helpers import (BLOCK_BYTES, IQ4_NL, PLANE_FORMATS, Q2_K, Q3_K, Q4_0, Q5_K, Q6_K, Q8_0, activations,
                     assert_close_reference, packed)


def _iq4nl():
    with open(os.path.join(os.path.dirname(__file__), "golden", "gguf_iq4nl_codebook.json")) as f:
        return json.load(f)["kvalues_iq4nl"]


def _f16(blocks, at):
    return blocks[:, at:at + 2].copy().view(np.float16).astype(np.float64)[:, 0]


def ggml_dequantize(fmt, w, rows, cols):
    """GGUF dequantizers, float64, rounded once to f32 at the end (every
    product below is exact in float64 and is a single f32 rounding in the
    reference's f32 arithmetic)."""
    blocks = w.reshape(-1, BLOCK_BYTES[fmt]).astype(np.int64)
    nblk = blocks.shape[0]
    if fmt == Q8_0:
        d = _f16(w.reshape(-1, 34), 0)
        q = blocks[:, 2:34].astype(np.uint8).view(np.int8).astype(np.int64)
        y = d[:, None] * q
    elif fmt in (Q4_0, IQ4_NL):
        d = _f16(w.reshape(-1, 18), 0)
        qs = blocks[:, 2:18]
        lo, hi = qs & 0xF, qs >> 4
        if fmt == Q4_0:
            vals = np.concatenate([lo - 8, hi - 8], axis=1)
        else:
            T = np.array(_iq4nl(), np.int64)
            vals = np.concatenate([T[lo], T[hi]], axis=1)
        y = d[:, None] * vals
    elif fmt == Q5_K:
        raw = w.reshape(-1, 176)
        d, dmin = _f16(raw, 0), _f16(raw, 2)
        s = blocks[:, 4:16]
        qh, ql = blocks[:, 16:48], blocks[:, 48:176]
        y = np.zeros((nblk, 256))
        for c in range(4):  # ggml: j = 64 c, is = 2 c, u1 = 1 << 2c, u2 = 2 << 2c
            out = []
            for t in (0, 1):
                isx = 2 * c + t
                if isx < 4:
                    sc, m = s[:, isx] & 63, s[:, isx + 4] & 63
                else:
                    sc = (s[:, isx + 4] & 0xF) | ((s[:, isx - 4] >> 6) << 4)
                    m = (s[:, isx + 4] >> 4) | ((s[:, isx] >> 6) << 4)
                u = 1 << (2 * c + t)
                nib = (ql[:, 32 * c:32 * c + 32] >> (4 * t)) & 0xF
                q = nib + np.where(qh & u, 16, 0)
                out.append((d * sc)[:, None] * q - (dmin * m)[:, None])
            y[:, 64 * c:64 * c + 32], y[:, 64 * c + 32:64 * c + 64] = out
    elif fmt == Q6_K:
        raw = w.reshape(-1, 210)
        d = _f16(raw, 208)
        sc = blocks[:, 192:208].astype(np.uint8).view(np.int8).astype(np.int64)
        y = np.zeros((nblk, 256))
        for n in range(2):  # 128-value halves
            ql = blocks[:, 64 * n:64 * n + 64]
            qh = blocks[:, 128 + 32 * n:128 + 32 * n + 32]
            s = sc[:, 8 * n:8 * n + 8]
            q1 = ((ql[:, :32] & 0xF) | (((qh >> 0) & 3) << 4)) - 32
            q2 = ((ql[:, 32:] & 0xF) | (((qh >> 2) & 3) << 4)) - 32
            q3 = ((ql[:, :32] >> 4) | (((qh >> 4) & 3) << 4)) - 32
            q4 = ((ql[:, 32:] >> 4) | (((qh >> 6) & 3) << 4)) - 32
            is_ = np.arange(32) // 16
            for i, q in enumerate((q1, q2, q3, q4)):
                y[:, 128 * n + 32 * i:128 * n + 32 * i + 32] = (d[:, None] * s[:, is_ + 2 * i]) * q
    elif fmt == Q2_K:
        raw = w.reshape(-1, 84)
        d, dmin = _f16(raw, 80), _f16(raw, 82)
        sc, qs = blocks[:, 0:16], blocks[:, 16:80]
        y = np.zeros((nblk, 256))
        isx = 0
        for n in range(2):  # ggml: per 128 values, shift 0, 2, 4, 6 over the same 32 bytes
            q = qs[:, 32 * n:32 * n + 32]
            for j in range(4):
                for half in range(2):
                    s_ = sc[:, isx]
                    isx += 1
                    vals = (q[:, 16 * half:16 * half + 16] >> (2 * j)) & 3
                    at = 128 * n + 32 * j + 16 * half
                    y[:, at:at + 16] = (d * (s_ & 0xF))[:, None] * vals - (dmin * (s_ >> 4))[:, None]
    elif fmt == Q3_K:
        raw = w.reshape(-1, 110)
        d = _f16(raw, 108)
        hm, qs, b = blocks[:, 0:32], blocks[:, 32:96], blocks[:, 96:108]
        # scale i: low nibble of byte i % 8 (nibble i // 8), high 2 bits from
        # byte 8 + i % 4 at bit 2 (i // 4)
        scales = np.stack([((b[:, i % 8] >> (4 * (i // 8))) & 0xF) | (((b[:, 8 + i % 4] >> (2 * (i // 4))) & 3) << 4)
                           for i in range(16)], axis=1) - 32
        y = np.zeros((nblk, 256))
        isx, m = 0, 1
        for n in range(2):
            q = qs[:, 32 * n:32 * n + 32]
            for j in range(4):
                for half in range(2):
                    sl = slice(16 * half, 16 * half + 16)
                    vals = ((q[:, sl] >> (2 * j)) & 3) - np.where(hm[:, sl] & m, 0, 4)
                    at = 128 * n + 32 * j + 16 * half
                    y[:, at:at + 16] = (d * scales[:, isx])[:, None] * vals
                    isx += 1
                m <<= 1
    else:
        raise ValueError(fmt)
    return y.reshape(rows, cols).astype(np.float32)


@pytest.mark.parametrize("fmt", PLANE_FORMATS)
def test_dequant_random_blocks_match_ggml_dequantizer(fmt):
    """`runs_decode_like_the_runtime` (src/native/tests.rs:106-130) with the
    runtime's dequantizer replaced by ggml's: reference-style random
    blocks (src/native/tests.rs:45-67), bit for bit."""
    rows, cols = 3, 512
    w = packed(fmt, rows, cols, 11)
    np.testing.assert_array_equal(oracle.dequantize(fmt, w, rows, cols), ggml_dequantize(fmt, w, rows, cols))


def _block(fmt, d_bits=0x3C00):
    blk = np.zeros(BLOCK_BYTES[fmt], np.uint8)
    at = 208 if fmt == Q6_K else 0
    blk[at], blk[at + 1] = d_bits & 0xFF, d_bits >> 8
    return blk


def test_q8_0_known_answer():
    blk = _block(Q8_0, 0x4000)  # d = 2
    q = np.arange(-16, 16, dtype=np.int8)
    blk[2:] = q.view(np.uint8)
    np.testing.assert_array_equal(oracle.dequantize(Q8_0, blk, 1, 32)[0], 2.0 * q.astype(np.float32))


def test_q4_0_known_answer_is_q_minus_8():
    blk = _block(Q4_0, 0x3800)  # d = 0.5
    blk[2:] = (np.arange(16) | (15 - np.arange(16)) << 4).astype(np.uint8)
    got = oracle.dequantize(Q4_0, blk, 1, 32)[0]
    np.testing.assert_array_equal(got[:16], 0.5 * (np.arange(16) - 8))
    np.testing.assert_array_equal(got[16:], 0.5 * (15 - np.arange(16) - 8))


def test_iq4_nl_known_answer_is_the_codebook():
    blk = _block(IQ4_NL, 0x3400)  # d = 0.25
    blk[2:] = (np.arange(16) | (np.arange(16) << 4)).astype(np.uint8)
    T = np.array(_iq4nl(), np.float32)
    got = oracle.dequantize(IQ4_NL, blk, 1, 32)[0]
    np.testing.assert_array_equal(got[:16], 0.25 * T)
    np.testing.assert_array_equal(got[16:], 0.25 * T)


def test_q5_k_high_bit_plane_and_scales():
    """d = 1, dmin = 0, every 6-bit scale 1: value = nibble + 16 * bit
    `run` of the high-bit byte at the value's position."""
    blk = _block(Q5_K)
    blk[4:8] = 1   # runs 0..3 scale 1
    blk[12:16] = 1  # runs 4..7 scale low nibble 1 (high bits from bytes 0..3 >> 6 = 0)
    blk[16:48] = (1 << (np.arange(32) % 8)).astype(np.uint8)  # value l of run l % 8 gets +16
    blk[48:176] = 0x53  # low nibble 3 (even runs), high nibble 5 (odd runs)
    got = oracle.dequantize(Q5_K, blk, 1, 256)[0].reshape(8, 32)
    for run in range(8):
        base = 3 if run % 2 == 0 else 5
        exp = base + 16 * (np.arange(32) % 8 == run)
        np.testing.assert_array_equal(got[run], exp.astype(np.float32))


def test_q6_k_sign_offset_and_per_half_scales():
    """d = 1, scales i8 = half index + 1 (negative for odd halves): value =
    s_half * ((low | high << 4) - 32)."""
    blk = _block(Q6_K)
    scales = np.array([(i + 1) * (-1 if i % 2 else 1) for i in range(16)], np.int8)
    blk[192:208] = scales.view(np.uint8)
    blk[0:128] = 0xA5   # low nibble 5, high nibble 10
    blk[128:192] = 0xE4  # 2-bit fields 0, 1, 2, 3 from the bottom
    got = oracle.dequantize(Q6_K, blk, 1, 256)[0]
    for v in range(256):
        h, rem = divmod(v, 128)
        g, l = divmod(rem, 32)
        nib = 5 if g < 2 else 10
        q = (nib | (g << 4)) - 32
        s = int(scales[8 * h + 2 * g + l // 16])
        assert got[v] == np.float32(s * q), v


@pytest.mark.parametrize("fmt", PLANE_FORMATS)
def test_decode_run_is_the_dequant_run(fmt):
    """`element` / `dequantize_row` (quant.rs:1690-1711) are scale[p] q -
    min[p] of the decoded run."""
    be = 32 if fmt in (Q8_0, Q4_0, IQ4_NL) else 256
    w = packed(fmt, 1, be, 5)
    full = oracle.dequantize(fmt, w, 1, be)[0]
    for run in range(be // 32):
        q, scale, mn = oracle.decode_run(fmt, w[0], run)
        p = np.arange(32) // 16
        exp = (scale[p] * q.astype(np.float32) - mn[p]).astype(np.float32)
        np.testing.assert_array_equal(full[32 * run:32 * run + 32], exp)


@pytest.mark.parametrize("fmt", PLANE_FORMATS)
def test_scalar_columns_match_reference_cpu(fmt):
    """`packed_matmuls_match_the_reference_cpu` (src/native/tests.rs:134-154):
    int8 mode within the reference tolerance of matmul(int8_rounded(a), W);
    f32 mode bit-identical to the dense matmul."""
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


@pytest.mark.parametrize("fmt", [Q8_0, IQ4_NL, Q4_0])
def test_odd_run_counts(fmt):
    """`odd_run_counts_match_the_reference_cpu` (src/native/tests.rs:158-177):
    k = 96, three 32-value blocks per row."""
    k, n = 96, 5
    w = packed(fmt, n, k, 23)
    dense_t = oracle.dequantize(fmt, w, n, k)
    a = activations(2, k, 7)
    exp = oracle.matmul_dense(oracle.int8_rounded(a), dense_t, False, True)
    assert_close_reference(oracle.columns_scalar(fmt, w, n, k, a, True), exp, "odd runs")


def test_k_must_be_whole_blocks():
    w = packed(Q5_K, 1, 256, 3)
    with pytest.raises(ValueError):
        oracle.dequantize(Q5_K, w, 1, 96)


def test_q3_k_scale_unpacking_inverts_the_gguf_packing():
    """Sixteen 6-bit scales packed as the GGUF Q3_K encoder packs them (low
    nibbles into bytes 0..7, low half first; the top 2 bits into bytes
    8..11, two bits per group of four) unpack to themselves."""
    r = np.random.default_rng(12)
    for _ in range(50):
        L = r.integers(0, 64, 16)
        packed12 = np.zeros(12, np.int64)
        for j in range(16):
            lj = int(L[j])
            if j < 8:
                packed12[j] = lj & 0xF
            else:
                packed12[j - 8] |= (lj & 0xF) << 4
            packed12[8 + j % 4] |= (lj >> 4) << (2 * (j // 4))
        np.testing.assert_array_equal(oracle.q3_k_scales(packed12.astype(np.uint8)), L)


def test_q2_k_known_answer():
    """d = 1, dmin = 0.5; run (h, j) half p reads scale byte 8h + 2j + p
    (low nibble scale, high nibble min) and 2-bit field j of the half's
    32 quant bytes."""
    blk = np.zeros(84, np.uint8)
    blk[80:82] = [0x00, 0x3C]  # d = 1
    blk[82:84] = [0x00, 0x38]  # dmin = 0.5
    blk[0:16] = [(i % 15 + 1) | ((i % 4) << 4) for i in range(16)]
    blk[16:80] = 0b11100100  # fields j = 0..3 hold 0, 1, 2, 3
    got = oracle.dequantize(Q2_K, blk, 1, 256)[0]
    for v in range(256):
        h, rem = divmod(v, 128)
        j, l = divmod(rem, 32)
        b = int(blk[8 * h + 2 * j + l // 16])
        assert got[v] == np.float32((b & 0xF) * j - 0.5 * (b >> 4)), v


def test_q3_k_high_bit_mask_and_offset():
    """All scales 33 (scale 1 after -32), d = 1: value = 2-bit field j of the
    quant byte, minus 4 unless bit 4h + j of the mask byte is set."""
    blk = np.zeros(110, np.uint8)
    blk[108:110] = [0x00, 0x3C]
    L = np.full(16, 33)
    twelve = np.zeros(12, np.int64)
    for j in range(16):
        twelve[j % 8] |= (L[j] & 0xF) << (4 * (j // 8))
        twelve[8 + j % 4] |= (L[j] >> 4) << (2 * (j // 4))
    blk[96:108] = twelve.astype(np.uint8)
    blk[32:96] = 0b10110001  # fields 1, 0, 3, 2
    blk[0:32] = (1 << (np.arange(32) % 8)).astype(np.uint8)  # value l keeps its top bit in run l % 8
    got = oracle.dequantize(Q3_K, blk, 1, 256)[0]
    fields = [1, 0, 3, 2]
    for v in range(256):
        h, rem = divmod(v, 128)
        j, l = divmod(rem, 32)
        run = 4 * h + j
        exp = fields[j] - (0 if l % 8 == run else 4)
        assert got[v] == np.float32(exp), v
