"""Pins of the oracle's IQ2 / IQ3 grid-format decode (oracle/oracle.c
`or_decode_run`, restating src/native/quant.rs:207-277).

The grid tables themselves are external (magnetar-provider-api `iq_grids`,
not vendored): the decode is pinned with stand-in tables of the real
tables' shapes and magnitude alphabets (`synthetic_iq_grids`), so the table
VALUES stay "parity unpinned" while every index, sign and scale path is
checked. The checks are the public ggml dequantizers
(`dequantize_row_iq2_xxs` ... `dequantize_row_iq3_s`), which walk a block
by 32-value groups with their own pointer arithmetic (IQ3_S two runs at a
time, its grid index high bits shifted from qh the other way), written in
float64 numpy; hand-built blocks give exact known answers; the sign table
is pinned by its parity property."""

import numpy as np
import pytest

import oracle
from helpers import (BLOCK_BYTES, GRID_FORMATS, IQ2_S, IQ2_XS, IQ2_XXS, IQ3_S, IQ3_XXS, activations,
                     assert_close_reference, packed, synthetic_iq_grids)

GRIDS = synthetic_iq_grids(1)


@pytest.fixture(autouse=True)
def _grids():
    oracle.set_iq_grids(GRIDS)


def _f16(blocks, at):
    return blocks[:, at:at + 2].copy().view(np.float16).astype(np.float64)[:, 0]


def _ksigns(i):
    """ggml's ksigns_iq2xs[i]: i with bit 7 set when popcount(i) is odd."""
    i = np.asarray(i, np.int64) & 127
    par = np.zeros_like(i)
    for b in range(7):
        par ^= (i >> b) & 1
    return i | (par << 7)


def _grid_bytes(table, idx, width):
    """Magnitudes (the entry's bytes as i8) of table entries idx: [..., width]."""
    e = np.asarray(table)[np.asarray(idx)]
    shifts = np.arange(width, dtype=e.dtype) * e.dtype.type(8)
    b = (e[..., None] >> shifts) & e.dtype.type(0xFF)
    return b.astype(np.uint8).view(np.int8).astype(np.int64)


def _signed(mag, signs):
    """mag [..., 8], signs [...] sign bytes: bit j negates value j."""
    bits = (np.asarray(signs, np.int64)[..., None] >> np.arange(8)) & 1
    return np.where(bits == 1, -mag, mag)


def ggml_dequantize(fmt, w, rows, cols):
    raw = w.reshape(-1, BLOCK_BYTES[fmt])
    b = raw.astype(np.int64)
    nblk = b.shape[0]
    d = _f16(raw, 0)
    y = np.zeros((nblk, 256))
    t2xxs, t2xs, t2s, t3xxs, t3s = GRIDS
    for ib32 in range(8):
        at = 32 * ib32
        if fmt == IQ2_XXS:
            q2 = raw[:, 2 + 8 * ib32:2 + 8 * ib32 + 8].copy().view(np.uint32).astype(np.int64)
            aux0, aux1 = q2[:, 0], q2[:, 1]
            db = d * (0.5 + (aux1 >> 28)) * 0.25
            for l in range(4):
                mag = _grid_bytes(t2xxs, (aux0 >> (8 * l)) & 0xFF, 8)
                y[:, at + 8 * l:at + 8 * l + 8] = db[:, None] * _signed(mag, _ksigns(aux1 >> (7 * l)))
        elif fmt == IQ2_XS:
            qs = raw[:, 2:66].copy().view(np.uint16).astype(np.int64)
            sc = b[:, 66 + ib32]
            db = [d * (0.5 + (sc & 0xF)) * 0.25, d * (0.5 + (sc >> 4)) * 0.25]
            for l in range(4):
                code = qs[:, 4 * ib32 + l]
                mag = _grid_bytes(t2xs, code & 511, 8)
                y[:, at + 8 * l:at + 8 * l + 8] = db[l // 2][:, None] * _signed(mag, _ksigns(code >> 9))
        elif fmt == IQ2_S:
            qs, signs, qh, scales = b[:, 2:34], b[:, 34:66], b[:, 66:74], b[:, 74:82]
            db = [d * (0.5 + (scales[:, ib32] & 0xF)) * 0.25, d * (0.5 + (scales[:, ib32] >> 4)) * 0.25]
            for l in range(4):
                idx = qs[:, 4 * ib32 + l] | ((qh[:, ib32] << (8 - 2 * l)) & 0x300)
                mag = _grid_bytes(t2s, idx, 8)
                y[:, at + 8 * l:at + 8 * l + 8] = db[l // 2][:, None] * _signed(mag, signs[:, 4 * ib32 + l])
        elif fmt == IQ3_XXS:
            qs = b[:, 2 + 8 * ib32:2 + 8 * ib32 + 8]
            aux = raw[:, 66 + 4 * ib32:70 + 4 * ib32].copy().view(np.uint32).astype(np.int64)[:, 0]
            db = d * (0.5 + (aux >> 28)) * 0.5
            for l in range(4):
                mag = np.concatenate([_grid_bytes(t3xxs, qs[:, 2 * l], 4), _grid_bytes(t3xxs, qs[:, 2 * l + 1], 4)],
                                     axis=-1)
                y[:, at + 8 * l:at + 8 * l + 8] = db[:, None] * _signed(mag, _ksigns(aux >> (7 * l)))
    if fmt == IQ3_S:
        # two runs per step, as ggml: qh byte per run, scales nibble per run
        qs, qh, signs, scales = b[:, 2:66], b[:, 66:74], b[:, 74:106], b[:, 106:110]
        for ib32 in range(0, 8, 2):
            db1 = d * (1 + 2 * (scales[:, ib32 // 2] & 0xF))
            db2 = d * (1 + 2 * (scales[:, ib32 // 2] >> 4))
            for r, db in ((ib32, db1), (ib32 + 1, db2)):
                q, h, sg = qs[:, 8 * r:8 * r + 8], qh[:, r], signs[:, 4 * r:4 * r + 4]
                for l in range(4):
                    g1 = _grid_bytes(t3s, q[:, 2 * l] | ((h << (8 - 2 * l)) & 256), 4)
                    g2 = _grid_bytes(t3s, q[:, 2 * l + 1] | ((h << (7 - 2 * l)) & 256), 4)
                    mag = np.concatenate([g1, g2], axis=-1)
                    y[:, 32 * r + 8 * l:32 * r + 8 * l + 8] = db[:, None] * _signed(mag, sg[:, l])
    return y.reshape(rows, cols).astype(np.float32)


@pytest.mark.parametrize("fmt", GRID_FORMATS)
def test_dequant_random_blocks_match_ggml_dequantizer(fmt):
    rows, cols = 3, 512
    w = packed(fmt, rows, cols, 11)
    np.testing.assert_array_equal(oracle.dequantize(fmt, w, rows, cols), ggml_dequantize(fmt, w, rows, cols))


def test_sign_table_is_the_index_with_its_parity():
    for i in range(128):
        s = oracle.iq_signs(i)
        assert s & 0x7F == i
        assert bin(s).count("1") % 2 == 0
    # only the low 7 bits of the argument count
    assert oracle.iq_signs(0x1FF) == oracle.iq_signs(0x7F) == 0xFF


def _blank(fmt, d_bits=0x3C00):
    blk = np.zeros(BLOCK_BYTES[fmt], np.uint8)
    blk[0], blk[1] = d_bits & 0xFF, d_bits >> 8
    return blk


def _mags(table, i, width):
    v = int(table[i])
    return [(v >> (8 * j)) & 0xFF for j in range(width)]


def test_iq2_xxs_known_answer():
    """Run 1: grid indices 5, 6, 7, 8; sign index 1 for group 0 (values 0
    and 7 negated), 0 elsewhere; scale nibble 3: (0.5 + 3) / 4 = 0.875."""
    blk = _blank(IQ2_XXS)
    blk[2 + 8:6 + 8] = [5, 6, 7, 8]
    aux = 1 | (3 << 28)
    blk[6 + 8:10 + 8] = np.frombuffer(np.uint32(aux).tobytes(), np.uint8)
    q, scale, mn = oracle.decode_run(IQ2_XXS, blk, 1)
    exp = sum((_mags(GRIDS[0], i, 8) for i in (5, 6, 7, 8)), [])
    exp[0], exp[7] = -exp[0], -exp[7]
    np.testing.assert_array_equal(q, exp)
    np.testing.assert_array_equal(scale, [0.875, 0.875])
    np.testing.assert_array_equal(mn, [0, 0])


def test_iq2_s_known_answer_uses_the_high_index_bits_and_raw_signs():
    blk = _blank(IQ2_S, 0x4000)  # d = 2
    run = 2
    blk[2 + 4 * run:6 + 4 * run] = [1, 2, 3, 4]
    blk[66 + run] = 0b11100100  # high bits 0, 1, 2, 3 for groups 0..3
    blk[34 + 4 * run:38 + 4 * run] = [0xFF, 0, 0x01, 0x80]
    blk[74 + run] = 0x52  # scales 2 (values 0..15), 5 (16..31)
    q, scale, _ = oracle.decode_run(IQ2_S, blk, run)
    exp = []
    for l, (i, s) in enumerate(zip([1, 2 + 256, 3 + 512, 4 + 768], [0xFF, 0, 0x01, 0x80])):
        m = _mags(GRIDS[2], i, 8)
        exp += [-v if (s >> j) & 1 else v for j, v in enumerate(m)]
    np.testing.assert_array_equal(q, exp)
    np.testing.assert_array_equal(scale, [2 * 2.5 * 0.25, 2 * 5.5 * 0.25])


def test_iq3_s_known_answer_scale_is_odd_multiple():
    blk = _blank(IQ3_S)
    run = 3
    blk[2 + 8 * run:10 + 8 * run] = np.arange(10, 18)
    blk[66 + run] = 0b10000001  # index bit 8 for entries 0 and 7
    blk[74 + 4 * run:78 + 4 * run] = [0x0F, 0, 0, 0xF0]
    blk[106 + run // 2] = 0x70  # run 3 is the high nibble: 7 -> 1 + 14 = 15
    q, scale, _ = oracle.decode_run(IQ3_S, blk, run)
    idx = [10 + 256, 11, 12, 13, 14, 15, 16, 17 + 256]
    exp = []
    for l in range(4):
        m = _mags(GRIDS[4], idx[2 * l], 4) + _mags(GRIDS[4], idx[2 * l + 1], 4)
        s = [0x0F, 0, 0, 0xF0][l]
        exp += [-v if (s >> j) & 1 else v for j, v in enumerate(m)]
    np.testing.assert_array_equal(q, exp)
    np.testing.assert_array_equal(scale, [15.0, 15.0])


@pytest.mark.parametrize("fmt", GRID_FORMATS)
def test_decode_run_is_the_dequant_run(fmt):
    w = packed(fmt, 1, 256, 5)
    full = oracle.dequantize(fmt, w, 1, 256)[0]
    for run in range(8):
        q, scale, mn = oracle.decode_run(fmt, w[0], run)
        p = np.arange(32) // 16
        exp = (scale[p] * q.astype(np.float32) - mn[p]).astype(np.float32)
        np.testing.assert_array_equal(full[32 * run:32 * run + 32], exp)


@pytest.mark.parametrize("fmt", GRID_FORMATS)
def test_scalar_columns_match_reference_cpu(fmt):
    """`packed_matmuls_match_the_reference_cpu` (src/native/tests.rs:134-154)
    over the grid formats: int8 mode within the reference tolerance, f32
    mode bit-identical to the dense matmul."""
    k, n = 512, 21
    w = packed(fmt, n, k, 21)
    dense_t = oracle.dequantize(fmt, w, n, k)
    for m in (1, 3):
        a = activations(m, k, m)
        exp8 = oracle.matmul_dense(oracle.int8_rounded(a), dense_t, False, True)
        assert_close_reference(oracle.columns_scalar(fmt, w, n, k, a, True), exp8, f"int8 m {m}")
        exp32 = oracle.matmul_dense(a, dense_t, False, True)
        got32 = oracle.columns_scalar(fmt, w, n, k, a, False)
        np.testing.assert_array_equal(got32.view(np.uint32), exp32.view(np.uint32))


def test_changing_a_table_entry_changes_only_its_users():
    """The decode reads the set tables (not built-in values): replacing one
    IQ2_XXS entry changes exactly the values whose group index is that entry."""
    w = packed(IQ2_XXS, 2, 512, 3)
    before = oracle.dequantize(IQ2_XXS, w, 2, 512)
    t = [a.copy() for a in GRIDS]
    raw = w.reshape(-1, 66)
    target = int(raw[0, 2])  # group 0 of run 0 of the first block
    t[0][target] ^= np.uint64(0x0101010101010101)  # 8 -> 9, 25 -> 24, 43 -> 42
    oracle.set_iq_grids(t)
    after = oracle.dequantize(IQ2_XXS, w, 2, 512)
    groups = np.concatenate([raw[:, 2 + 8 * r:6 + 8 * r] for r in range(8)], axis=1).reshape(-1)
    uses = np.repeat(groups == target, 8)
    np.testing.assert_array_equal(before.reshape(-1)[~uses], after.reshape(-1)[~uses])
    assert np.all(before.reshape(-1)[uses] != after.reshape(-1)[uses])
