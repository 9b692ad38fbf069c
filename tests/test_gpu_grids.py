"""GPU parity of the IQ2 / IQ3 grid formats (IQ2_XXS, IQ2_XS, IQ2_S,
IQ3_XXS, IQ3_S) through the C ABI against the oracle.

The grid tables are the caller's (mq_set_iq_grids); both sides get the
same stand-in tables (`synthetic_iq_grids`: the real tables' shapes and
magnitude alphabets), so the table values are parity unpinned while every
index, sign and scale path is compared. Bars as for the other formats:
dequantization bit-exact, matmuls within max|d| <= 1e-3 ||row||_inf of the
mode-matched dense oracle, and the decode GEMV within the reference's
2e-5 max(1, max|e|) of the reference's own int8 column loop."""

import numpy as np
import pytest

import magnetar_gpu as mg
import oracle
from helpers import (GRID_FORMATS, IQ2_XXS, IQ3_S, activations, assert_close_reference, assert_row_tolerance,
                     packed, synthetic_iq_grids)

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

GRIDS = synthetic_iq_grids(1)


@pytest.fixture(scope="module")
def gctx(ctx):
    ctx.set_iq_grids(GRIDS)
    oracle.set_iq_grids(GRIDS)
    return ctx


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def dense(fmt, w, n, k, x, int8):
    dense_t = oracle.dequantize(fmt, w, n, k)
    a = oracle.int8_rounded(x) if int8 else x
    return oracle.matmul_dense(a, dense_t, False, True)


@pytest.mark.parametrize("fmt", GRID_FORMATS)
@pytest.mark.parametrize("rows,cols", [(3, 512), (37, 1024), (1, 256)])
def test_dequantize_bit_exact(gctx, fmt, rows, cols):
    w = packed(fmt, rows, cols, 11 + rows + fmt)
    exp = oracle.dequantize(fmt, w, rows, cols)
    h = gctx.upload(fmt, rows, cols, w)
    try:
        np.testing.assert_array_equal(gctx.dequantize(h).view(np.uint32), exp.view(np.uint32))
        got_l = gctx.dequantize(h, logical=True)
        np.testing.assert_array_equal(got_l.view(np.uint32), np.ascontiguousarray(exp.T).view(np.uint32))
    finally:
        h.release()


@pytest.mark.parametrize("fmt", GRID_FORMATS)
@pytest.mark.parametrize("int8", [True, False])
def test_gemv_every_m(gctx, fmt, int8):
    """m = 1..8 on a ragged row count; the int8 mode also against the
    reference's own int8 column loop (the oracle's restatement) at its
    2e-5 tolerance."""
    n, k = 300, 1024
    w = packed(fmt, n, k, 31 + fmt)
    h = gctx.upload(fmt, n, k, w)
    try:
        for m in range(1, 9):
            x = activations(m, k, 40 + m)
            got = gctx.matmul(h, x, int8=int8)
            assert_row_tolerance(got, dense(fmt, w, n, k, x, int8), f"m {m}")
            if int8:
                assert_close_reference(got, oracle.columns_scalar(fmt, w, n, k, x, True), f"m {m} column loop")
    finally:
        h.release()


@pytest.mark.parametrize("fmt", [IQ2_XXS, IQ3_S])
def test_prefill_huge_block_scales(gctx, fmt):
    """Block scales near 65504 (dequantized values far beyond f16's range):
    the grid GEMM's f16 operands stay in range through the weight's
    power-of-two factor; both activation modes meet the dense oracle's bar."""
    m, n, k = 96, 300, 1024
    w = packed(fmt, n, k, 51 + fmt).copy()
    blocks = w.reshape(n, k // 256, -1)  # a view: each block's f16 d is bytes 0-1
    bits = blocks[:, :, 0].astype(np.uint16) | (blocks[:, :, 1].astype(np.uint16) << 8)
    bits = (bits & np.uint16(0x83FF)) | np.uint16(29 << 10)
    blocks[:, :, 0] = (bits & 0xFF).astype(np.uint8)
    blocks[:, :, 1] = (bits >> 8).astype(np.uint8)
    x = activations(m, k, 52)
    h = gctx.upload(fmt, n, k, w)
    try:
        for int8 in (True, False):
            got = gctx.matmul(h, x, int8=int8)
            assert np.isfinite(got).all()
            assert_row_tolerance(got, dense(fmt, w, n, k, x, int8), f"int8 {int8}")
    finally:
        h.release()


@pytest.mark.parametrize("fmt", GRID_FORMATS)
def test_prefill_rows_and_residual(gctx, fmt):
    """M = 40 (past 16 rows: the MFMA prefill GEMM) and the residual
    epilogue with one broadcast row and with M rows."""
    m, n, k = 40, 136, 768
    w = packed(fmt, n, k, 51)
    x = activations(m, k, 52)
    h = gctx.upload(fmt, n, k, w)
    try:
        base = dense(fmt, w, n, k, x, True)
        assert_row_tolerance(gctx.matmul(h, x), base, "prefill")
        xd = dev(x)
        for r_rows in (1, m):
            r = activations(r_rows, n, 53 + r_rows)
            rd = dev(r)
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")
            gctx.matmul_add_dev(h, xd.data_ptr(), m, k, rd.data_ptr(), r_rows, y.data_ptr())
            torch.cuda.synchronize()
            assert_row_tolerance(y.cpu().numpy(), (base + r).astype(np.float32), f"residual {r_rows}")
    finally:
        h.release()


@pytest.mark.parametrize("fmt", GRID_FORMATS)
@pytest.mark.parametrize("m,k", [(3, 512), (1, 4096), (8, 4096), (3, 14336), (4, 14336)])
def test_prequantized_entry_point(gctx, fmt, m, k):
    """The pre-quantized entry point equals the f32 entry point (quantized
    by the quantization kernel) bit for bit, with the quantized rows
    staged in LDS (they fit with the grid table) and read from memory (the
    4 x 14336 case does not fit)."""
    n = 64
    w = packed(fmt, n, k, 61)
    x = activations(m, k, 62)
    values, scales, sums = oracle.quantize_rows(x)
    h = gctx.upload(fmt, n, k, w)
    try:
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        vd, sd, hd = dev(values), dev(scales), dev(sums)
        gctx.matmul_prequantized_dev(h, vd.data_ptr(), sd.data_ptr(), hd.data_ptr(), m, k, y.data_ptr())
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y.cpu().numpy(), gctx.matmul(h, x))
    finally:
        h.release()


@pytest.mark.parametrize("fmt", GRID_FORMATS)
def test_input_major_product_and_embedding(gctx, fmt):
    """An untransposed grid-format table: read untransposed it is the
    input-major (axpy) product; its rows are embedding rows."""
    k, n = 48, 512  # stored rows = the k inputs, each n values
    w = packed(fmt, k, n, 71)
    table = oracle.dequantize(fmt, w, k, n)
    x = activations(3, k, 72)
    x[:, ::5] = 0.0
    h = gctx.upload(fmt, k, n, w, transposed=False)
    try:
        got = gctx.matmul(h, x)
        assert_row_tolerance(got, oracle.matmul_dense(x, table), "axpy")
        ids = np.array([0, 47, 5, 5], np.uint32)
        np.testing.assert_array_equal(gctx.embedding(h, ids), table[ids])
    finally:
        h.release()


@pytest.mark.parametrize("fmt", GRID_FORMATS)
def test_gemv_long_rows_staged_and_unstaged(gctx, fmt):
    """K = 14336 (the FFN down rows): the int8 activations are staged in LDS
    with the grid table while m K (1 + 4 / 32) bytes and the table fit 64 KiB
    (m <= 3), and read from memory beyond (m >= 4); both against the
    reference's int8 column loop."""
    n, k = 40, 14336
    w = packed(fmt, n, k, 37 + fmt)
    h = gctx.upload(fmt, n, k, w)
    try:
        for m in (1, 3, 4, 8):
            x = activations(m, k, 140 + m)
            got = gctx.matmul(h, x)
            assert_row_tolerance(got, dense(fmt, w, n, k, x, True), f"m {m}")
            assert_close_reference(got, oracle.columns_scalar(fmt, w, n, k, x, True), f"m {m} column loop")
    finally:
        h.release()


def test_full_size_gemv_sampled_columns(gctx):
    """IQ2_XXS at the Llama FFN up shape, m = 1: 8 sampled output columns
    against the reference's column loop."""
    fmt, n, k = IQ2_XXS, 14336, 4096
    rng = np.random.default_rng(81)
    w = rng.integers(0, 256, size=(n * k // 256, 66), dtype=np.uint8)
    d_bits = ((3 + rng.integers(0, 5, size=w.shape[0])) << 10) | rng.integers(0, 1024, size=w.shape[0])
    w[:, 0], w[:, 1] = d_bits & 0xFF, d_bits >> 8  # small positive f16 scales, as packed()
    w = w.reshape(n, -1)
    x = activations(1, k, 82)
    h = gctx.upload(fmt, n, k, w)
    try:
        got = gctx.matmul(h, x)
    finally:
        h.release()
    cols = np.random.default_rng(3).choice(n, 256, replace=False)
    for c in cols[:8]:
        exp = oracle.columns_scalar(fmt, w, n, k, x, True, first=int(c), count=1)
        assert_close_reference(got[:, c:c + 1], exp, f"column {c}")
    assert np.isfinite(got).all()


def _context_with(env):
    """A Context whose launch choices are forced through the environment
    (read once, at creation)."""
    import os
    old = {k: os.environ.get(k) for k in env}
    os.environ.update({k: str(v) for k, v in env.items()})
    try:
        return mg.Context(0)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


@pytest.mark.parametrize("fmt", GRID_FORMATS)
@pytest.mark.parametrize("variant", [0, 2, 3])
def test_prefill_gemm_tiles_and_ragged_edges(gctx, fmt, variant):
    """The MFMA prefill (register-B form decoding the raw blocks per lane)
    with 128 x 128 (variant 3) and 128 x 256 (variant 2) tiles: M and N
    ragged against both tile sizes, both activation modes, and the f16
    operand entry point against the same dense product."""
    c = _context_with({"MQ_GEMM_VARIANT": variant})
    try:
        for m, n, k in ((130, 300, 1024), (17, 257, 512), (64, 40, 2304)):
            w = packed(fmt, n, k, 61 + n)
            x = activations(m, k, 62 + m)
            h = c.upload(fmt, n, k, w)
            try:
                for int8 in (True, False):
                    assert_row_tolerance(c.matmul(h, x, int8=int8), dense(fmt, w, n, k, x, int8),
                                         f"m {m} n {n} k {k} int8 {int8}")
                xd = dev(x)
                a16 = torch.empty(m * k + 2 * m, dtype=torch.float16, device="cuda")  # values, row factors
                c.prepare_activations_f16_dev(xd.data_ptr(), m, k, a16.data_ptr(), int8=False)
                y = torch.empty((m, n), dtype=torch.float32, device="cuda")
                c.matmul_f16_dev(h, a16.data_ptr(), m, k, y.data_ptr())
                torch.cuda.synchronize()
                exp = dense(fmt, w, n, k, x.astype(np.float16).astype(np.float32), False)
                assert_row_tolerance(y.cpu().numpy(), exp, f"f16 entry m {m} n {n} k {k}")
            finally:
                h.release()
    finally:
        c.close()


def test_prefill_falls_back_for_wide_grid_bytes(gctx):
    """Grid tables holding a magnitude byte of 128 or more: the MFMA
    prefill (unsigned magnitudes) is not used; the prefill runs as 8-row
    GEMVs (i8 magnitudes, as the reference) and the f16 entry point
    declines. The stand-in tables are restored afterwards."""
    wide = [t.copy() for t in GRIDS]
    wide[0][5] |= np.uint64(0x90)  # one IQ2_XXS entry's byte 0 -> 0x90 | b
    gctx.set_iq_grids(tuple(wide))
    oracle.set_iq_grids(tuple(wide))
    try:
        m, n, k = 40, 72, 512
        w = packed(IQ2_XXS, n, k, 71)
        x = activations(m, k, 72)
        h = gctx.upload(IQ2_XXS, n, k, w)
        try:
            assert_row_tolerance(gctx.matmul(h, x), dense(IQ2_XXS, w, n, k, x, True), "prefill, wide bytes")
            a16 = torch.zeros(m * k + 2 * m, dtype=torch.float16, device="cuda")
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")
            with pytest.raises(mg.Declined):
                gctx.matmul_f16_dev(h, a16.data_ptr(), m, k, y.data_ptr())
        finally:
            h.release()
    finally:
        gctx.set_iq_grids(GRIDS)
        oracle.set_iq_grids(GRIDS)


def test_declines(gctx):
    w = packed(IQ2_XXS, 8, 256, 91)
    h = gctx.upload(IQ2_XXS, 8, 256, w)
    try:
        y = torch.empty((4, 8), dtype=torch.float32, device="cuda")
        x = torch.zeros((1, 256), dtype=torch.float32, device="cuda")
        with pytest.raises(mg.Declined):
            gctx.decode_matmul_dev(h, x.data_ptr(), 256, y.data_ptr())
    finally:
        h.release()
