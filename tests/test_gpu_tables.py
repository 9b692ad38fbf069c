"""GPU parity of the untransposed packed weights through the C ABI: the
input-major (axpy) product, the tied output head and the embedding lookup
(src/native/mod.rs:154-194, 217-227, 389-449; src/native/quant.rs:1652-1711),
every format, against the oracle's dequantization: lookups bit-exact,
products within the reference's 2e-5 max(1, max|e|)."""

import numpy as np
import pytest

import magnetar_gpu as mg
import oracle
from helpers import (IQ4_XS, PLANE_FORMATS, Q4_K, Q8_0, activations, assert_close_reference, assert_row_tolerance,
                     packed)

pytestmark = pytest.mark.gpu

ALL = PLANE_FORMATS + [Q4_K, IQ4_XS]


@pytest.mark.parametrize("fmt", ALL)
@pytest.mark.parametrize("m", [1, 4, 9])
def test_input_major_product(ctx, fmt, m):
    """`input_major_weights_multiply_packed` (src/native/tests.rs:193-209):
    untransposed [64, 256], f32 activations whatever the int8 flag."""
    w = packed(fmt, 64, 256, 61)
    dense = oracle.dequantize(fmt, w, 64, 256)
    h = ctx.upload(fmt, 64, 256, w, transposed=False)
    try:
        a = activations(m, 64, 62)
        got = ctx.matmul(h, a)
        exp = oracle.matmul_dense(a, dense)
        assert_close_reference(got, exp, f"m {m}")
        np.testing.assert_array_equal(ctx.matmul(h, a, int8=False), got)
        # a transposed weight read with transpose_b is input-major too
        ht = ctx.upload(fmt, 64, 256, w, transposed=True)
        try:
            assert_close_reference(ctx.matmul(ht, a, transpose_b=True), exp, "transposed, transpose_b")
        finally:
            ht.release()
    finally:
        h.release()


@pytest.mark.parametrize("fmt", [Q4_K, Q8_0])
def test_input_major_product_at_size_with_residual(ctx, fmt):
    """K = 1024 stored rows of N = 4096, m = 3, with a residual addend and
    exact zeros in the activations (skipped, as the reference skips them)."""
    k, n = 1024, 4096
    w = packed(fmt, k, n, 5)
    a = activations(3, k, 9)
    a[:, ::7] = 0.0
    res = activations(3, n, 10)
    h = ctx.upload(fmt, k, n, w, transposed=False)
    try:
        x = torch_dev(a)
        r = torch_dev(res)
        y = torch_dev(np.zeros((3, n), np.float32))
        ctx.matmul_add_dev(h, x.data_ptr(), 3, k, r.data_ptr(), 3, y.data_ptr())
        got = y.cpu().numpy()
    finally:
        h.release()
    exp = oracle.matmul_dense(a, oracle.dequantize(fmt, w, k, n)) + res
    assert_row_tolerance(got, exp)
    assert_close_reference(got, exp)


def torch_dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


@pytest.mark.parametrize("fmt", ALL)
def test_embedding_lookup_and_tied_head(ctx, fmt):
    """`packed_tables_serve_lookups_and_tied_heads` (src/native/tests.rs:178-191):
    an untransposed table [50, dim] gathers rows bit for bit and, read with
    transpose_b, is the output head."""
    dim = 64 if fmt in (Q8_0, mg.Q4_0, mg.IQ4_NL) else 256
    table = packed(fmt, 50, dim, 31)
    dense = oracle.dequantize(fmt, table, 50, dim)
    h = ctx.upload(fmt, 50, dim, table, transposed=False)
    try:
        ids = [7, 0, 49, 7, 12]
        np.testing.assert_array_equal(ctx.embedding(h, ids), dense[ids])
        np.testing.assert_array_equal(ctx.embedding(h, ids, scale=3.0), dense[ids] * np.float32(3.0))
        a = activations(2, dim, 3)
        exp = oracle.matmul_dense(oracle.int8_rounded(a), dense, False, True)
        assert_close_reference(ctx.matmul(h, a, transpose_b=True), exp, "tied head")
    finally:
        h.release()


@pytest.mark.parametrize("fmt", [Q4_K, mg.Q6_K, IQ4_XS])
def test_embedding_of_a_transposed_table(ctx, fmt):
    """A table stored [dim][vocab] (transposed): each token's value in every
    stored row (`quant::element`, src/native/quant.rs:1690-1698)."""
    dim, vocab = 40, 512
    t = packed(fmt, dim, vocab, 77)
    dense = oracle.dequantize(fmt, t, dim, vocab)
    h = ctx.upload(fmt, dim, vocab, t, transposed=True)
    try:
        ids = [0, 31, 32, 511, 300]
        np.testing.assert_array_equal(ctx.embedding(h, ids), dense[:, ids].T)
    finally:
        h.release()


def test_embedding_rejects_bad_token_ids(ctx):
    """The reference's id check and text (src/native/mod.rs:399-404)."""
    table = packed(Q8_0, 50, 64, 31)
    h = ctx.upload(Q8_0, 50, 64, table, transposed=False)
    try:
        for bad, text in ((50.0, "50"), (-1.0, "-1"), (7.5, "7.5"), (float("nan"), "NaN")):
            with pytest.raises(mg.GpuError) as e:
                ctx.embedding(h, [3.0, bad])
            assert e.value.code == mg.ERR_SHAPE
            assert e.value.reason == f"token id {text} is not below the vocabulary size 50"
        assert ctx.embedding(h, []).shape == (0, 64)
    finally:
        h.release()
