"""GPU parity of the plane formats (Q8_0, Q4_0, IQ4_NL, Q5_K, Q6_K) through
the C ABI against the oracle, with the bars of the Q4_K / IQ4_XS path:
dequantization bit-exact; matmul within max|d| <= 1e-3 ||row||_inf of the
mode-matched dense oracle, and the decode GEMV (m <= 8) also within the
reference's own 2e-5 max(1, max|e|) (src/native/tests.rs:91-103)."""

import numpy as np
import pytest

import magnetar_gpu as mg
import oracle
from helpers import (BLOCK_ELEMENTS, IQ4_NL, PLANE_FORMATS, Q4_0, Q6_K, Q8_0, activations, assert_close_reference,
                     assert_row_tolerance, packed)
from magnetar_gpu import workloads

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def expected(fmt, w, n, k, x, int8):
    dense_t = oracle.dequantize(fmt, w, n, k)
    a = oracle.int8_rounded(x) if int8 else x
    return oracle.matmul_dense(a, dense_t, False, True)


def shapes(fmt):
    base = [(3, 512), (37, 512), (65, 4096)]
    if BLOCK_ELEMENTS[fmt] == 32:
        base += [(5, 96), (9, 800)]  # rows ending inside a 256-value group
    return base


@pytest.mark.parametrize("fmt", PLANE_FORMATS)
def test_dequantize_bit_exact(ctx, fmt):
    for rows, cols in shapes(fmt):
        w = packed(fmt, rows, cols, 11 + rows)
        exp = oracle.dequantize(fmt, w, rows, cols)
        h = ctx.upload(fmt, rows, cols, w)
        try:
            got = ctx.dequantize(h)
            np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32), f"{rows}x{cols}")
            got_l = ctx.dequantize(h, logical=True)
            np.testing.assert_array_equal(got_l.view(np.uint32), np.ascontiguousarray(exp.T).view(np.uint32))
        finally:
            h.release()


@pytest.mark.parametrize("fmt", PLANE_FORMATS)
@pytest.mark.parametrize("int8", [True, False])
@pytest.mark.parametrize("m", [1, 3, 9])
def test_packed_matmul_matches_reference_cpu(ctx, fmt, int8, m):
    """`packed_matmuls_match_the_reference_cpu` (src/native/tests.rs:134-154):
    K = 512, N = 37, M in {1, 3, 9}, every format."""
    k, n = 512, 37
    w = packed(fmt, n, k, 21)
    a = activations(m, k, m)
    h = ctx.upload(fmt, n, k, w)
    try:
        got = ctx.matmul(h, a, int8=int8)
    finally:
        h.release()
    exp = expected(fmt, w, n, k, a, int8)
    assert_row_tolerance(got, exp, f"fmt {fmt} int8 {int8} m {m}")
    if m <= 8:
        assert_close_reference(got, exp, f"fmt {fmt} int8 {int8} m {m}")
    if int8 and m <= 8:
        # the mode-matched scalar column kernel itself
        assert_row_tolerance(got, oracle.columns_scalar(fmt, w, n, k, a, True), "vs columns_scalar")


@pytest.mark.parametrize("fmt", [Q8_0, IQ4_NL, Q4_0])
@pytest.mark.parametrize("m", [2, 9])
def test_odd_run_counts(ctx, fmt, m):
    """`odd_run_counts_match_the_reference_cpu` (src/native/tests.rs:158-177):
    K = 96 (three runs), N = 5; GEMV and GEMM."""
    k, n = 96, 5
    w = packed(fmt, n, k, 23)
    a = activations(m, k, 7)
    h = ctx.upload(fmt, n, k, w)
    try:
        for int8 in (True, False):
            got = ctx.matmul(h, a, int8=int8)
            exp = expected(fmt, w, n, k, a, int8)
            assert_row_tolerance(got, exp, f"int8 {int8}")
            if m <= 8:
                assert_close_reference(got, exp, f"int8 {int8}")
    finally:
        h.release()


@pytest.mark.parametrize("fmt", PLANE_FORMATS)
def test_gemv_every_row_count_and_k_split(ctx, fmt):
    """m = 1..8 on a 1000 x 2048 weight (K-splits by the LDS rule), then a
    14336-long row (m = 8 needs 3 K-splits to fit LDS)."""
    for n, k in ((1000, 2048), (96, 14336)):
        w = packed(fmt, n, k, 5 + n)
        h = ctx.upload(fmt, n, k, w)
        try:
            for m in (range(1, 9) if k == 2048 else (1, 8)):
                a = mg.gaussian(100 + m, 1.0, m * k).reshape(m, k)
                for int8 in (True, False):
                    got = ctx.matmul(h, a, int8=int8)
                    exp = expected(fmt, w, n, k, a, int8)
                    assert_row_tolerance(got, exp, f"{n}x{k} m {m} int8 {int8}")
                    assert_close_reference(got, exp, f"{n}x{k} m {m} int8 {int8}")
        finally:
            h.release()


@pytest.mark.parametrize("fmt", PLANE_FORMATS)
def test_fused_m1_equals_prequantized(ctx, fmt):
    """m = 1 with fused quantization equals the pre-quantized GEMV bit for
    bit, whichever staging the shape takes: wave-local where the rows are
    whole 256-value groups and each wave has at most two blocks of its K
    split (K = 1024, 4096), work-group staging where rows end inside a group
    (K = 800, the 32-value formats) or a split holds more blocks."""
    ks = (1024, 4096, 8192) + ((800,) if BLOCK_ELEMENTS[fmt] == 32 else ())
    for k in ks:
        n = 200
        w = packed(fmt, n, k, 33 + k)
        h = ctx.upload(fmt, n, k, w)
        try:
            a1 = mg.gaussian(9 + k, 1.0, k).reshape(1, k)
            x = torch.from_numpy(a1).cuda()
            xq = torch.empty(k, dtype=torch.int8, device="cuda")
            xs = torch.empty(k // 32, dtype=torch.float32, device="cuda")
            xh = torch.empty(k // 16, dtype=torch.int32, device="cuda")
            y = torch.empty((1, n), dtype=torch.float32, device="cuda")
            s = torch.cuda.current_stream().cuda_stream
            ctx.quantize_activations_dev(x.data_ptr(), 1, k, xq.data_ptr(), xs.data_ptr(), xh.data_ptr(), s)
            ctx.matmul_prequantized_dev(h, xq.data_ptr(), xs.data_ptr(), xh.data_ptr(), 1, k, y.data_ptr(),
                                        stream=s)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(y.cpu().numpy(), ctx.matmul(h, a1), f"k {k}")
        finally:
            h.release()


@pytest.mark.parametrize("fmt", PLANE_FORMATS)
def test_prequantized_and_f16_entry_points(ctx, fmt):
    """The prequantized GEMV agrees with mq_matmul on the same weight, and
    the GEMM (m = 40) meets the bar; the 32-value formats take K = 800,
    rows ending inside a 256-value group."""
    n, k = 300, (800 if BLOCK_ELEMENTS[fmt] == 32 else 1024)
    w = packed(fmt, n, k, 31)
    h = ctx.upload(fmt, n, k, w)
    try:
        a1 = mg.gaussian(7, 1.0, 2 * k).reshape(2, k)
        x = torch.from_numpy(a1).cuda()
        xq = torch.empty(2 * k, dtype=torch.int8, device="cuda")
        xs = torch.empty(2 * k // 32, dtype=torch.float32, device="cuda")
        xh = torch.empty(2 * k // 16, dtype=torch.int32, device="cuda")
        y = torch.empty((2, n), dtype=torch.float32, device="cuda")
        s = torch.cuda.current_stream().cuda_stream
        ctx.quantize_activations_dev(x.data_ptr(), 2, k, xq.data_ptr(), xs.data_ptr(), xh.data_ptr(), s)
        ctx.matmul_prequantized_dev(h, xq.data_ptr(), xs.data_ptr(), xh.data_ptr(), 2, k, y.data_ptr(), stream=s)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y.cpu().numpy(), ctx.matmul(h, a1))
        a2 = mg.gaussian(8, 1.0, 40 * k).reshape(40, k)
        exp = expected(fmt, w, n, k, a2, True)
        assert_row_tolerance(ctx.matmul(h, a2), exp, "gemm int8")
    finally:
        h.release()


@pytest.mark.parametrize("fmt", PLANE_FORMATS)
def test_prefill_gemm_llama_shape(ctx, fmt):
    """M = 512 prefill on a 4096 x 4096 weight, sampled rows of the output
    against the dense oracle (rows are independent)."""
    n, k, m = 4096, 4096, 512
    w = workloads.random_blocks(fmt, n, k, 9)
    a = mg.gaussian(900, 1.0, m * k).reshape(m, k)
    h = ctx.upload(fmt, n, k, w)
    try:
        got = ctx.matmul(h, a)
    finally:
        h.release()
    rows = np.array([0, 1, 255, 256, 511])
    exp = expected(fmt, w, n, k, a[rows], True)
    assert_row_tolerance(got[rows], exp, "sampled rows")


def test_q6k_decode_gemv_llama_ffn_up(ctx):
    """Q6_K decode GEMV x [1, 4096] . W [14336, 4096]^T (the output / FFN
    projection format of Q4_K_M checkpoints)."""
    n, k = 14336, 4096
    w = workloads.random_blocks(Q6_K, n, k, 14)
    a = mg.gaussian(14500, 1.0, k).reshape(1, k)
    h = ctx.upload(Q6_K, n, k, w)
    try:
        got = ctx.matmul(h, a)
    finally:
        h.release()
    exp = oracle.columns_scalar(Q6_K, w, n, k, a, True)
    assert_row_tolerance(got, exp)
    assert_close_reference(got, exp)
