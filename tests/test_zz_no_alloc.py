"""mq_matmul_noalloc_dev: the matmul without any device allocation (its
temporaries in one fixed device array per GPU), called through the C ABI
and checked against mq_matmul_dev on the same inputs, bit for bit, on two
calls in a row with the second smaller, over every path that needs
temporaries: the fused decode GEMV, the split-K GEMV with its counters and
partials, the pre-quantized rows' workspace, the plane formats, the split-K
MFMA prefill and the input-major product. Also the size limit."""

import ctypes

import numpy as np
import pytest

import magnetar_gpu as mg
import oracle
from helpers import packed

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def noalloc(ctx, weight, x, m, k, y, int8=True):
    flags = mg.INT8_ACTIVATIONS if int8 else 0
    return mg.gpu_lib().mq_matmul_noalloc_dev(ctx.ptr, weight.handle, ctypes.c_void_p(x.data_ptr()), m, k, flags,
                                              ctypes.c_void_p(y.data_ptr()), None)


def both(ctx, weight, n, k, m, seed, int8=True):
    """(noalloc output, mq_matmul_dev output) for one seeded x[m, k]."""
    x = torch.from_numpy(mg.gaussian(seed, 1.0, m * k).reshape(m, k)).cuda()
    y_ref = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    ctx.matmul_dev(weight, x.data_ptr(), m, k, y_ref.data_ptr(), int8=int8)
    rc = noalloc(ctx, weight, x, m, k, y, int8)
    assert rc == mg.OK, mg.gpu_lib().mq_last_error(ctx.ptr)
    torch.cuda.synchronize()
    return y.cpu().numpy(), y_ref.cpu().numpy(), x.cpu().numpy()


# (format, stored rows n, k, first m, second m): the first call's
# temporaries are larger than the second's
CASES = [
    (mg.Q4_K, 14336, 4096, 3, 1),   # fused decode GEMV, one super-block per wave
    (mg.Q4_K, 1000, 2048, 8, 2),    # split-K GEMV (counters, partials), pre-quantized rows
    (mg.IQ4_XS, 4096, 14336, 4, 1),  # the 16-row form
    (mg.Q6_K, 4096, 4096, 6, 1),    # plane format, split-K
    (mg.Q4_K, 4096, 4096, 128, 40),  # MFMA prefill (split-K partials at 128 rows)
    (mg.Q8_0, 300, 1024, 24, 17),   # plane-format prefill
]


@pytest.mark.parametrize("fmt,n,k,m1,m2", CASES)
def test_noalloc_matches_the_allocating_entry_point(ctx, fmt, n, k, m1, m2):
    if fmt in (mg.Q4_K, mg.IQ4_XS):
        w = mg.quantize(fmt, mg.gaussian(n + k + fmt, 0.02, n * k).reshape(n, k))
    else:
        w = packed(fmt, n, k, n + k)
    h = ctx.upload(fmt, n, k, w)
    try:
        for m, seed in ((m1, 11), (m2, 12)):
            got, ref, x = both(ctx, h, n, k, m, seed)
            assert not np.isnan(got).any()
            np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32), err_msg=f"m={m}")
        if m2 == 1 and fmt == mg.Q4_K:
            # and the oracle's bar on the decode row (the reference's int8 path)
            exp = oracle.columns_scalar(fmt, w, n, k, x, True)
            tol = 1e-3 * np.max(np.abs(exp), axis=1, keepdims=True)
            assert np.all(np.abs(got - exp) <= tol)
    finally:
        h.release()


def test_noalloc_f32_activations_and_input_major(ctx):
    """f32 activations and the input-major (axpy) product of an untransposed
    weight, whose K-split partials live in the scratch."""
    k, n = 512, 256
    w = mg.quantize(mg.Q4_K, mg.gaussian(5, 0.02, k * n).reshape(k, n))
    h = ctx.upload(mg.Q4_K, k, n, w, transposed=False)
    try:
        for m, seed in ((5, 21), (2, 22)):
            got, ref, _ = both(ctx, h, n, k, m, seed, int8=False)
            np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    finally:
        h.release()
    h = ctx.upload(mg.Q4_K, n, k, mg.quantize(mg.Q4_K, mg.gaussian(6, 0.02, n * k).reshape(n, k)))
    try:
        for m, seed in ((7, 23), (1, 24)):
            got, ref, _ = both(ctx, h, n, k, m, seed, int8=False)
            np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    finally:
        h.release()


def test_noalloc_rejects_temporaries_above_the_limit(ctx):
    """A prefill whose f16 activations alone exceed the 32 MiB array is
    refused with the sizes in the message; nothing is launched, and the next
    call still works."""
    n, k, m = 256, 4096, 4096  # 32 MiB of f16 activations, above 32 MiB - 64 KiB
    h = ctx.upload(mg.Q4_K, n, k, mg.quantize(mg.Q4_K, mg.gaussian(7, 0.02, n * k).reshape(n, k)))
    try:
        x = torch.zeros((m, k), dtype=torch.float32, device="cuda")
        y = torch.zeros((m, n), dtype=torch.float32, device="cuda")
        rc = noalloc(ctx, h, x, m, k, y)
        assert rc == mg.ERR_SHAPE
        msg = mg.gpu_lib().mq_last_error(ctx.ptr).decode()
        assert "temporaries" in msg and "no-allocation" in msg
        got, ref, _ = both(ctx, h, n, k, 40, 31)
        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    finally:
        h.release()
