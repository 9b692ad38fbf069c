"""GPU parity: the gfx950 path through the C ABI against the oracle.

Bars: dequantization and int8 activation quantization bit-exact; matmul
outputs within max|d| <= 1e-3 ||row||_inf of the mode-matched dense
oracle (int8 mode: matmul(int8_rounded(x), dequantize(W)); f32 mode:
matmul(x, dequantize(W))), f32 accumulate. The decode GEMV (m <= 8) also
meets the reference's own 2e-5 max(1, max|e|) tolerance."""

import numpy as np
import pytest

import magnetar_gpu as mg
import oracle
from helpers import (IQ4_XS, Q2_K, Q4_K, Q6_K, Q8_0, activations, assert_close_reference, assert_row_tolerance, packed,
                     row_tolerance_violation)
from magnetar_gpu import workloads

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def expected(fmt, w, n, k, x, int8, rows=None):
    """Dense oracle on the (optionally row-sampled) activations."""
    dense_t = oracle.dequantize(fmt, w, n, k)
    xs = x if rows is None else x[rows]
    a = oracle.int8_rounded(xs) if int8 else xs
    return oracle.matmul_dense(a, dense_t, False, True)


# ---- dequantization ------------------------------------------------------------

@pytest.mark.parametrize("fmt", [Q4_K, IQ4_XS])
@pytest.mark.parametrize("rows,cols,gen", [(3, 512, "packed"), (37, 512, "packed"), (8, 4096, "gauss"),
                                           (1, 256, "packed"), (65, 1024, "gauss")])
def test_dequantize_bit_exact(ctx, fmt, rows, cols, gen):
    if gen == "packed":
        w = packed(fmt, rows, cols, 11 + rows)
    else:
        w = mg.quantize(fmt, mg.gaussian(rows, 0.02, rows * cols).reshape(rows, cols))
    exp = oracle.dequantize(fmt, w, rows, cols)
    h = ctx.upload(fmt, rows, cols, w)
    try:
        got = ctx.dequantize(h)
        np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))
        got_l = ctx.dequantize(h, logical=True)
        assert got_l.shape == (cols, rows)
        np.testing.assert_array_equal(got_l.view(np.uint32), np.ascontiguousarray(exp.T).view(np.uint32))
    finally:
        h.release()


def test_dequantize_full_size_bit_exact(ctx):
    name = "q4k_14336x4096_s1"
    fmt, n, k, _, _ = workloads.WEIGHTS[name]
    w = workloads.weight_bytes(name)
    h = ctx.upload(fmt, n, k, w)
    try:
        got = ctx.dequantize(h)
        exp = oracle.dequantize(fmt, w, n, k)
        np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))
    finally:
        h.release()


# ---- activation quantization -----------------------------------------------------

def _special_blocks():
    b = []
    b.append(np.zeros(32, np.float32))
    t = np.zeros(32, np.float32); t[0] = 127; t[1] = 2.5; t[2] = 3.5; t[3] = -2.5; t[4] = 0.5; t[5] = -0.5
    b.append(t)
    t = np.ones(32, np.float32); t[5] = np.nan; b.append(t)
    t = np.ones(32, np.float32); t[7] = np.inf; t[8] = -np.inf; b.append(t)
    b.append(np.full(32, np.nan, np.float32))
    b.append(np.full(32, -0.0, np.float32))
    b.append(np.full(32, 1e-42, np.float32))
    t = np.linspace(-3e38, 3e38, 32).astype(np.float32); b.append(t)
    return np.concatenate(b)


@pytest.mark.parametrize("m,k", [(1, 256), (3, 512), (9, 4096), (1, 14336), (512, 4096)])
def test_quantize_activations_bit_exact(ctx, m, k):
    rng = np.random.default_rng(m * 7 + k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    if m * k >= 256:
        s = _special_blocks()
        x.reshape(-1)[:s.size] = s
    ev, es, eh = oracle.quantize_rows(x)
    xd = dev(x)
    v = torch.empty(m * k, dtype=torch.int8, device="cuda")
    sc = torch.empty(m * k // 32, dtype=torch.float32, device="cuda")
    sm = torch.empty(m * k // 32 * 2, dtype=torch.int32, device="cuda")
    ctx.quantize_activations_dev(xd.data_ptr(), m, k, v.data_ptr(), sc.data_ptr(), sm.data_ptr(),
                                 torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(v.cpu().numpy(), ev)
    np.testing.assert_array_equal(sc.cpu().numpy().view(np.uint32), es.view(np.uint32))
    np.testing.assert_array_equal(sm.cpu().numpy().reshape(-1, 2), eh)


# ---- matmul at the reference's own test shapes --------------------------------

@pytest.mark.parametrize("fmt", [Q4_K, IQ4_XS])
@pytest.mark.parametrize("int8", [True, False])
@pytest.mark.parametrize("m", [1, 3, 9])
def test_packed_matmul_matches_reference_cpu(ctx, fmt, int8, m):
    """`packed_matmuls_match_the_reference_cpu` (src/native/tests.rs:134-154):
    K = 512, N = 37 (not a multiple of the 8-row group), M in {1, 3, 9}."""
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


@pytest.mark.parametrize("fmt", [Q4_K, IQ4_XS])
@pytest.mark.parametrize("int8", [True, False])
def test_gemv_every_row_count(ctx, fmt, int8):
    n, k = 1000, 2048
    w = mg.quantize(fmt, mg.gaussian(77, 0.02, n * k).reshape(n, k))
    h = ctx.upload(fmt, n, k, w)
    try:
        for m in range(1, 9):
            a = mg.gaussian(100 + m, 1.0, m * k).reshape(m, k)
            got = ctx.matmul(h, a, int8=int8)
            exp = expected(fmt, w, n, k, a, int8)
            assert_row_tolerance(got, exp, f"m {m}")
            assert_close_reference(got, exp, f"m {m}")
    finally:
        h.release()


# ---- the benchmark workloads -----------------------------------------------------

@pytest.mark.parametrize("int8", [True, False])
def test_decode_gemv_q4k_llama_ffn_up(ctx, int8):
    """Q4_K decode GEMV, x [M, 4096], W [14336, 4096], M in {1, 2, 4, 8}, seed 1."""
    name = "q4k_14336x4096_s1"
    fmt, n, k, seed, _ = workloads.WEIGHTS[name]
    w = workloads.weight_bytes(name)
    h = ctx.upload(fmt, n, k, w)
    try:
        for m in (1, 2, 4, 8):
            a = workloads.activations(seed, m, k)
            got = ctx.matmul(h, a, int8=int8)
            exp = expected(fmt, w, n, k, a, int8)
            assert_row_tolerance(got, exp, f"m {m}")
    finally:
        h.release()


def test_q4k_matvec_cpu_config(ctx):
    """Q4_K matvec x [1, 4096] . W [4096, 4096]^T, seed 0."""
    name = "q4k_4096x4096_s0"
    fmt, n, k, seed, _ = workloads.WEIGHTS[name]
    w = workloads.weight_bytes(name)
    a = workloads.activations(seed, 1, k)
    h = ctx.upload(fmt, n, k, w)
    try:
        got = ctx.matmul(h, a)
    finally:
        h.release()
    exp = expected(fmt, w, n, k, a, True)
    assert_row_tolerance(got, exp)
    assert_close_reference(got, exp)


@pytest.mark.parametrize("int8", [True, False])
def test_iq4xs_gemv_llama_ffn_down(ctx, int8):
    """IQ4_XS GEMV x [1, 14336] . W [4096, 14336]^T, seed 3."""
    name = "iq4xs_4096x14336_s3"
    fmt, n, k, seed, _ = workloads.WEIGHTS[name]
    w = workloads.weight_bytes(name)
    a = workloads.activations(seed, 1, k)
    h = ctx.upload(fmt, n, k, w)
    try:
        got = ctx.matmul(h, a, int8=int8)
    finally:
        h.release()
    exp = expected(fmt, w, n, k, a, int8)
    assert_row_tolerance(got, exp)
    assert_close_reference(got, exp)


@pytest.mark.parametrize("name", ["q4k_4096x4096_s2", "q4k_14336x4096_s2"])
@pytest.mark.parametrize("m", [128, 512, 2048])
@pytest.mark.parametrize("int8", [True, False])
def test_prefill_gemm(ctx, name, m, int8):
    """Q4_K prefill GEMM x [M, 4096], M in {128, 512, 2048}, seed 2; the dense
    oracle runs on 24 sampled rows (it is row-independent, so each sampled
    row is exactly the full product's row)."""
    fmt, n, k, seed, _ = workloads.WEIGHTS[name]
    w = workloads.weight_bytes(name)
    a = workloads.activations(seed, m, k)
    h = ctx.upload(fmt, n, k, w)
    try:
        got = ctx.matmul(h, a, int8=int8)
    finally:
        h.release()
    rows = np.unique(np.concatenate([[0, m - 1], np.random.default_rng(m).integers(0, m, 22)]))
    exp = expected(fmt, w, n, k, a, int8, rows)
    assert_row_tolerance(got[rows], exp, f"{name} m {m}")
    assert np.isfinite(got).all()


@pytest.fixture(scope="module")
def ks_ctx():
    """A context whose GEMMs all take the Q4_K K-split form (variant 5),
    whatever the shape."""
    import os

    old = os.environ.get("MQ_GEMM_VARIANT")
    os.environ["MQ_GEMM_VARIANT"] = "5"
    try:
        c = mg.Context(0)
    finally:
        if old is None:
            del os.environ["MQ_GEMM_VARIANT"]
        else:
            os.environ["MQ_GEMM_VARIANT"] = old
    yield c
    c.close()


@pytest.mark.parametrize("m,n,k", [(200, 300, 768), (17, 520, 256), (129, 257, 1280), (512, 1024, 4096),
                                   (40, 8, 512)])
@pytest.mark.parametrize("int8", [True, False])
def test_gemm_k_split_form_ragged(ks_ctx, m, n, k, int8):
    """The K-split GEMM on ragged M and N (partial 128 x 256 tiles, a row
    group of zero padding) and on odd super-block counts (K = 768, 1280: one
    K half ends with a block of zeros; K = 256: the second half has none)."""
    w = packed(Q4_K, n, k, 5 + m + n)
    a = activations(m, k, 70 + m)
    h = ks_ctx.upload(Q4_K, n, k, w)
    try:
        got = ks_ctx.matmul(h, a, int8=int8)
    finally:
        h.release()
    assert_row_tolerance(got, expected(Q4_K, w, n, k, a, int8), f"{m}x{n}x{k}")


def test_gemm_k_split_form_residual(ks_ctx):
    """matmul-residual through the K-split epilogue: y = x W^T + r with r of
    one broadcast row and of M rows."""
    m, n, k = 160, 384, 1024
    w = packed(Q4_K, n, k, 9)
    a = activations(m, k, 71)
    h = ks_ctx.upload(Q4_K, n, k, w)
    try:
        base = expected(Q4_K, w, n, k, a, True)
        x = dev(a)
        for r_rows in (1, m):
            r = activations(r_rows, n, 72 + r_rows)
            rd = dev(r)
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")
            ks_ctx.matmul_add_dev(h, x.data_ptr(), m, k, rd.data_ptr(), r_rows, y.data_ptr())
            torch.cuda.synchronize()
            assert_row_tolerance(y.cpu().numpy(), (base + r).astype(np.float32), f"residual rows {r_rows}")
    finally:
        h.release()


@pytest.mark.parametrize("fmt", [Q4_K, IQ4_XS, Q6_K])
def test_gemm_split_k_register_b_form(ctx, fmt):
    """Under-filled register-B GEMMs split K over work-groups and sum the
    partials in split order (splits 4, 2 and 8 here, the second capped by
    the row's two super-blocks): within the bar of the dense oracle,
    deterministic, and the residual added after the sum (equal to the
    product plus r bit for bit)."""
    for m, n, k in ((160, 384, 1024), (40, 300, 512), (130, 1024, 4096)):
        w = packed(fmt, n, k, 90 + m)
        a = activations(m, k, 91 + m)
        h = ctx.upload(fmt, n, k, w)
        try:
            got = ctx.matmul(h, a)
            assert_row_tolerance(got, expected(fmt, w, n, k, a, True), f"m {m} n {n} k {k}")
            np.testing.assert_array_equal(got.view(np.uint32), ctx.matmul(h, a).view(np.uint32))
            x = dev(a)
            for r_rows in (1, m):
                r = activations(r_rows, n, 92 + r_rows)
                y = torch.empty((m, n), dtype=torch.float32, device="cuda")
                ctx.matmul_add_dev(h, x.data_ptr(), m, k, dev(r).data_ptr(), r_rows, y.data_ptr())
                torch.cuda.synchronize()
                np.testing.assert_array_equal(y.cpu().numpy(), (got + r).astype(np.float32),
                                              err_msg=f"residual rows {r_rows}, m {m} n {n}")
        finally:
            h.release()


# ---- properties at full size -------------------------------------------------------

@pytest.mark.parametrize("m", [1, 8, 512])
def test_int8_power_of_two_scaling_is_exact(ctx, m):
    """y(2^e x) = 2^e y(x) bit for bit in int8 mode: the activation scales
    change by 2^e, the quantized values do not."""
    name = "q4k_14336x4096_s1"
    fmt, n, k, seed, _ = workloads.WEIGHTS[name]
    h = ctx.upload(fmt, n, k, workloads.weight_bytes(name))
    try:
        a = workloads.activations(seed, m, k)
        y = ctx.matmul(h, a)
        for e in (-2, 3):
            y2 = ctx.matmul(h, a * np.float32(2.0 ** e))
            np.testing.assert_array_equal(y2, (y * np.float32(2.0 ** e)).astype(np.float32))
    finally:
        h.release()


@pytest.mark.parametrize("int8", [True, False])
def test_prefill_power_of_two_scaling_is_exact(ctx, int8):
    """M = 512 through the f16 MFMA GEMM: y(2^e x) = 2^e y(x) bit for bit in
    both activation modes, for e far outside f16's range (2^-40 x holds only
    f16 subnormals and zeros unscaled, 2^30 x only infinities): each row's
    power-of-two factor absorbs e, so the f16 operand is the same."""
    name = "q4k_4096x4096_s2"
    fmt, n, k, seed, _ = workloads.WEIGHTS[name]
    h = ctx.upload(fmt, n, k, workloads.weight_bytes(name))
    try:
        a = workloads.activations(seed, 512, k)
        y = ctx.matmul(h, a, int8=int8)
        for e in (-40, 30):
            y2 = ctx.matmul(h, (a * np.float32(2.0 ** e)).astype(np.float32), int8=int8)
            np.testing.assert_array_equal(y2, (y.astype(np.float64) * 2.0 ** e).astype(np.float32),
                                          err_msg=f"e {e}")
    finally:
        h.release()


@pytest.mark.parametrize("scale", [1e-6, 1e5])
@pytest.mark.parametrize("int8", [True, False])
def test_prefill_activations_far_from_unit_scale(ctx, scale, int8):
    """Activations scaled by 1e-6 (below f16's normal range) and 1e5 (above
    its 65504) at M = 512: the GEMM rows stay finite and within the bar of
    the dense oracle, like the decode GEMV's (M = 1 here)."""
    name = "q4k_4096x4096_s2"
    fmt, n, k, seed, _ = workloads.WEIGHTS[name]
    w = workloads.weight_bytes(name)
    a = (workloads.activations(seed, 512, k) * np.float32(scale)).astype(np.float32)
    h = ctx.upload(fmt, n, k, w)
    try:
        got = ctx.matmul(h, a, int8=int8)
        one = ctx.matmul(h, a[:1], int8=int8)
    finally:
        h.release()
    rows = np.unique(np.concatenate([[0, 511], np.random.default_rng(7).integers(0, 512, 14)]))
    exp = expected(fmt, w, n, k, a, int8, rows)
    assert np.isfinite(got).all()
    assert_row_tolerance(got[rows], exp, f"scale {scale}")
    assert_row_tolerance(one, exp[:1], f"scale {scale}, m 1")


# block-scale exponent fields and mantissa masks: the smallest f16
# subnormals (at most 15 x 2^-24), and scales near 65504
_TINY_SCALES = ((0,), 0x00F)
_HUGE_SCALES = ((28, 29, 30), 0x3FF)


@pytest.mark.parametrize("int8", [True, False])
def test_prefill_rows_longer_than_the_register_hold(ctx, int8):
    """K = 16640 (65 super-blocks): the f16 operand's rows are read twice
    instead of held in registers; both activation modes against the oracle."""
    m, n, k = 24, 72, 16640
    w = packed(Q4_K, n, k, 86)
    a = activations(m, k, 87)
    h = ctx.upload(Q4_K, n, k, w)
    try:
        assert_row_tolerance(ctx.matmul(h, a, int8=int8), expected(Q4_K, w, n, k, a, int8), f"int8 {int8}")
    finally:
        h.release()


def _rescaled_block_scales(fmt, w, scales, seed):
    """w with every f16 block scale (d, dmin) given an exponent field drawn
    from scales[0] and its mantissa masked by scales[1]."""
    from helpers import BLOCK_BYTES, half_offsets

    exponents, mantissa = scales
    out = w.copy().reshape(-1, BLOCK_BYTES[fmt])
    rng = np.random.default_rng(seed)
    for at in half_offsets(fmt):
        bits = out[:, at].astype(np.uint16) | (out[:, at + 1].astype(np.uint16) << 8)
        ex = rng.choice(np.asarray(exponents, np.uint16), size=bits.shape[0])
        bits = (bits & np.uint16(0x8000 | mantissa)) | (ex << np.uint16(10))
        out[:, at] = (bits & 0xFF).astype(np.uint8)
        out[:, at + 1] = (bits >> 8).astype(np.uint8)
    return out.reshape(w.shape)


@pytest.mark.parametrize("fmt", [Q4_K, IQ4_XS, Q6_K, Q8_0, Q2_K])
@pytest.mark.parametrize("scales", [_TINY_SCALES, _HUGE_SCALES], ids=["tiny", "huge"])
def test_prefill_weights_far_from_unit_scale(ctx, fmt, scales):
    """Weights whose block scales are the smallest f16 subnormals
    (dequantized values at most about 1e-4) or near 65504 (values up to
    3e8, far beyond f16): the weight's power-of-two factor keeps the GEMM's
    f16 operands in range, so the register-B and split-K register-B forms
    meet the bar of the dense oracle in both activation modes, as the
    decode GEMV does."""
    for m, n, k in ((160, 384, 1024), (512, 512, 1024)):
        w = _rescaled_block_scales(fmt, packed(fmt, n, k, 80 + m), scales, m)
        a = activations(m, k, 81 + m)
        h = ctx.upload(fmt, n, k, w)
        try:
            for int8 in (True, False):
                exp = expected(fmt, w, n, k, a, int8)
                got = ctx.matmul(h, a, int8=int8)
                assert np.isfinite(got).all(), f"m {m} int8 {int8}"
                assert_row_tolerance(got, exp, f"m {m} n {n} int8 {int8}")
                assert_row_tolerance(ctx.matmul(h, a[:3], int8=int8), exp[:3], f"m 3 n {n} int8 {int8}")
        finally:
            h.release()


@pytest.mark.parametrize("scales", [_TINY_SCALES, _HUGE_SCALES], ids=["tiny", "huge"])
def test_k_split_form_weights_far_from_unit_scale(ks_ctx, scales):
    """The Q4_K K-split GEMM on weights with subnormal or near-65504 block
    scales, both activation modes, against the dense oracle."""
    m, n, k = 200, 300, 768
    w = _rescaled_block_scales(Q4_K, packed(Q4_K, n, k, 83), scales, 84)
    a = activations(m, k, 85)
    h = ks_ctx.upload(Q4_K, n, k, w)
    try:
        for int8 in (True, False):
            got = ks_ctx.matmul(h, a, int8=int8)
            assert np.isfinite(got).all()
            assert_row_tolerance(got, expected(Q4_K, w, n, k, a, int8), f"int8 {int8}")
    finally:
        h.release()


def test_matmul_is_deterministic_and_linear_in_weights_rows(ctx):
    """Repeated calls are bit-identical; each output column depends on its
    stored row only (a permutation of stored rows permutes the outputs)."""
    n, k = 512, 4096
    w = mg.quantize(Q4_K, mg.gaussian(9, 0.02, n * k).reshape(n, k))
    perm = np.random.default_rng(1).permutation(n)
    a = mg.gaussian(10, 1.0, 4 * k).reshape(4, k)
    h = ctx.upload(Q4_K, n, k, w)
    hp = ctx.upload(Q4_K, n, k, w[perm])
    try:
        for m in (1, 4):
            y1 = ctx.matmul(h, a[:m])
            np.testing.assert_array_equal(y1, ctx.matmul(h, a[:m]))
            np.testing.assert_array_equal(ctx.matmul(hp, a[:m]), y1[:, perm])
    finally:
        h.release()
        hp.release()


# ---- device-pointer entry points ------------------------------------------------------

def test_device_entry_points_agree_with_host_entry_point(ctx):
    name = "q4k_14336x4096_s1"
    fmt, n, k, seed, _ = workloads.WEIGHTS[name]
    h = ctx.upload(fmt, n, k, workloads.weight_bytes(name))
    try:
        stream = torch.cuda.current_stream().cuda_stream
        for m in (1, 4, 200):
            a = workloads.activations(seed, m, k)
            host = ctx.matmul(h, a)
            xd = dev(a)
            yd = torch.empty((m, n), dtype=torch.float32, device="cuda")
            ctx.matmul_dev(h, xd.data_ptr(), m, k, yd.data_ptr(), stream=stream)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(yd.cpu().numpy(), host)
            if m <= 8:
                v = torch.empty(m * k, dtype=torch.int8, device="cuda")
                sc = torch.empty(m * k // 32, dtype=torch.float32, device="cuda")
                sm = torch.empty(m * k // 16, dtype=torch.int32, device="cuda")
                ctx.quantize_activations_dev(xd.data_ptr(), m, k, v.data_ptr(), sc.data_ptr(), sm.data_ptr(),
                                             stream)
                y2 = torch.empty((m, n), dtype=torch.float32, device="cuda")
                ctx.matmul_prequantized_dev(h, v.data_ptr(), sc.data_ptr(), sm.data_ptr(), m, k,
                                            y2.data_ptr(), stream)
                torch.cuda.synchronize()
                np.testing.assert_array_equal(y2.cpu().numpy(), host)
        out = torch.empty((n, k), dtype=torch.float32, device="cuda")
        ctx.dequantize_dev(h, out.data_ptr(), stream=stream)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), ctx.dequantize(h))
    finally:
        h.release()


@pytest.mark.parametrize("fmt", [Q4_K, IQ4_XS])
@pytest.mark.parametrize("n,k", [(37, 512), (300, 4096), (520, 8192), (9, 256)])
def test_prequantized_every_m_matches_fused(ctx, fmt, n, k):
    """The pre-quantized GEMV (activations quantized by the caller) equals
    the fused one bit for bit at m = 1..8, over block counts that take the
    wave-local staging (<= 2 blocks per wave) and ones that do not."""
    w = packed(fmt, n, k, 95 + n)
    h = ctx.upload(fmt, n, k, w)
    stream = torch.cuda.current_stream().cuda_stream
    try:
        for m in range(1, 9):
            a = activations(m, k, 96 + m)
            host = ctx.matmul(h, a)
            assert_row_tolerance(host, expected(fmt, w, n, k, a, True), f"m {m}")
            xd = dev(a)
            v = torch.empty(m * k, dtype=torch.int8, device="cuda")
            sc = torch.empty(m * k // 32, dtype=torch.float32, device="cuda")
            sm = torch.empty(m * k // 16, dtype=torch.int32, device="cuda")
            ctx.quantize_activations_dev(xd.data_ptr(), m, k, v.data_ptr(), sc.data_ptr(), sm.data_ptr(), stream)
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")
            ctx.matmul_prequantized_dev(h, v.data_ptr(), sc.data_ptr(), sm.data_ptr(), m, k, y.data_ptr(), stream)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(y.cpu().numpy(), host, err_msg=f"m {m}")
    finally:
        h.release()


# ---- boundary behaviour ---------------------------------------------------------------

def test_boundary_errors_and_declines(ctx):
    w = packed(Q4_K, 4, 256, 41)
    with pytest.raises(mg.Declined):
        ctx.upload(19, 4, 256, np.zeros(4 * 50, np.uint8))  # IQ1_S has no GPU path
    with pytest.raises(mg.GpuError) as e:
        ctx.upload(Q4_K, 4, 256, w[:, :100])
    assert e.value.code == mg.ERR_SHAPE
    with pytest.raises(mg.GpuError) as e:
        ctx.upload(Q4_K, 4, 200, np.zeros(4 * 144, np.uint8))
    assert e.value.code == mg.ERR_SHAPE
    h = ctx.upload(Q4_K, 4, 256, w)
    try:
        info = ctx.info(h)
        assert (info["stored_rows"], info["stored_cols"], info["type"]) == (4, 256, Q4_K)
        assert h.logical_shape == (256, 4)
        with pytest.raises(mg.GpuError) as e:
            ctx.matmul(h, np.zeros((1, 512), np.float32))
        assert e.value.code == mg.ERR_SHAPE and "512 columns" in e.value.reason
        assert ctx.matmul(h, np.zeros((0, 256), np.float32)).shape == (0, 4)
    finally:
        h.release()
    with pytest.raises(mg.GpuError) as e:
        ctx.matmul(h, np.zeros((1, 256), np.float32))
    assert e.value.code == mg.ERR_ARGUMENT


def test_non_finite_activations(ctx):
    """f32 mode: a NaN activation makes its output row NaN (no zero-skip);
    int8 mode: NaN quantizes to 0, as the reference's `as i8` does. M = 40
    takes the f16 GEMM, whose row factor ignores the NaN."""
    n, k = 64, 512
    w = packed(Q4_K, n, k, 3)
    h = ctx.upload(Q4_K, n, k, w)
    try:
        for m in (1, 12, 40):
            a = activations(m, k, 5)
            a[0, 17] = np.nan
            y32 = ctx.matmul(h, a, int8=False)
            assert np.isnan(y32[0]).all() and np.isfinite(y32[1:]).all()
            y8 = ctx.matmul(h, a, int8=True)
            exp = expected(Q4_K, w, n, k, a, True)
            assert np.isfinite(y8).all()
            assert row_tolerance_violation(y8, exp) <= 1.0
    finally:
        h.release()


# ---- every decode-GEMV form and K-split ------------------------------------------

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


@pytest.mark.parametrize("fmt", [Q4_K, IQ4_XS])
def test_gemv_narrow_form(fmt):
    """The 16-row form (four lane quarters over the chunks of a block, no K
    split), forced for every shape: ragged row counts, 1..32 blocks (wave-
    and work-group-staged activations), m = 1..8, fused and pre-quantized
    (bit-identical to each other and when repeated), and with a residual;
    within the reference's tolerance of the dense oracle."""
    c = _context_with({"MQ_GEMV_NARROW": 1})
    stream = torch.cuda.current_stream().cuda_stream
    try:
        for n, k in ((1000, 2048), (37, 1280), (300, 4608), (9, 256), (40, 8192)):
            w = mg.quantize(fmt, mg.gaussian(n + k + 7, 0.02, n * k).reshape(n, k))
            h = c.upload(fmt, n, k, w)
            try:
                for m in (1, 3, 4, 5, 8):
                    a = mg.gaussian(500 + m, 1.0, m * k).reshape(m, k)
                    got = c.matmul(h, a)
                    np.testing.assert_array_equal(got.view(np.uint32), c.matmul(h, a).view(np.uint32))
                    exp = expected(fmt, w, n, k, a, True)
                    assert_close_reference(got, exp, f"n {n} k {k} m {m}")
                    xd = dev(a)
                    v = torch.empty(m * k, dtype=torch.int8, device="cuda")
                    sc = torch.empty(m * k // 32, dtype=torch.float32, device="cuda")
                    sm = torch.empty(m * k // 16, dtype=torch.int32, device="cuda")
                    c.quantize_activations_dev(xd.data_ptr(), m, k, v.data_ptr(), sc.data_ptr(), sm.data_ptr(),
                                               stream)
                    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
                    c.matmul_prequantized_dev(h, v.data_ptr(), sc.data_ptr(), sm.data_ptr(), m, k, y.data_ptr(),
                                              stream)
                    torch.cuda.synchronize()
                    np.testing.assert_array_equal(y.cpu().numpy(), got, err_msg=f"pre-quantized n {n} m {m}")
                    r = mg.gaussian(600 + m, 1.0, m * n).reshape(m, n)
                    rd = dev(r)
                    y2 = torch.empty((m, n), dtype=torch.float32, device="cuda")
                    c.matmul_add_dev(h, xd.data_ptr(), m, k, rd.data_ptr(), m, y2.data_ptr())
                    torch.cuda.synchronize()
                    np.testing.assert_array_equal(y2.cpu().numpy(), (got + r).astype(np.float32),
                                                  err_msg=f"residual n {n} m {m}")
            finally:
                h.release()
    finally:
        c.close()


@pytest.mark.parametrize("fmt", [Q4_K, IQ4_XS])
@pytest.mark.parametrize("variant,ksplit,splits", [(0, 1, 0), (0, 2, 0), (0, 3, 4), (0, 5, 8), (0, 16, 16),
                                                   (3, 4, 2), (3, 7, 0), (2, 1, 8), (1, 1, 4)])
def test_gemv_forms_and_k_splits(fmt, variant, ksplit, splits):
    """Every decode form (fused, LDS-staged, row-per-lane, 8 lanes per row)
    at K-splits that do and do not divide the super-block count (5 and 8
    blocks), ragged row counts, m = 1..8: within the reference's tolerance
    of the dense oracle, and bit-identical when repeated (the split-K
    epilogue adds the partials in a fixed order)."""
    c = _context_with({"MQ_GEMV_VARIANT": variant, "MQ_GEMV_KSPLIT": ksplit, "MQ_GEMV_SPLITS": splits})
    try:
        for n, k in ((1000, 2048), (37, 1280)):
            w = mg.quantize(fmt, mg.gaussian(n + k, 0.02, n * k).reshape(n, k))
            h = c.upload(fmt, n, k, w)
            try:
                for m in (1, 4, 5, 8):
                    a = mg.gaussian(300 + m, 1.0, m * k).reshape(m, k)
                    got = c.matmul(h, a)
                    again = c.matmul(h, a)
                    np.testing.assert_array_equal(got.view(np.uint32), again.view(np.uint32))
                    exp = expected(fmt, w, n, k, a, True)
                    assert_close_reference(got, exp, f"n {n} k {k} m {m}")
            finally:
                h.release()
    finally:
        c.close()
