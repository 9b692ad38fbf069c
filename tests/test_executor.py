"""The Provider-side contract of the GPU packed-weight matmul Kernel, ported
from the reference's own executor tests (src/native/tests.rs:251-331) and
the fused-epilogue tests (src/tests.rs:740-888)."""

import numpy as np
import pytest

import magnetar_gpu as mg
import oracle
from helpers import (IQ4_XS, PLANE_FORMATS, Q4_K, Q8_0, activations, assert_close_reference, assert_row_tolerance,
                     packed)
from magnetar_gpu import executor as ex


# ---- CPU-side -----------------------------------------------------------------

def test_kernel_advertisements_under_the_gpu_identity():
    """`provider_identity_is_distinct` (src/native/tests.rs:315-331): matmul is
    advertised, every advertisement under this Provider's identity, with the
    reference's f32 / contiguous / Host / TimeoutOnly shape."""
    ads = ex.kernel_advertisements()
    names = {a["name"] for a in ads}
    assert {"matmul", "matmul-bias", "matmul-residual", "embedding", "rmsnorm", "rope", "kv-write", "attention",
            "silu-mul", "add", "residual-add"} == names
    for a in ads:
        assert a["provider"] == "magnetar-provider-gpu-mi355x"
        assert a["provider"] != "magnetar-provider-cpu-reference"
        assert a["input_dtypes"] == ["f32"] and a["output_dtypes"] == ["f32"]
        assert a["layouts"] == ["Contiguous"] and a["memory_classes"] == ["Host"]
        assert a["cancellation"] == "TimeoutOnly"
        assert a["conformance_profile"] == "reference-cpu-conformance-v1"
    assert [a["rank"] for a in ads if a["name"] == "matmul"] == [2]


def test_absurd_tensor_shape_is_an_error_not_an_abort():
    """No exception crosses the C ABI: a [2^30, 2^30] tensor (4 EiB of f32)
    cannot be held, and mg_write_tensor returns MG_ERR_OOM instead of
    terminating the process (the host copy is attempted first)."""
    import ctypes

    L = ex.lib()
    shape = (ctypes.c_uint64 * 2)(1 << 30, 1 << 30)
    data = (ctypes.c_float * 4)()
    rc = L.mg_write_tensor(None, b"t", shape, 2, data)
    assert rc == ex.ERR_OOM
    assert b"memory" in L.mg_executor_last_error(None) or b"size" in L.mg_executor_last_error(None)
    # a shape whose byte count overflows 64 bits is rejected as an argument
    shape = (ctypes.c_uint64 * 2)(1 << 40, 1 << 40)
    assert L.mg_write_tensor(None, b"t", shape, 2, data) == ex.ERR_ARGUMENT


def test_executor_without_a_device_reports_an_error():
    """No GPU: creation fails with a structured error, nothing aborts."""
    torch = pytest.importorskip("torch")
    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is present")
    with pytest.raises(ex.ExecutorError) as e:
        ex.GpuExecutor(0)
    assert e.value.code == ex.ERR_DEVICE


# ---- GPU ------------------------------------------------------------------------

gpu = pytest.mark.gpu


@pytest.fixture
def executor():
    e = ex.GpuExecutor(0, packed_weights=True, int8_activations=True)
    yield e
    e.close()


@gpu
def test_executor_stores_packed_weights(executor):
    """`executor_stores_packed_weights` (src/native/tests.rs:251-274)."""
    w = packed(Q4_K, 4, 256, 41)
    assert executor.write_packed_weight_tensor("w", Q4_K, 4, 256, w)
    assert executor.is_packed("w")
    got = executor.read_tensor("w")
    exp = oracle.dequantize(Q4_K, w, 4, 256).T
    np.testing.assert_array_equal(got.view(np.uint32), np.ascontiguousarray(exp).view(np.uint32))
    assert executor.resident_shape("w") == [256, 4]
    assert executor.materializations() == 1
    assert executor.release_tensor("w")
    assert not executor.is_packed("w")
    declining = ex.GpuExecutor(0, packed_weights=False)
    try:
        assert not declining.write_packed_weight_tensor("w", Q4_K, 4, 256, w)
    finally:
        declining.close()
    # a format without a GPU path (IQ1_S) is declined; an untransposed
    # weight is stored with its logical shape [stored_rows, stored_cols]
    assert not executor.write_packed_weight_tensor("iq1", 19, 2, 256, np.zeros(2 * 50, np.uint8))
    assert executor.write_packed_weight_tensor("t", Q4_K, 4, 256, w, transposed=False)
    assert executor.resident_shape("t") == [4, 256]


@gpu
def test_packed_weights_yield_to_f32_writes_and_admission(executor):
    """`packed_weights_survive_opaque_writes_and_yield_to_copies`
    (src/native/tests.rs:276-313) for the writes this executor takes: an f32
    write replaces the packed weight; a denied admission leaves it resident."""
    w = packed(Q4_K, 2, 256, 43)
    assert executor.write_packed_weight_tensor("w", Q4_K, 2, 256, w)
    assert executor.read_tensor_value_is_opaque("w")
    replacement = np.full((256, 2), 0.5, np.float32)
    executor.write_tensor_admitted("w", replacement)
    assert not executor.is_packed("w")
    np.testing.assert_array_equal(executor.read_tensor("w"), replacement)
    small = ex.GpuExecutor(0, memory_capacity=1500)  # the weight's 1152 device bytes, not 2048 f32 ones
    try:
        assert small.write_packed_weight_tensor("w", Q4_K, 2, 256, w)
        assert small.memory_used() == 1152
        with pytest.raises(ex.ExecutorError) as e:
            small.write_tensor_admitted("w", replacement)
        assert e.value.code == ex.MEMORY_DENIED
        assert small.is_packed("w")
    finally:
        small.close()


@gpu
@pytest.mark.parametrize("fmt", [Q4_K, IQ4_XS])
@pytest.mark.parametrize("int8", [True, False])
def test_submitted_matmul_matches_reference_cpu(fmt, int8):
    """A `matmul` Kernel invocation through submit/complete, reading a packed
    weight: mode-matched against the dense oracle (src/native/tests.rs:134-154)."""
    e = ex.GpuExecutor(0, int8_activations=int8)
    try:
        k, n = 512, 37
        w = packed(fmt, n, k, 21)
        assert e.write_packed_weight_tensor("w", fmt, n, k, w)
        dense_t = oracle.dequantize(fmt, w, n, k)
        for m in (1, 3, 9):
            a = activations(m, k, m)
            e.write_tensor("a", a)
            h = e.submit_kernel("matmul", f"inv{m}", ["a", "w"], "y")
            r = e.complete_kernel(h)
            assert r.succeeded, r.reason
            got = e.read_tensor("y")
            exp = oracle.matmul_dense(oracle.int8_rounded(a) if int8 else a, dense_t, False, True)
            assert_row_tolerance(got, exp, f"m {m}")
            if m <= 8:
                assert_close_reference(got, exp, f"m {m}")
    finally:
        e.close()


@gpu
def test_fused_epilogues_equal_their_unfused_pairs(executor):
    """`matmul-bias` / `matmul-residual` bit-identical to matmul then add
    (src/tests.rs:740-888): the product is rounded before the addition."""
    k, n = 512, 64
    w = mg.quantize(Q4_K, mg.gaussian(3, 0.02, n * k).reshape(n, k))
    executor.write_packed_weight_tensor("w", Q4_K, n, k, w)
    for m in (1, 4, 12):
        a = mg.gaussian(10 + m, 1.0, m * k).reshape(m, k)
        executor.write_tensor("a", a)
        executor.complete_kernel(executor.submit_kernel("matmul", "p", ["a", "w"], "y"))
        y = executor.read_tensor("y")
        bias = mg.gaussian(20 + m, 1.0, n)
        residual = mg.gaussian(30 + m, 1.0, m * n).reshape(m, n)
        for kernel, extra, shape in (("matmul-bias", bias, (n,)), ("matmul-bias", bias.reshape(1, n), (1, n)),
                                     ("matmul-residual", residual, (m, n))):
            executor.write_tensor("x2", extra.reshape(shape))
            r = executor.complete_kernel(executor.submit_kernel(kernel, "f", ["a", "w", "x2"], "z"))
            assert r.succeeded, r.reason
            exp = (y + extra.reshape(1, n) if extra.size == n else residual + y).astype(np.float32)
            np.testing.assert_array_equal(executor.read_tensor("z"), exp)


@gpu
def test_transpose_a_takes_the_f32_path(executor):
    """`transpose_a` expands to the dense f32 matmul in the reference
    (src/native/mod.rs:221-222): f32 activations, read transposed."""
    k, n, m = 256, 16, 3
    w = packed(Q4_K, n, k, 8)
    executor.write_packed_weight_tensor("w", Q4_K, n, k, w)
    a_t = activations(k, m, 2)  # stored [k, m]
    executor.write_tensor("a", a_t)
    r = executor.complete_kernel(executor.submit_kernel("matmul", "t", ["a", "w"], "y", {"transpose_a": "true"}))
    assert r.succeeded, r.reason
    exp = oracle.matmul_dense(a_t, oracle.dequantize(Q4_K, w, n, k), True, True)
    assert_close_reference(executor.read_tensor("y"), exp)


@gpu
def test_kernel_errors_and_single_completion(executor):
    """Deadline 0 -> KernelTimeout before dispatch; f16 accumulation rejected
    (src/lib.rs:2445-2456); unknown Kernel; a second completion of one handle
    is rejected (src/lib.rs:2337-2356); a column mismatch carries the
    reference's reason text."""
    w = packed(Q4_K, 8, 256, 1)
    executor.write_packed_weight_tensor("w", Q4_K, 8, 256, w)
    executor.write_tensor("a", activations(1, 256, 1))
    h = executor.submit_kernel("matmul", "d0", ["a", "w"], "y", deadline_millis=0)
    assert executor.complete_kernel(h).error == ex.KERNEL_TIMEOUT
    with pytest.raises(ex.ExecutorError) as e:
        executor.complete_kernel(h)
    assert e.value.code == ex.UNKNOWN
    h = executor.submit_kernel("matmul", "f16", ["a", "w"], "y", {"accumulation_dtype": "f16"})
    assert executor.complete_kernel(h).error == ex.KERNEL_DTYPE_UNSUPPORTED
    h = executor.submit_kernel("softmax", "s", ["a"], "y")
    assert executor.complete_kernel(h).error == ex.KERNEL_NOT_FOUND
    executor.write_tensor("b", activations(1, 512, 1))
    r = executor.complete_kernel(executor.submit_kernel("matmul", "k", ["b", "w"], "y"))
    assert r.error == ex.KERNEL_EXECUTION_FAILED and "512 columns" in r.reason
    kinds = [k for k, _ in executor.observations()]
    assert kinds[:2] == ["ProviderRegistered", "DeviceDetected"]
    assert "KernelTimeout" in kinds and "KernelDispatchFailed" in kinds


@gpu
def test_output_admission_denial_does_not_store(executor):
    small = ex.GpuExecutor(0, memory_capacity=1160)  # the weight's 1152 device bytes, not the 32-byte output
    try:
        w = packed(Q4_K, 8, 256, 1)
        assert small.write_packed_weight_tensor("w", Q4_K, 8, 256, w)
        small.write_tensor("a", activations(1, 256, 1))
        r = small.complete_kernel(small.submit_kernel("matmul", "big", ["a", "w"], "y"))
        assert r.error == ex.KERNEL_EXECUTION_FAILED and "admission denied" in r.reason
        assert small.read_tensor("y") is None
        assert ("KernelMemoryFeasibilityFailed", "matmul") in small.observations()
    finally:
        small.close()


@gpu
def test_packed_weight_device_bytes_are_admitted(executor):
    """A packed upload the memory ledger cannot hold is declined and leaves
    the previous weight of the id resident; releases return the bytes."""
    small = ex.GpuExecutor(0, memory_capacity=3000)
    try:
        w1 = packed(Q4_K, 8, 256, 2)
        assert small.write_packed_weight_tensor("w", Q4_K, 8, 256, w1)
        assert small.memory_used() == 1152
        big = packed(Q4_K, 24, 256, 3)  # 3 row groups: 3456 device bytes
        assert not small.write_packed_weight_tensor("w", Q4_K, 24, 256, big)
        assert small.is_packed("w") and small.resident_shape("w") == [256, 8]
        assert small.release_tensor("w")
        assert small.memory_used() == 0
    finally:
        small.close()


@gpu
@pytest.mark.parametrize("fmt", [Q8_0, Q4_K])
def test_embedding_kernel_on_packed_tables(executor, fmt):
    """`packed_tables_serve_lookups_and_tied_heads` (src/native/tests.rs:178-191)
    through Kernels: an untransposed packed table [50, 64] serves `embedding`
    (bit-exact rows, the `scale` attribute) and, read transposed, a tied
    output head; a transposed table [dim, vocab] gathers each token's column."""
    cols = 64 if fmt == Q8_0 else 256
    table = packed(fmt, 50, cols, 31)
    dense = oracle.dequantize(fmt, table, 50, cols)  # logical [vocab, dim]
    assert executor.write_packed_weight_tensor("tab", fmt, 50, cols, table, transposed=False)
    executor.write_tensor("ids", np.array([7, 0, 49, 7], np.float32))
    r = executor.complete_kernel(executor.submit_kernel("embedding", "e", ["tab", "ids"], "rows"))
    assert r.succeeded, r.reason
    np.testing.assert_array_equal(executor.read_tensor("rows"), dense[[7, 0, 49, 7]])
    r = executor.complete_kernel(executor.submit_kernel("embedding", "e2", ["tab", "ids"], "rows", {"scale": "0.5"}))
    assert r.succeeded, r.reason
    np.testing.assert_array_equal(executor.read_tensor("rows"), dense[[7, 0, 49, 7]] * np.float32(0.5))
    executor.write_tensor("bad", np.array([50], np.float32))
    r = executor.complete_kernel(executor.submit_kernel("embedding", "e3", ["tab", "bad"], "rows"))
    assert r.error == ex.KERNEL_EXECUTION_FAILED
    assert r.reason == "token id 50 is not below the vocabulary size 50"
    # tied head: the untransposed table read transposed multiplies output-major
    a = activations(2, cols, 3)
    executor.write_tensor("h", a)
    r = executor.complete_kernel(executor.submit_kernel("matmul", "head", ["h", "tab"], "logits",
                                                        {"transpose_b": "true"}))
    assert r.succeeded, r.reason
    exp = oracle.matmul_dense(oracle.int8_rounded(a), dense, False, True)
    assert_close_reference(executor.read_tensor("logits"), exp, "tied head")
    # a transposed table: stored [dim][vocab]
    tt = packed(fmt, 40, cols, 33)
    dense_t = oracle.dequantize(fmt, tt, 40, cols)  # stored rows = dim
    assert executor.write_packed_weight_tensor("tt", fmt, 40, cols, tt, transposed=True)
    executor.write_tensor("ids2", np.array([3, 63], np.float32))
    r = executor.complete_kernel(executor.submit_kernel("embedding", "e4", ["tt", "ids2"], "cols"))
    assert r.succeeded, r.reason
    np.testing.assert_array_equal(executor.read_tensor("cols"), dense_t[:, [3, 63]].T)


@gpu
@pytest.mark.parametrize("fmt", PLANE_FORMATS + [Q4_K, IQ4_XS])
def test_input_major_weights_multiply_packed(executor, fmt):
    """`input_major_weights_multiply_packed` (src/native/tests.rs:193-209):
    an untransposed [64, 256] weight read without transpose_b multiplies
    through the axpy product, f32 activations, every format."""
    w = packed(fmt, 64, 256, 61)
    dense = oracle.dequantize(fmt, w, 64, 256)  # logical [k, n]
    assert executor.write_packed_weight_tensor("w", fmt, 64, 256, w, transposed=False)
    for m in (1, 4, 9):
        a = activations(m, 64, 62)
        executor.write_tensor("a", a)
        r = executor.complete_kernel(executor.submit_kernel("matmul", f"ax{m}", ["a", "w"], "y"))
        assert r.succeeded, r.reason
        assert_close_reference(executor.read_tensor("y"), oracle.matmul_dense(a, dense), f"m {m}")
