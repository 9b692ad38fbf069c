"""The Provider with device-resident tensors: the storage half of
`ProviderExecutionApi` (src/native/mod.rs:622-806; src/lib.rs:1556-1868)
and the decoder-layer Kernels (src/lib.rs:2528-3058) submitted through
mg_submit_kernel / mg_complete_kernel, up to one whole Llama-3-8B-shaped
decode step against the oracle."""

import os

import numpy as np
import pytest

import oracle
from helpers import Q4_K, Q8_0, activations, packed
from magnetar_gpu import decoder
from magnetar_gpu import executor as ex

pytestmark = pytest.mark.gpu


@pytest.fixture
def executor():
    e = ex.GpuExecutor(0, packed_weights=True, int8_activations=True)
    yield e
    e.close()


def run(e, kernel, inputs, output, attributes=None, name=None):
    r = e.complete_kernel(e.submit_kernel(kernel, name or kernel, inputs, output, attributes))
    assert r.succeeded, f"{kernel}: [{r.error}] {r.reason}"


def close(got, exp, rel, what=""):
    scale = max(float(np.max(np.abs(exp))), 1e-30)
    err = float(np.max(np.abs(got.astype(np.float64) - exp.astype(np.float64))))
    assert err <= rel * scale, f"{what}: max|d| {err:.3e} > {rel:.1e} * {scale:.3e}"


def test_packed_weights_survive_opaque_writes_and_yield_to_copies(executor):
    """`packed_weights_survive_opaque_writes_and_yield_to_copies`
    (src/native/tests.rs:276-313): writing back the Opaque value a packed
    weight reads as keeps it; a copy onto its identity replaces it."""
    w = packed(Q8_0, 2, 32, 43)
    assert executor.write_packed_weight_tensor("w", Q8_0, 2, 32, w)
    assert executor.read_tensor_value_is_opaque("w")
    executor.write_tensor_value("w")  # the Opaque value back
    assert executor.is_packed("w")
    executor.write_tensor_value("w", admitted=True)
    assert executor.is_packed("w")
    replacement = np.full((32, 2), 0.5, np.float32)
    executor.write_tensor_admitted("source", replacement)
    executor.copy_tensor_admitted("source", "w")
    assert not executor.is_packed("w")
    np.testing.assert_array_equal(executor.read_tensor("w"), replacement)
    # a Host value replaces a packed weight too
    assert executor.write_packed_weight_tensor("w2", Q8_0, 2, 32, w)
    executor.write_tensor_value("w2", replacement)
    assert not executor.is_packed("w2")
    np.testing.assert_array_equal(executor.read_tensor("w2"), replacement)


def test_copy_of_a_packed_weight_is_its_materialization(executor):
    """copy_tensor_admitted from a packed weight stores its logical values;
    a missing source is an admission error with the reference's text
    (src/lib.rs:1768-1772)."""
    w = packed(Q4_K, 8, 256, 5)
    assert executor.write_packed_weight_tensor("w", Q4_K, 8, 256, w)
    executor.copy_tensor_admitted("w", "dense")
    exp = oracle.dequantize(Q4_K, w, 8, 256).T
    np.testing.assert_array_equal(executor.read_tensor("dense").view(np.uint32),
                                  np.ascontiguousarray(exp).view(np.uint32))
    assert executor.is_packed("w") and not executor.is_packed("dense")
    with pytest.raises(ex.ExecutorError) as e:
        executor.copy_tensor_admitted("nowhere", "x")
    assert e.value.code == ex.MEMORY_DENIED and "source resource 'nowhere' not found" in e.value.reason


def test_admission_release_and_workspaces():
    """The memory ledger: write_tensor_admitted and copies admit their bytes,
    release_admitted_tensor returns them, workspaces are admitted and
    released by allocation id, and a denied copy leaves the target."""
    e = ex.GpuExecutor(0, memory_capacity=4096)
    try:
        e.write_tensor_admitted("a", np.ones((4, 64), np.float32))  # 1024 B
        assert e.memory_used() == 1024
        e.copy_tensor_admitted("a", "b")
        assert e.memory_used() == 2048
        ws = e.allocate_workspace(1024)
        assert e.memory_used() == 3072
        with pytest.raises(ex.ExecutorError) as err:
            e.allocate_workspace(2048)
        assert err.value.code == ex.MEMORY_DENIED
        e.copy_tensor_admitted("a", "c")  # 4096 of 4096
        with pytest.raises(ex.ExecutorError) as err:
            e.copy_tensor_admitted("a", "d")
        assert err.value.code == ex.MEMORY_DENIED
        assert e.read_tensor("d") is None
        e.release_workspace(ws)
        with pytest.raises(ex.ExecutorError):
            e.release_workspace(ws)
        assert e.release_admitted_tensor("b")
        assert e.read_tensor("b") is None
        np.testing.assert_array_equal(e.read_tensor("a"), np.ones((4, 64), np.float32))
    finally:
        e.close()


def test_zeroed_kv_store_and_kv_write(executor):
    """`write_zeroed_kv_store` (src/lib.rs:1633-1690): a zeroed f32 store of
    whole heads, replacing a packed weight of the id; TurboQuant precisions
    and ragged widths are declined. `kv-write` in place and into a copy
    (src/lib.rs:2458-2526), with the reference's bounds text."""
    w = packed(Q4_K, 8, 256, 9)
    assert executor.write_packed_weight_tensor("K", Q4_K, 8, 256, w)
    assert executor.write_zeroed_kv_store("K", [16, 256], 128)
    assert not executor.is_packed("K")
    np.testing.assert_array_equal(executor.read_tensor("K"), np.zeros((16, 256), np.float32))
    assert not executor.write_zeroed_kv_store("bad", [16, 200], 128)
    assert not executor.write_zeroed_kv_store("tq", [16, 256], 128, precision=1)
    rows = activations(3, 256, 4)
    executor.write_tensor("rows", rows)
    run(executor, "kv-write", ["K", "rows"], "K", {"row_offset": 5})
    exp = np.zeros((16, 256), np.float32)
    exp[5:8] = rows
    np.testing.assert_array_equal(executor.read_tensor("K"), exp)
    run(executor, "kv-write", ["K", "rows"], "K2", {"row_offset": 13})
    exp2 = exp.copy()
    exp2[13:16] = rows
    np.testing.assert_array_equal(executor.read_tensor("K2"), exp2)
    np.testing.assert_array_equal(executor.read_tensor("K"), exp)  # the store itself unchanged
    r = executor.complete_kernel(executor.submit_kernel("kv-write", "over", ["K", "rows"], "K", {"row_offset": 14}))
    assert r.error == ex.KERNEL_EXECUTION_FAILED
    assert r.reason == "kv-write of 3 rows at 14 exceeds the store's 16 rows"
    r = executor.complete_kernel(executor.submit_kernel("kv-write", "no", ["K", "rows"], "K"))
    assert r.error == ex.KERNEL_ATTRIBUTE_UNSUPPORTED


def test_layer_kernels_match_the_oracle(executor):
    """rmsnorm (one weight row, per-row weights; the forms without a GPU
    path refused), rope (interleaved and half_split, position offset), attention (causal,
    GQA, key_count, scale), silu-mul, add and residual-add (equal shapes and
    one broadcast row) through submitted Kernels, against the oracle."""
    r = np.random.default_rng(3)
    x = r.standard_normal((3, 512)).astype(np.float32)
    g = (1 + 0.02 * r.standard_normal(512)).astype(np.float32)
    gr = (1 + 0.02 * r.standard_normal((3, 512))).astype(np.float32)
    executor.write_tensor("x", x)
    executor.write_tensor("g", g)
    executor.write_tensor("gr", gr)
    run(executor, "rmsnorm", ["x", "g"], "xn", {"epsilon": "1e-5"})
    close(executor.read_tensor("xn"), oracle.rmsnorm(x, g, 1e-5), 2e-6, "rmsnorm")
    run(executor, "rmsnorm", ["x", "gr"], "xn", {"epsilon": "1e-5"})
    close(executor.read_tensor("xn"), oracle.rmsnorm(x, gr, 1e-5), 2e-6, "rmsnorm per row")
    # the head-block and weightless forms (external rmsnorm_blocks in the
    # reference) and a contradicting with_scale are refused
    for inputs, attrs in ((["x"], {}), (["x", "g"], {"head_count": 4, "head_dimension": 128}),
                          (["x", "g"], {"with_scale": "false"})):
        res = executor.complete_kernel(executor.submit_kernel("rmsnorm", "r", inputs, "xn", attrs))
        assert res.error == ex.KERNEL_ATTRIBUTE_UNSUPPORTED, (inputs, attrs)
    executor.write_tensor("g7", g[:7])
    res = executor.complete_kernel(executor.submit_kernel("rmsnorm", "r", ["x", "g7"], "xn"))
    assert res.error == ex.KERNEL_EXECUTION_FAILED and res.reason.startswith("RMSNorm weight shape must be [512]")

    for pairing in ("interleaved", "half_split"):
        run(executor, "rope", ["x"], "xr", {"base": "500000", "dimension": 128, "position_offset": 7,
                                          "head_count": 4, "rotation_pairing": pairing})
        exp = oracle.rope(x, 5e5, 1.0, 128, 7, 4, half_split=pairing == "half_split")
        close(executor.read_tensor("xr"), exp, 2e-6, f"rope {pairing}")
    res = executor.complete_kernel(executor.submit_kernel("rope", "y", ["x"], "xr", {"dimension": 128,
                                                                                   "rope_type": "yarn"}))
    assert res.error == ex.KERNEL_ATTRIBUTE_UNSUPPORTED
    res = executor.complete_kernel(executor.submit_kernel("rope", "n", ["x"], "xr", {"dimension": 128,
                                                                                   "position_offset": -1}))
    assert res.error == ex.KERNEL_ATTRIBUTE_UNSUPPORTED and "must not be negative" in res.reason

    q = r.standard_normal((2, 8 * 128)).astype(np.float32)
    kv = r.standard_normal((2, 40, 2 * 128)).astype(np.float32)
    executor.write_tensor("q", q)
    executor.write_tensor("K", kv[0])
    executor.write_tensor("V", kv[1])
    for causal, scale in ((True, None), (False, 0.05)):
        attrs = {"head_count": 8, "head_dimension": 128, "kv_head_count": 2, "causal": "true" if causal else "false",
                 "key_count": 33}
        if scale is not None:
            attrs["scale"] = str(scale)
        run(executor, "attention", ["q", "K", "V"], "att", attrs)
        exp = oracle.attention(q, kv[0][:33], kv[1][:33], 8, 128, 2, causal, scale)
        close(executor.read_tensor("att"), exp, 1e-5, f"attention causal={causal}")
    res = executor.complete_kernel(executor.submit_kernel("attention", "w", ["q", "K", "V"], "att",
                                                          {"head_count": 8, "head_dimension": 128, "window_size": 4}))
    assert res.error == ex.KERNEL_ATTRIBUTE_UNSUPPORTED
    res = executor.complete_kernel(executor.submit_kernel("attention", "kc", ["q", "K", "V"], "att",
                                                          {"head_count": 8, "head_dimension": 128,
                                                           "kv_head_count": 2, "key_count": 41}))
    assert res.error == ex.KERNEL_EXECUTION_FAILED and res.reason == "key_count 41 exceeds the 40 rows of K/V"

    gate = (4 * r.standard_normal((2, 700))).astype(np.float32)
    up = r.standard_normal((2, 700)).astype(np.float32)
    executor.write_tensor("gate", gate)
    executor.write_tensor("up", up)
    run(executor, "silu-mul", ["gate", "up"], "f")
    close(executor.read_tensor("f"), oracle.silu_mul(gate, up), 1e-6, "silu-mul")
    executor.write_tensor("row", up[0])
    res = executor.complete_kernel(executor.submit_kernel("silu-mul", "s", ["gate", "row"], "f"))
    assert res.error == ex.KERNEL_EXECUTION_FAILED and "shape mismatch" in res.reason
    for kernel in ("add", "residual-add"):
        run(executor, kernel, ["gate", "up"], "sum")
        np.testing.assert_array_equal(executor.read_tensor("sum"), gate + up)
        run(executor, kernel, ["gate", "row"], "sum")
        np.testing.assert_array_equal(executor.read_tensor("sum"), gate + up[0])
    # an output that is also an input is computed into a new buffer
    run(executor, "add", ["gate", "up"], "gate")
    np.testing.assert_array_equal(executor.read_tensor("gate"), gate + up)
    executor.write_tensor("bad", up[:, :7])
    res = executor.complete_kernel(executor.submit_kernel("add", "b", ["up", "bad"], "sum"))
    assert res.error == ex.KERNEL_EXECUTION_FAILED
    assert res.reason == "add expects b to match a's shape [2, 700] or broadcast as [700]/[1, 700], got [2, 7]"


def test_matmul_residual_broadcasts_a_one_row_product(executor):
    """`matmul-residual` is residual_add(residual, product) = add(residual,
    product) (src/native/mod.rs:232-233): a [1, n] product adds as one
    broadcast row to an [r, n] residual, the output the residual's shape."""
    k, n = 256, 48
    w = packed(Q4_K, n, k, 12)
    assert executor.write_packed_weight_tensor("w", Q4_K, n, k, w)
    a = activations(1, k, 3)
    residual = activations(5, n, 4)
    executor.write_tensor("a", a)
    executor.write_tensor("res", residual)
    run(executor, "matmul", ["a", "w"], "p")
    run(executor, "matmul-residual", ["a", "w", "res"], "out")
    p = executor.read_tensor("p")
    np.testing.assert_array_equal(executor.read_tensor("out"), residual + p)
    executor.write_tensor("bad", activations(5, n + 1, 4))
    res = executor.complete_kernel(executor.submit_kernel("matmul-residual", "b", ["a", "w", "bad"], "out"))
    assert res.error == ex.KERNEL_EXECUTION_FAILED and "add expects b" in res.reason


def test_decode_step_through_the_provider_matches_the_oracle(executor):
    """One Llama-3-8B-shaped decoder layer decode step (hidden 4096, 32/8
    heads of 128, FFN 14336, Q4_K projections, eps 1e-5, theta 5e5, 4095
    cached tokens, seed 4) submitted Kernel by Kernel as the Runtime would:
    every tensor stays on the device between Kernels, the K/V rows are
    written into the caches in place. The output within 1e-3 * max|out|
    (the packed matmul's bar) of the same step on the oracle; the caches'
    old rows untouched, the new rows within 1e-3 of their scale."""
    data = decoder.LayerData(seed=4)
    for name, (n, k) in decoder.PROJECTIONS.items():
        assert executor.write_packed_weight_tensor(f"w_{name}", Q4_K, n, k, data.weights[name])
    executor.write_tensor("g_attn", data.g_attn)
    executor.write_tensor("g_ffn", data.g_ffn)
    width = decoder.KV_HEADS * decoder.HEAD_DIM
    assert executor.write_zeroed_kv_store("k_cache", [data.capacity, width], decoder.HEAD_DIM)
    assert executor.write_zeroed_kv_store("v_cache", [data.capacity, width], decoder.HEAD_DIM)
    executor.write_tensor("k_prefill", data.k_cache[:data.prefilled])
    executor.write_tensor("v_prefill", data.v_cache[:data.prefilled])
    run(executor, "kv-write", ["k_cache", "k_prefill"], "k_cache", {"row_offset": 0})
    run(executor, "kv-write", ["v_cache", "v_prefill"], "v_cache", {"row_offset": 0})
    executor.write_tensor("x", data.x)
    pos = data.prefilled
    eps = str(decoder.EPS)
    rope = {"base": str(decoder.THETA), "dimension": decoder.HEAD_DIM, "position_offset": pos}
    run(executor, "rmsnorm", ["x", "g_attn"], "xn", {"epsilon": eps})
    for p in ("q", "k", "v"):
        run(executor, "matmul", ["xn", f"w_{p}"], p)
    run(executor, "rope", ["q"], "q_rot", dict(rope, head_count=decoder.HEADS))
    run(executor, "rope", ["k"], "k_rot", dict(rope, head_count=decoder.KV_HEADS))
    run(executor, "kv-write", ["k_cache", "k_rot"], "k_cache", {"row_offset": pos})
    run(executor, "kv-write", ["v_cache", "v"], "v_cache", {"row_offset": pos})
    run(executor, "attention", ["q_rot", "k_cache", "v_cache"], "attn",
        {"head_count": decoder.HEADS, "head_dimension": decoder.HEAD_DIM, "kv_head_count": decoder.KV_HEADS,
         "causal": "true", "attention_mask_kind": "causal", "key_count": pos + 1})
    run(executor, "matmul-residual", ["attn", "w_o", "x"], "h")
    run(executor, "rmsnorm", ["h", "g_ffn"], "hn", {"epsilon": eps})
    run(executor, "matmul", ["hn", "w_gate"], "gate")
    run(executor, "matmul", ["hn", "w_up"], "up")
    run(executor, "silu-mul", ["gate", "up"], "f")
    run(executor, "matmul-residual", ["f", "w_down", "h"], "out")
    for rid in ("q_rot", "attn", "h", "out"):
        assert executor.read_tensor_value_is_opaque(rid)
    out = executor.read_tensor("out")
    kc, vc = executor.read_tensor("k_cache"), executor.read_tensor("v_cache")
    exp, ekc, evc = decoder.reference_step(data, pos, oracle)
    assert out.shape == (1, decoder.HIDDEN)
    close(out, exp, 1e-3, "decode step through the Provider")
    np.testing.assert_array_equal(kc[:pos], data.k_cache[:pos])
    np.testing.assert_array_equal(vc[:pos], data.v_cache[:pos])
    close(kc[pos], ekc[pos], 1e-3, "new K row")
    close(vc[pos], evc[pos], 1e-3, "new V row")
    kinds = [k for k, _ in executor.observations()]
    assert "KernelDispatchFailed" not in kinds


def test_profile_times_each_kernel():
    """MAGNETAR_GPU_PROFILE=1 (the reference's MAGNETAR_CPU_PROFILE,
    src/native/mod.rs:29-31, 605-619): calls and seconds per Kernel name."""
    os.environ["MAGNETAR_GPU_PROFILE"] = "1"
    try:
        e = ex.GpuExecutor(0)
    finally:
        del os.environ["MAGNETAR_GPU_PROFILE"]
    try:
        w = packed(Q4_K, 64, 256, 2)
        assert e.write_packed_weight_tensor("w", Q4_K, 64, 256, w)
        e.write_tensor("a", activations(1, 256, 1))
        for i in range(3):
            run(e, "matmul", ["a", "w"], "y", name=f"m{i}")
        run(e, "add", ["y", "y"], "z")
        prof = {name: (calls, secs) for name, calls, secs in e.profile()}
        assert prof["matmul"][0] == 3 and prof["add"][0] == 1
        assert all(secs > 0 for _, secs in prof.values())
    finally:
        e.close()
    plain = ex.GpuExecutor(0)
    try:
        assert plain.profile() == []
    finally:
        plain.close()
