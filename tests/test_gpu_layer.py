"""GPU parity of the decoder-layer operators and of the full decode step
against the oracle (oracle/layer.c). Tolerances are written per test: these
are f32 operators whose reductions add in a different (tree) order than
the reference's left-to-right sums, and whose exp / sin / cos come from the
device math library, so they agree to a few ulps of the output scale."""

import numpy as np
import pytest

import magnetar_gpu as mg
import oracle
from magnetar_gpu import decoder

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def close(got, exp, rel, what=""):
    scale = max(float(np.max(np.abs(exp))), 1e-30)
    err = float(np.max(np.abs(got.astype(np.float64) - exp.astype(np.float64))))
    assert err <= rel * scale, f"{what}: max|d| {err:.3e} > {rel:.1e} * {scale:.3e}"


def rng(seed):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("rows,cols,per_row", [(1, 4096, False), (5, 4096, True), (3, 100, False), (2, 14336, False)])
def test_rmsnorm(ctx, rows, cols, per_row):
    r = rng(rows + cols)
    x = (r.standard_normal((rows, cols)) * 3).astype(np.float32)
    w = r.standard_normal((rows, cols) if per_row else cols).astype(np.float32)
    out = torch.empty((rows, cols), dtype=torch.float32, device="cuda")
    xd, wd = dev(x), dev(w)  # kept alive until the kernel has run
    ctx.rmsnorm_dev(xd.data_ptr(), rows, cols, wd.data_ptr(), rows if per_row else 1, 1e-5, out.data_ptr())
    close(host(out), oracle.rmsnorm(x, w, 1e-5), 2e-6, "rmsnorm")


def test_rmsnorm_epsilon_rule_matches_the_reference(ctx):
    """The reference rejects epsilon <= 0 and nothing else (src/lib.rs:388):
    zero and negative epsilons are shape errors, NaN runs and gives NaN."""
    x = torch.from_numpy(rng(7).standard_normal((2, 256)).astype(np.float32)).cuda()
    w = torch.ones(256, dtype=torch.float32, device="cuda")
    out = torch.empty_like(x)
    for eps in (0.0, -1e-5):
        with pytest.raises(mg.GpuError) as e:
            ctx.rmsnorm_dev(x.data_ptr(), 2, 256, w.data_ptr(), 1, eps, out.data_ptr())
        assert e.value.code == mg.ERR_SHAPE and "epsilon must be positive" in e.value.reason
    ctx.rmsnorm_dev(x.data_ptr(), 2, 256, w.data_ptr(), 1, float("nan"), out.data_ptr())
    assert torch.isnan(out).all()


@pytest.mark.parametrize("heads,dim,offset,half,inplace", [(32, 128, 4095, False, False), (8, 128, 4095, False, True),
                                                           (4, 64, 7, True, False), (2, 16, 100000, False, False)])
def test_rope(ctx, heads, dim, offset, half, inplace):
    r = rng(heads * dim + offset)
    rows = 3
    x = r.standard_normal((rows, heads * dim)).astype(np.float32)
    xd = dev(x)
    out = xd if inplace else torch.empty_like(xd)
    ctx.rope_dev(xd.data_ptr(), rows, heads * dim, 5e5, 1.0, dim, offset, heads, out.data_ptr(), half_split=half)
    close(host(out), oracle.rope(x, 5e5, 1.0, dim, offset, heads, half_split=half), 1e-6, "rope")


def test_rope_partial_dimension_copies_the_tail(ctx):
    x = rng(11).standard_normal((2, 4 * 32)).astype(np.float32)
    out = torch.full((2, 128), 7.0, dtype=torch.float32, device="cuda")
    xd = dev(x)
    ctx.rope_dev(xd.data_ptr(), 2, 128, 10000.0, 1.0, 16, 3, 4, out.data_ptr())
    got = host(out)
    exp = oracle.rope(x, 10000.0, 1.0, 16, 3, 4)
    close(got, exp, 1e-6, "partial rope")
    for h in range(4):
        np.testing.assert_array_equal(got[:, h * 32 + 16:(h + 1) * 32], x[:, h * 32 + 16:(h + 1) * 32])


def test_kv_write_is_exact_and_bounded(ctx):
    store = np.zeros((16, 64), np.float32)
    rows = rng(12).standard_normal((3, 64)).astype(np.float32)
    sd, rd = dev(store), dev(rows)
    ctx.kv_write_dev(sd.data_ptr(), 16, 64, rd.data_ptr(), 3, 10)
    np.testing.assert_array_equal(host(sd), oracle.kv_write(store.copy(), rows, 10))
    with pytest.raises(mg.GpuError):
        ctx.kv_write_dev(sd.data_ptr(), 16, 64, rd.data_ptr(), 3, 14)


@pytest.mark.parametrize("seq,key_count,kv_rows,heads,kv_heads,causal", [
    (1, 4096, 4096, 32, 8, True),   # the Llama-3-8B decode step
    (1, 5000, 5000, 32, 8, True),   # 79 chunks: past the combine's 16 prefetched chunks per wave
    (1, 100, 4096, 32, 8, True),    # key_count below the store's rows
    (5, 300, 512, 8, 8, True),      # multi-row, causal
    (3, 65, 65, 16, 2, False),      # bidirectional
    (2, 130, 200, 8, 1, True),
])
def test_attention(ctx, seq, key_count, kv_rows, heads, kv_heads, causal):
    r = rng(seq * 7 + key_count)
    dim = 128
    q = r.standard_normal((seq, heads * dim)).astype(np.float32)
    k = r.standard_normal((kv_rows, kv_heads * dim)).astype(np.float32)
    v = r.standard_normal((kv_rows, kv_heads * dim)).astype(np.float32)
    out = torch.empty((seq, heads * dim), dtype=torch.float32, device="cuda")
    qd, kd, vd = dev(q), dev(k), dev(v)
    ctx.attention_dev(qd.data_ptr(), seq, kd.data_ptr(), vd.data_ptr(), kv_rows, key_count, heads, dim,
                      kv_heads, out.data_ptr(), causal=causal)
    exp = oracle.attention(q, k[:key_count], v[:key_count], heads, dim, kv_heads, causal)
    close(host(out), exp, 2e-5, "attention")


def test_attention_decode_step_equals_the_prefill_row(ctx):
    """`attention_decode_step_matches_the_corresponding_prefill_row`
    (src/tests.rs:283-334): the last query row of a causal prefill is the
    same computation as a one-row decode step, bit for bit."""
    r = rng(13)
    heads, kv_heads, dim, n = 8, 2, 128, 200
    qf = r.standard_normal((n, heads * dim)).astype(np.float32)
    k = dev(r.standard_normal((n, kv_heads * dim)).astype(np.float32))
    v = dev(r.standard_normal((n, kv_heads * dim)).astype(np.float32))
    full = torch.empty((n, heads * dim), dtype=torch.float32, device="cuda")
    qd, qs = dev(qf), dev(qf[-1:])
    ctx.attention_dev(qd.data_ptr(), n, k.data_ptr(), v.data_ptr(), n, n, heads, dim, kv_heads, full.data_ptr())
    step = torch.empty((1, heads * dim), dtype=torch.float32, device="cuda")
    ctx.attention_dev(qs.data_ptr(), 1, k.data_ptr(), v.data_ptr(), n, n, heads, dim, kv_heads, step.data_ptr())
    np.testing.assert_array_equal(host(step)[0], host(full)[-1])


def test_attention_rejects_and_declines(ctx):
    zt = torch.zeros(1 << 16, dtype=torch.float32, device="cuda")
    z = zt.data_ptr()
    with pytest.raises(mg.GpuError):  # head_count not a multiple of kv_head_count
        ctx.attention_dev(z, 1, z, z, 8, 8, 6, 128, 4, z)
    with pytest.raises(mg.GpuError):  # key_count beyond the store
        ctx.attention_dev(z, 1, z, z, 8, 9, 8, 128, 8, z)
    with pytest.raises(mg.Declined):  # head_dim without a GPU path
        ctx.attention_dev(z, 1, z, z, 8, 8, 8, 64, 8, z)


def test_silu_mul_and_add(ctx):
    r = rng(14)
    g = (r.standard_normal(14336) * 4).astype(np.float32)
    u = r.standard_normal(14336).astype(np.float32)
    out = torch.empty(14336, dtype=torch.float32, device="cuda")
    gd, ud = dev(g), dev(u)
    ctx.silu_mul_dev(gd.data_ptr(), ud.data_ptr(), 14336, out.data_ptr())
    close(host(out), oracle.silu_mul(g, u), 1e-6, "silu-mul")
    a = r.standard_normal((3, 64)).astype(np.float32)
    b = r.standard_normal(64).astype(np.float32)
    o2 = torch.empty((3, 64), dtype=torch.float32, device="cuda")
    ad, bd = dev(a), dev(b)
    ctx.add_dev(ad.data_ptr(), a.size, bd.data_ptr(), b.size, o2.data_ptr())
    np.testing.assert_array_equal(host(o2), oracle.add(a, b))


def test_decoder_layer_decode_step_matches_the_oracle(ctx):
    """The Llama-3-8B-shaped layer (hidden 4096, 32/8 heads of 128, FFN
    14336, Q4_K projections, eps 1e-5, theta 5e5, 4095 cached tokens, seed
    4), one decode step at position 4095, device-resident, against the same
    step on the oracle with the reference's int8 packed matmul: the output
    within 1e-3 * max|out| (the packed matmul's own bar), the new K/V rows
    within 1e-3 of their scale."""
    data = decoder.LayerData(seed=4)
    layer = decoder.DecoderLayer(ctx, torch, data)
    try:
        out = host(layer.step(4095))
        kc, vc = host(layer.k_cache), host(layer.v_cache)
    finally:
        layer.release()
    exp, ekc, evc = decoder.reference_step(data, 4095, oracle)
    close(out, exp, 1e-3, "decoder layer output")
    np.testing.assert_array_equal(kc[:4095], data.k_cache[:4095])
    close(kc[4095], ekc[4095], 1e-3, "new K row")
    close(vc[4095], evc[4095], 1e-3, "new V row")


# ---- decode-step fusions (mq_decode_matmul_dev) -----------------------------------

def test_decoder_layer_fused_step_matches_the_oracle(ctx):
    """The same step in 6 launches (rmsnorm, rope and kv-write fused into
    the QKV GEMV; rmsnorm and silu-mul into the gate/up GEMV) against the
    oracle, at the packed matmul's 1e-3 bar."""
    data = decoder.LayerData(seed=4)
    layer = decoder.DecoderLayer(ctx, torch, data, fused=True)
    try:
        out = host(layer.step(4095))
        kc, vc = host(layer.k_cache), host(layer.v_cache)
    finally:
        layer.release()
    exp, ekc, evc = decoder.reference_step(data, 4095, oracle)
    close(out, exp, 1e-3, "fused decoder layer output")
    np.testing.assert_array_equal(kc[:4095], data.k_cache[:4095])
    close(kc[4095], ekc[4095], 1e-3, "new K row")
    close(vc[4095], evc[4095], 1e-3, "new V row")


def _q4k(seed, n, k):
    return mg.quantize(mg.Q4_K, mg.gaussian(seed, 0.02, n * k).reshape(n, k))


@pytest.fixture(params=["default", "narrow"])
def form_ctx(request, ctx):
    """The session context (this test's shapes take the 64-row GEMV form),
    and one whose GEMVs all take the 16-row form."""
    if request.param == "default":
        yield ctx
        return
    import os
    old = os.environ.get("MQ_GEMV_NARROW")
    os.environ["MQ_GEMV_NARROW"] = "1"
    try:
        c = mg.Context(0)
    finally:
        if old is None:
            del os.environ["MQ_GEMV_NARROW"]
        else:
            os.environ["MQ_GEMV_NARROW"] = old
    yield c
    c.close()


def test_rope_kv_epilogue_equals_the_unfused_chain(form_ctx):
    """GEMV + rope + kv-write in one launch equals matmul_dev, rope_dev and
    kv_write_dev bit for bit (same kernel results, same rotation), in
    either GEMV form."""
    ctx = form_ctx
    n, k, dim, pos = 768, 1024, 64, 37
    w = _q4k(5, n, k)
    h = ctx.upload(mg.Q4_K, n, k, w)
    x = dev(rng(3).standard_normal((1, k)))
    try:
        y = torch.empty((1, n), dtype=torch.float32, device="cuda")
        ctx.matmul_dev(h, x.data_ptr(), 1, k, y.data_ptr())
        ref = torch.empty_like(y)
        ctx.rope_dev(y.data_ptr(), 1, 512, 10000.0, 1.0, dim, pos, 512 // dim, ref.data_ptr())
        exp = host(y).copy()
        exp[:, :512] = host(ref)[:, :512]
        q = torch.zeros((1, 384), dtype=torch.float32, device="cuda")
        kc = torch.zeros((4, 128), dtype=torch.float32, device="cuda")
        vc = torch.zeros((4, 256), dtype=torch.float32, device="cuda")
        ctx.decode_matmul_dev(h, x.data_ptr(), k, epilogue=mg.EPILOGUE_ROPE_KV, rope_rows=512, rope_dim=dim,
                              rope_offset=pos, rope_base=10000.0,
                              segments=[(0, q.data_ptr()), (384, kc.data_ptr() + 2 * 128 * 4),
                                        (512, vc.data_ptr() + 1 * 256 * 4)])
        got = np.concatenate([host(q)[0], host(kc)[2], host(vc)[1]])
        np.testing.assert_array_equal(got, exp[0])
        assert not host(kc)[[0, 1, 3]].any() and not host(vc)[[0, 2, 3]].any()
    finally:
        h.release()


def test_silu_pairs_epilogue_equals_silu_mul(ctx):
    """Interleaved gate/up GEMV with silu-mul in the epilogue equals the
    plain GEMV followed by silu_mul_dev, bit for bit."""
    f, k = 640, 1024
    g, u = _q4k(6, f, k), _q4k(7, f, k)
    wi = decoder.interleave_gate_up(g, u)
    h = ctx.upload(mg.Q4_K, 2 * f, k, wi)
    x = dev(rng(4).standard_normal((1, k)))
    try:
        y = torch.empty((1, 2 * f), dtype=torch.float32, device="cuda")
        ctx.matmul_dev(h, x.data_ptr(), 1, k, y.data_ptr())
        yy = host(y)[0].reshape(-1, 2, 32)
        gd, ud = dev(yy[:, 0].reshape(-1)), dev(yy[:, 1].reshape(-1))
        exp = torch.empty(f, dtype=torch.float32, device="cuda")
        ctx.silu_mul_dev(gd.data_ptr(), ud.data_ptr(), f, exp.data_ptr())
        out = torch.empty(f, dtype=torch.float32, device="cuda")
        ctx.decode_matmul_dev(h, x.data_ptr(), k, out.data_ptr(), epilogue=mg.EPILOGUE_SILU_PAIRS)
        np.testing.assert_array_equal(host(out), host(exp))
    finally:
        h.release()


@pytest.mark.parametrize("n", [4096, 6144, 14336])
def test_norm_staging_matches_rmsnorm_then_matmul(ctx, n):
    """rmsnorm folded into the GEMV's staging: within the matmul bar of the
    rmsnorm_dev + matmul_dev chain (the sum of squares adds in another
    order, so an int8 rounding may differ), and of the oracle; at row
    counts that take the 16-row form (4096, 6144) and the 64-row form."""
    k = 4096
    w = _q4k(8, n, k)
    h = ctx.upload(mg.Q4_K, n, k, w)
    xh = (rng(5).standard_normal((1, k)) * 3).astype(np.float32)
    gh = (1 + 0.1 * rng(6).standard_normal(k)).astype(np.float32)
    x, gw = dev(xh), dev(gh)
    try:
        xn = torch.empty_like(x)
        ctx.rmsnorm_dev(x.data_ptr(), 1, k, gw.data_ptr(), 1, 1e-5, xn.data_ptr())
        y1 = torch.empty((1, n), dtype=torch.float32, device="cuda")
        ctx.matmul_dev(h, xn.data_ptr(), 1, k, y1.data_ptr())
        y2 = torch.empty_like(y1)
        ctx.decode_matmul_dev(h, x.data_ptr(), k, y2.data_ptr(), norm_weight_ptr=gw.data_ptr(), norm_epsilon=1e-5)
        close(host(y2), host(y1), 1e-3, "fused vs chained")
        exp = oracle.columns_scalar(mg.Q4_K, w, n, k, oracle.rmsnorm(xh, gh, 1e-5), True)
        close(host(y2), exp, 1e-3, "fused vs oracle")
    finally:
        h.release()


def test_decode_fusion_rejects_and_declines(ctx):
    w8 = mg.quantize(mg.Q4_K, mg.gaussian(1, 0.02, 96 * 256).reshape(96, 256))
    h = ctx.upload(mg.Q4_K, 96, 256, w8)
    z = torch.zeros(1 << 12, dtype=torch.float32, device="cuda")
    try:
        with pytest.raises(mg.GpuError):  # gate/up pairs need a multiple of 64 rows
            ctx.decode_matmul_dev(h, z.data_ptr(), 256, z.data_ptr(), epilogue=mg.EPILOGUE_SILU_PAIRS)
        with pytest.raises(mg.GpuError):  # rope rows must be whole heads
            ctx.decode_matmul_dev(h, z.data_ptr(), 256, epilogue=mg.EPILOGUE_ROPE_KV, rope_rows=50, rope_dim=64,
                                  segments=[(0, z.data_ptr())])
        with pytest.raises(mg.GpuError):  # k mismatch
            ctx.decode_matmul_dev(h, z.data_ptr(), 512, z.data_ptr())
    finally:
        h.release()
    from magnetar_gpu import workloads
    hq = ctx.upload(mg.Q8_0, 64, 256, workloads.random_blocks(mg.Q8_0, 64, 256, 3))
    try:
        with pytest.raises(mg.Declined):
            ctx.decode_matmul_dev(hq, z.data_ptr(), 256, z.data_ptr(), epilogue=mg.EPILOGUE_SILU_PAIRS)
    finally:
        hq.release()
