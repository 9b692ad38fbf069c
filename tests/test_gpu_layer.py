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
