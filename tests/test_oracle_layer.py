"""Pins of the decoder-layer oracle (oracle/layer.c) against closed forms,
float64 restatements and exact invariants, none of which retype the
oracle's own formula in f32."""

import math

import numpy as np
import pytest

import oracle


def rng(seed):
    return np.random.default_rng(seed)


# ---- rmsnorm (src/lib.rs:348-402) ------------------------------------------------

def test_rmsnorm_known_answer():
    x = np.array([[3.0, 4.0]], np.float32)
    got = oracle.rmsnorm(x, np.ones(2, np.float32), 1e-6)
    s = 1.0 / math.sqrt(12.5 + 1e-6)
    np.testing.assert_allclose(got, [[3 * s, 4 * s]], rtol=1e-7)


def test_rmsnorm_against_float64_and_weight_shapes():
    r = rng(1)
    x = r.standard_normal((5, 4096)).astype(np.float32)
    w = r.standard_normal(4096).astype(np.float32)
    x64 = x.astype(np.float64)
    exp = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + 1e-5) * w
    np.testing.assert_allclose(oracle.rmsnorm(x, w, 1e-5), exp, rtol=2e-6, atol=1e-6)
    # a [1, cols] weight is the same broadcast; a [rows, cols] weight is per row
    np.testing.assert_array_equal(oracle.rmsnorm(x, w.reshape(1, -1), 1e-5), oracle.rmsnorm(x, w, 1e-5))
    w2 = r.standard_normal((5, 4096)).astype(np.float32)
    for i in range(5):
        np.testing.assert_array_equal(oracle.rmsnorm(x, w2, 1e-5)[i], oracle.rmsnorm(x[i:i + 1], w2[i], 1e-5)[0])


def test_rmsnorm_is_scale_invariant_and_rejects_bad_epsilon():
    r = rng(2)
    x = r.standard_normal((2, 256)).astype(np.float32)
    w = np.ones(256, np.float32)
    # a power-of-two scale of x leaves the normalised value (eps negligible)
    np.testing.assert_allclose(oracle.rmsnorm(4 * x, w, 1e-12), oracle.rmsnorm(x, w, 1e-12), rtol=1e-6)
    with pytest.raises(ValueError):
        oracle.rmsnorm(x, w, 0.0)
    with pytest.raises(ValueError):
        oracle.rmsnorm(x, w, -1e-5)
    with pytest.raises(ValueError):
        oracle.rmsnorm(x, np.ones(3, np.float32), 1e-5)
    # the reference tests `epsilon <= 0.0` (src/lib.rs:388): NaN is accepted
    # and propagates through the scale
    assert np.all(np.isnan(oracle.rmsnorm(x, w, float("nan"))))


# ---- rope (src/lib.rs:427-687) -----------------------------------------------------

def test_rope_position_zero_is_identity():
    x = rng(3).standard_normal((1, 4096)).astype(np.float32)
    np.testing.assert_array_equal(oracle.rope(x, 5e5, 1.0, 128, 0, 32), x)


def test_rope_matches_rotation_of_its_f32_angles():
    """Each pair is rotated by the angle (offset + r) * scale * base^(-2p/d)
    computed in f32 (as the reference does); sin/cos of that angle in
    float64 pin the rotation to within f32 rounding."""
    r = rng(4)
    rows, heads, dim = 3, 4, 128
    x = r.standard_normal((rows, heads * dim)).astype(np.float32)
    got = oracle.rope(x, 5e5, 1.0, dim, 4093, heads)
    for row in range(rows):
        pos = np.float32(4093 + row) * np.float32(1.0)
        for h in range(heads):
            for p in range(dim // 2):
                f = np.float32(np.float32(5e5) ** np.float32(np.float32(-2.0 * p) / np.float32(dim)))
                ang = float(np.float32(pos * f))
                a, b = float(x[row, h * dim + 2 * p]), float(x[row, h * dim + 2 * p + 1])
                ea = a * math.cos(ang) - b * math.sin(ang)
                eb = a * math.sin(ang) + b * math.cos(ang)
                tol = 4e-7 * (abs(a) + abs(b)) + 1e-7
                assert abs(got[row, h * dim + 2 * p] - ea) <= tol
                assert abs(got[row, h * dim + 2 * p + 1] - eb) <= tol


def test_rope_half_split_is_a_column_permutation_of_interleaved():
    r = rng(5)
    dim, heads = 8, 2
    x = r.standard_normal((2, heads * dim)).astype(np.float32)
    # interleaved pair p = (2p, 2p+1); half-split pair p = (p, p + dim/2)
    perm = np.concatenate([np.arange(0, dim, 2), np.arange(1, dim, 2)])
    cols = np.concatenate([h * dim + perm for h in range(heads)])
    inter = oracle.rope(x, 100.0, 1.0, dim, 7, heads)
    half = oracle.rope(x[:, cols], 100.0, 1.0, dim, 7, heads, half_split=True)
    np.testing.assert_array_equal(half, inter[:, cols])


def test_rope_partial_dimension_leaves_the_tail_and_rejects_bad_shapes():
    x = rng(6).standard_normal((2, 16)).astype(np.float32)
    out = oracle.rope(x, 10000.0, 1.0, 4, 5, 2)
    np.testing.assert_array_equal(out[:, 4:8], x[:, 4:8])
    np.testing.assert_array_equal(out[:, 12:16], x[:, 12:16])
    assert not np.array_equal(out[:, 0:4], x[:, 0:4])
    for args in ((10000.0, 1.0, 3, 0, 2), (10000.0, 1.0, 10, 0, 2), (10000.0, 1.0, 4, 0, 3), (-1.0, 1.0, 4, 0, 2)):
        with pytest.raises(ValueError):
            oracle.rope(x, *args)


# ---- kv-write (src/lib.rs:740-768) -------------------------------------------------

def test_kv_write_in_place_and_bounds():
    store = np.zeros((6, 4), np.float32)
    rows = np.arange(8, dtype=np.float32).reshape(2, 4)
    oracle.kv_write(store, rows, 3)
    np.testing.assert_array_equal(store[3:5], rows)
    assert not store[:3].any() and not store[5:].any()
    with pytest.raises(ValueError):
        oracle.kv_write(store, rows, 5)


# ---- attention (src/lib.rs:780-990) ------------------------------------------------

def attention64(q, k, v, heads, dim, kv_heads, causal):
    seq, kv_seq = q.shape[0], k.shape[0]
    out = np.zeros((seq, heads * dim))
    g = heads // kv_heads
    for h in range(heads):
        kh = h // g
        for t in range(seq):
            upper = kv_seq - seq + t + 1 if causal else kv_seq
            qv = q[t, h * dim:(h + 1) * dim].astype(np.float64)
            kk = k[:upper, kh * dim:(kh + 1) * dim].astype(np.float64)
            vv = v[:upper, kh * dim:(kh + 1) * dim].astype(np.float64)
            s = kk @ qv / math.sqrt(dim)
            w = np.exp(s - s.max())
            out[t, h * dim:(h + 1) * dim] = (w / w.sum()) @ vv
    return out


@pytest.mark.parametrize("seq,kv_seq,causal", [(1, 257, True), (5, 5, True), (3, 9, False)])
def test_attention_against_float64_gqa(seq, kv_seq, causal):
    r = rng(7 + seq)
    heads, kv_heads, dim = 8, 2, 16
    q = r.standard_normal((seq, heads * dim)).astype(np.float32)
    k = r.standard_normal((kv_seq, kv_heads * dim)).astype(np.float32)
    v = r.standard_normal((kv_seq, kv_heads * dim)).astype(np.float32)
    got = oracle.attention(q, k, v, heads, dim, kv_heads, causal)
    np.testing.assert_allclose(got, attention64(q, k, v, heads, dim, kv_heads, causal), rtol=2e-5, atol=2e-6)


def test_attention_closed_forms():
    r = rng(8)
    dim = 4
    # one admitted key: the output is that key's value, exactly
    q = r.standard_normal((1, dim)).astype(np.float32)
    k = r.standard_normal((1, dim)).astype(np.float32)
    v = r.standard_normal((1, dim)).astype(np.float32)
    np.testing.assert_array_equal(oracle.attention(q, k, v, 1, dim, 1, True), v)
    # identical keys: uniform weights, the output is the mean of the values
    k = np.repeat(r.standard_normal((1, dim)).astype(np.float32), 8, axis=0)
    v = r.standard_normal((8, dim)).astype(np.float32)
    np.testing.assert_allclose(oracle.attention(q, k, v, 1, dim, 1, True)[0], v.mean(axis=0), rtol=1e-6, atol=1e-7)


def test_attention_uses_the_shared_kv_head_of_each_group():
    r = rng(9)
    heads, kv_heads, dim = 4, 2, 8
    q = np.tile(r.standard_normal((1, dim)).astype(np.float32), (1, heads))
    k = r.standard_normal((6, kv_heads * dim)).astype(np.float32)
    v = r.standard_normal((6, kv_heads * dim)).astype(np.float32)
    out = oracle.attention(q, k, v, heads, dim, kv_heads, True)
    # heads 0, 1 share kv head 0; heads 2, 3 share kv head 1
    np.testing.assert_array_equal(out[0, 0:dim], out[0, dim:2 * dim])
    np.testing.assert_array_equal(out[0, 2 * dim:3 * dim], out[0, 3 * dim:4 * dim])
    assert not np.array_equal(out[0, 0:dim], out[0, 2 * dim:3 * dim])


# ---- silu-mul and add ------------------------------------------------------------

def test_silu_mul_against_float64():
    r = rng(10)
    g = (r.standard_normal(14336) * 3).astype(np.float32)
    u = r.standard_normal(14336).astype(np.float32)
    g64 = g.astype(np.float64)
    np.testing.assert_allclose(oracle.silu_mul(g, u), g64 / (1 + np.exp(-g64)) * u, rtol=3e-6, atol=1e-7)
    np.testing.assert_array_equal(oracle.silu_mul(np.zeros(4, np.float32), np.ones(4, np.float32)), np.zeros(4))


def test_add_broadcasts_one_row():
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    b = np.array([1, 2, 3, 4], np.float32)
    np.testing.assert_array_equal(oracle.add(a, b), a + b)
    np.testing.assert_array_equal(oracle.add(a, a), a + a)
    with pytest.raises(ValueError):
        oracle.add(a, np.ones(5, np.float32))
