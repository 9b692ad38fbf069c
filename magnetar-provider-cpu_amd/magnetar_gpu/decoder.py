"""A Llama-3-8B-shaped decoder layer decode step, device-resident.

The step is the sequence of Kernels the Runtime submits for one generated
token, each one an entry point of ``libmagnetar_gpu.so``:

    xn  = rmsnorm(x, g_attn, eps)                     (src/lib.rs:348-402)
    q, k, v = xn . Wq^T, xn . Wk^T, xn . Wv^T          packed matmul (int8 activations),
                                                       one launch over the stacked rows
    q, k = rope(q), rope(k) at position `position`     (src/lib.rs:427-687)
    K[position], V[position] = k, v                    kv-write (src/lib.rs:740-768)
    a   = attention(q, K, V, key_count = position + 1) (src/lib.rs:780-990)
    h   = x + a . Wo^T                                 matmul-residual (src/lib.rs:2577-2590)
    hn  = rmsnorm(h, g_ffn, eps)
    f   = silu(hn . Wgate^T) * (hn . Wup^T)            silu-mul (src/lib.rs:2592-2596),
                                                       gate and up as one launch
    out = h + f . Wdown^T                              matmul-residual

All intermediates stay in HBM (torch tensors used as device allocations);
only the projections' packed weights and the f32 KV cache are read from
HBM in bulk. Shapes: hidden 4096, 32 query / 8 key-value heads of 128,
FFN 14336, rmsnorm eps 1e-5, rope theta 5e5.
"""

import numpy as np

from . import EPILOGUE_ROPE_KV, EPILOGUE_SILU_PAIRS, Q4_K, gaussian, quantize

HIDDEN = 4096
HEADS = 32
KV_HEADS = 8
HEAD_DIM = 128
FFN = 14336
EPS = 1e-5
THETA = 5e5

QKV_ROWS = (HEADS + 2 * KV_HEADS) * HEAD_DIM

# projection name -> (stored rows N, stored cols K)
PROJECTIONS = {
    "q": (HEADS * HEAD_DIM, HIDDEN),
    "k": (KV_HEADS * HEAD_DIM, HIDDEN),
    "v": (KV_HEADS * HEAD_DIM, HIDDEN),
    "o": (HIDDEN, HEADS * HEAD_DIM),
    "gate": (FFN, HIDDEN),
    "up": (FFN, HIDDEN),
    "down": (HIDDEN, FFN),
}


class LayerData:
    """Seeded synthetic layer (host arrays): Q4_K projections from
    N(0, 0.02), rmsnorm weights 1 + N(0, 0.02), a KV cache of `capacity`
    rows whose first `prefilled` rows are N(0, 1), and an N(0, 1) input
    hidden state. Generator seeds 1000 s + 1 + i for the i-th array."""

    def __init__(self, seed=4, capacity=4096, prefilled=4095, quantize_fn=quantize):
        base = 1000 * seed
        self.capacity, self.prefilled = capacity, prefilled
        self.weights = {}
        for i, (name, (n, k)) in enumerate(PROJECTIONS.items()):
            self.weights[name] = quantize_fn(Q4_K, gaussian(base + 1 + i, 0.02, n * k).reshape(n, k))
        self.g_attn = (1.0 + gaussian(base + 11, 0.02, HIDDEN)).astype(np.float32)
        self.g_ffn = (1.0 + gaussian(base + 12, 0.02, HIDDEN)).astype(np.float32)
        width = KV_HEADS * HEAD_DIM
        self.k_cache = np.zeros((capacity, width), np.float32)
        self.v_cache = np.zeros((capacity, width), np.float32)
        self.k_cache[:prefilled] = gaussian(base + 13, 1.0, prefilled * width).reshape(prefilled, width)
        self.v_cache[:prefilled] = gaussian(base + 14, 1.0, prefilled * width).reshape(prefilled, width)
        self.x = gaussian(base + 500, 1.0, HIDDEN).reshape(1, HIDDEN)

    def weight_bytes(self):
        return sum(int(w.size) for w in self.weights.values())


def interleave_gate_up(gate, up, block=32):
    """Stored rows of gate and up interleaved in blocks of `block` rows (the
    layout mq_decode_matmul_dev's silu-pairs epilogue reads)."""
    n, rb = gate.shape
    return np.stack([gate.reshape(n // block, block, rb), up.reshape(n // block, block, rb)], axis=1).reshape(2 * n, rb)


class DecoderLayer:
    """The layer on one device: uploads the packed weights and the KV
    cache, allocates every intermediate once, and runs `step` (all device
    work enqueued on one stream; nothing allocated per step).

    fused=True runs the step in 6 launches through mq_decode_matmul_dev:
    rmsnorm + QKV GEMV + rope + kv-write; attention partials; combine;
    O GEMV + residual; rmsnorm + gate/up GEMV + silu-mul; down GEMV +
    residual. fused=False runs each operator's own entry point (12)."""

    def __init__(self, ctx, torch, data, int8=True, fused=False):
        self.ctx, self.torch, self.int8, self.fused = ctx, torch, int8, fused
        if fused and not int8:
            raise ValueError("the fused decode step quantizes its activations to int8")
        dev = "cuda"
        # Q, K and V share their input, as do gate and up: each trio/pair is
        # uploaded as one matrix of stacked rows (a row's bytes do not
        # depend on its neighbours) and runs as one launch.
        w = data.weights
        self.w = {name: ctx.upload(Q4_K, *PROJECTIONS[name], w[name]) for name in ("o", "down")}
        self.w["qkv"] = ctx.upload(Q4_K, QKV_ROWS, HIDDEN, np.concatenate([w["q"], w["k"], w["v"]]))
        if fused:
            self.w["gate_up"] = ctx.upload(Q4_K, 2 * FFN, HIDDEN, interleave_gate_up(w["gate"], w["up"]))
        else:
            self.w["gate_up"] = ctx.upload(Q4_K, 2 * FFN, HIDDEN, np.concatenate([w["gate"], w["up"]]))
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
        self.g_attn, self.g_ffn = t(data.g_attn), t(data.g_ffn)
        self.k_cache, self.v_cache = t(data.k_cache), t(data.v_cache)
        self.capacity = data.capacity
        e = lambda n: torch.empty((1, n), dtype=torch.float32, device=dev)  # noqa: E731
        self.x = t(data.x)
        self.xn, self.qkv = e(HIDDEN), e(QKV_ROWS)
        self.a, self.h, self.hn = e(HEADS * HEAD_DIM), e(HIDDEN), e(HIDDEN)
        self.gu, self.f, self.out = e(2 * FFN), e(FFN), e(HIDDEN)

    def step(self, position, stream=None):
        """One decode step for the token at `position` (its K/V row is
        written there; attention reads rows 0..position)."""
        if not 0 <= position < self.capacity:
            raise ValueError(f"position {position} outside the {self.capacity}-row KV cache")
        if self.fused:
            return self._step_fused(position, stream)
        c, p = self.ctx, lambda t: t.data_ptr()  # noqa: E731
        c.rmsnorm_dev(p(self.x), 1, HIDDEN, p(self.g_attn), 1, EPS, p(self.xn), stream=stream)
        c.matmul_dev(self.w["qkv"], p(self.xn), 1, HIDDEN, p(self.qkv), int8=self.int8, stream=stream)
        # q rotated in place; k rotated straight into the K cache's row
        # `position`; v copied into the V cache's row (kv-write)
        width = KV_HEADS * HEAD_DIM
        q, k, v = p(self.qkv), p(self.qkv) + HIDDEN * 4, p(self.qkv) + (HIDDEN + width) * 4
        c.rope_dev(q, 1, HIDDEN, THETA, 1.0, HEAD_DIM, position, HEADS, q, stream=stream)
        c.rope_dev(k, 1, width, THETA, 1.0, HEAD_DIM, position, KV_HEADS, p(self.k_cache) + position * width * 4,
                   stream=stream)
        c.kv_write_dev(p(self.v_cache), self.capacity, width, v, 1, position, stream=stream)
        c.attention_dev(q, 1, p(self.k_cache), p(self.v_cache), self.capacity, position + 1, HEADS,
                        HEAD_DIM, KV_HEADS, p(self.a), causal=True, stream=stream)
        c.matmul_add_dev(self.w["o"], p(self.a), 1, HEADS * HEAD_DIM, p(self.x), 1, p(self.h), int8=self.int8,
                         stream=stream)
        c.rmsnorm_dev(p(self.h), 1, HIDDEN, p(self.g_ffn), 1, EPS, p(self.hn), stream=stream)
        c.matmul_dev(self.w["gate_up"], p(self.hn), 1, HIDDEN, p(self.gu), int8=self.int8, stream=stream)
        c.silu_mul_dev(p(self.gu), p(self.gu) + FFN * 4, FFN, p(self.f), stream=stream)
        c.matmul_add_dev(self.w["down"], p(self.f), 1, FFN, p(self.h), 1, p(self.out), int8=self.int8,
                         stream=stream)
        return self.out

    def _step_fused(self, position, stream):
        c, p = self.ctx, lambda t: t.data_ptr()  # noqa: E731
        width = KV_HEADS * HEAD_DIM
        q = p(self.qkv)
        c.decode_matmul_dev(self.w["qkv"], p(self.x), HIDDEN, norm_weight_ptr=p(self.g_attn), norm_epsilon=EPS,
                            epilogue=EPILOGUE_ROPE_KV, rope_rows=HIDDEN + width, rope_dim=HEAD_DIM,
                            rope_offset=position, rope_base=THETA, rope_scale=1.0,
                            segments=[(0, q), (HIDDEN, p(self.k_cache) + position * width * 4),
                                      (HIDDEN + width, p(self.v_cache) + position * width * 4)], stream=stream)
        c.attention_dev(q, 1, p(self.k_cache), p(self.v_cache), self.capacity, position + 1, HEADS,
                        HEAD_DIM, KV_HEADS, p(self.a), causal=True, stream=stream)
        c.matmul_add_dev(self.w["o"], p(self.a), 1, HEADS * HEAD_DIM, p(self.x), 1, p(self.h), int8=True,
                         stream=stream)
        c.decode_matmul_dev(self.w["gate_up"], p(self.h), HIDDEN, p(self.f), norm_weight_ptr=p(self.g_ffn),
                            norm_epsilon=EPS, epilogue=EPILOGUE_SILU_PAIRS, stream=stream)
        c.matmul_add_dev(self.w["down"], p(self.f), 1, FFN, p(self.h), 1, p(self.out), int8=True, stream=stream)
        return self.out

    def release(self):
        for w in self.w.values():
            w.release()
        self.w = {}


def reference_step(data, position, oracle, int8=True):
    """The same step on the CPU oracle (test infrastructure): the packed
    matmuls through the reference's scalar column kernel in the same
    activation mode, the other operators as restated in oracle/layer.c.
    Returns (out, k_cache, v_cache) with the caches updated."""
    def mm(name, x):
        n, k = PROJECTIONS[name]
        return oracle.columns_scalar(Q4_K, data.weights[name], n, k, x, int8)

    k_cache, v_cache = data.k_cache.copy(), data.v_cache.copy()
    xn = oracle.rmsnorm(data.x, data.g_attn, EPS)
    q = oracle.rope(mm("q", xn), THETA, 1.0, HEAD_DIM, position, HEADS)
    k = oracle.rope(mm("k", xn), THETA, 1.0, HEAD_DIM, position, KV_HEADS)
    v = mm("v", xn)
    oracle.kv_write(k_cache, k, position)
    oracle.kv_write(v_cache, v, position)
    a = oracle.attention(q, k_cache[:position + 1], v_cache[:position + 1], HEADS, HEAD_DIM, KV_HEADS, True)
    h = oracle.add(data.x, mm("o", a))
    hn = oracle.rmsnorm(h, data.g_ffn, EPS)
    f = oracle.silu_mul(mm("gate", hn), mm("up", hn))
    out = oracle.add(h, mm("down", f))
    return out, k_cache, v_cache
