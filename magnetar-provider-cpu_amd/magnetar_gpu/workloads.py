"""The benchmark workloads: shapes, seeds and synthetic data.

Weights are N(0, 0.02) f32 encoded by this package's GGUF encoders; the
activations are N(0, 1). Stream seeds: weight i of a workload with seed s
uses generator seed 1000 s + 1 + i, its activations 1000 s + 500
(``gg_gaussian_f32``: splitmix64 feeding Box-Muller).

Stored-row convention as the reference's packed weights: a projection
W [N, K] is stored as N rows (the output columns) of K values, transposed
(logical shape [K, N]), so y[M, N] = x[M, K] . W^T.
"""

import functools

import numpy as np

from . import BLOCK_BYTES, BLOCK_VALUES, IQ4_XS, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, gaussian, quantize

# name -> (gguf type, stored rows N, stored cols K, workload seed, weight index)
WEIGHTS = {
    "q4k_4096x4096_s0": (Q4_K, 4096, 4096, 0, 0),
    "q4k_14336x4096_s1": (Q4_K, 14336, 4096, 1, 0),
    "q4k_4096x4096_s2": (Q4_K, 4096, 4096, 2, 0),
    "q4k_14336x4096_s2": (Q4_K, 14336, 4096, 2, 1),
    "iq4xs_4096x14336_s3": (IQ4_XS, 4096, 14336, 3, 0),
}


def weight_seed(seed, index):
    return 1000 * seed + 1 + index


def activation_seed(seed):
    return 1000 * seed + 500


@functools.lru_cache(maxsize=8)
def weight_f32(name):
    fmt, n, k, seed, index = WEIGHTS[name]
    return gaussian(weight_seed(seed, index), 0.02, n * k).reshape(n, k)


@functools.lru_cache(maxsize=8)
def weight_bytes(name):
    fmt, n, k, seed, index = WEIGHTS[name]
    return quantize(fmt, weight_f32(name))


def activations(seed, m, k):
    return gaussian(activation_seed(seed), 1.0, m * k).reshape(m, k)


def weight_bytes_per_call(name):
    fmt, n, k, _, _ = WEIGHTS[name]
    return n * k // 256 * (144 if fmt == Q4_K else 136)


def scale_offsets(fmt):
    """Byte offsets of a block's f16 scale fields."""
    if fmt in (Q4_K, Q5_K):
        return (0, 2)
    return {Q6_K: (208,), Q2_K: (80, 82), Q3_K: (108,)}.get(fmt, (0,))


def random_blocks(fmt, rows, cols, seed):
    """Checkpoint-shaped random blocks for timing the formats without an
    encoder: uniform random bytes with every f16 scale field a small
    positive value (exponent 3..7, as the reference's own test matrices).
    uint8 [rows, row bytes]."""
    bb, bv = BLOCK_BYTES[fmt], BLOCK_VALUES[fmt]
    rng = np.random.default_rng(seed)
    blocks = rng.integers(0, 256, size=(rows * cols // bv, bb), dtype=np.uint8)
    for at in scale_offsets(fmt):
        bits = (rng.integers(3, 8, size=blocks.shape[0]) << 10) | rng.integers(0, 1024, size=blocks.shape[0])
        blocks[:, at] = bits & 0xFF
        blocks[:, at + 1] = bits >> 8
    return blocks.reshape(rows, cols // bv * bb)


def synthetic_iq_grids(seed=1):
    """Stand-in IQ2 / IQ3 grid tables (the real ones are the caller's:
    magnetar-provider-api `iq_grids`): the ggml tables' shapes and magnitude
    alphabets (IQ2: 8 bytes from {8, 25, 43}; IQ3_XXS: 4 bytes from
    {4, 12, ..., 62}; IQ3_S: 4 odd bytes 1..15), entries drawn at random.
    The five arrays in the order mq_set_iq_grids takes them."""
    rng = np.random.default_rng(seed)

    def table(n, width, alphabet, dtype):
        b = rng.choice(np.array(alphabet, np.uint8), size=(n, width))
        return b.view(dtype).reshape(n)

    iq2 = [8, 25, 43]
    return (table(256, 8, iq2, np.uint64), table(512, 8, iq2, np.uint64), table(1024, 8, iq2, np.uint64),
            table(256, 4, [4, 12, 20, 28, 36, 44, 52, 62], np.uint32),
            table(512, 4, [1, 3, 5, 7, 9, 11, 13, 15], np.uint32))
