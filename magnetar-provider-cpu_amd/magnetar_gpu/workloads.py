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

from . import IQ4_XS, Q4_K, gaussian, quantize

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
