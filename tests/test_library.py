"""CPU-side checks of the product libraries: they load without a GPU, export
every symbol their headers declare, and the host encoders and generator
behave. No GPU compute is called here."""

import ctypes
import hashlib
import os
import re

import numpy as np
import pytest

import magnetar_gpu as mg
import oracle
from helpers import IQ4_XS, Q4_K

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:mq|gg|mg)_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("header,lib", [
    ("magnetar_gpu.h", mg.GPU_LIB),
    ("magnetar_gguf.h", mg.GGUF_LIB),
    ("magnetar_executor.h", mg.EXECUTOR_LIB),
])
def test_library_exports_every_declared_symbol(header, lib):
    names = _declared(header)
    assert names, header
    handle = ctypes.CDLL(lib)
    missing = [n for n in names if not hasattr(handle, n)]
    assert not missing, f"{os.path.basename(lib)} lacks {missing}"


def test_gpu_library_reports_version_without_a_gpu():
    assert b"gfx950" in mg.gpu_lib().mq_version()


def test_f16_round_trip_matches_numpy():
    rng = np.random.default_rng(0)
    vals = np.concatenate([rng.standard_normal(2000) * 10.0 ** rng.integers(-9, 5, 2000),
                           [0.0, -0.0, 65504.0, 65520.0, 1e-8, 6e-8, 3e-8]]).astype(np.float32)
    L = mg.gguf_lib()
    for v in vals:
        assert L.gg_f32_to_f16(float(v)) == int(np.array([v], np.float32).astype(np.float16).view(np.uint16)[0]), v
    for bits in range(0, 65536, 7):
        h = np.array([bits], np.uint16).view(np.float16)[0]
        if not np.isnan(h):
            assert L.gg_f16_to_f32(bits) == np.float32(h)


def test_gaussian_generator_is_deterministic_and_normal():
    a = mg.gaussian(1, 0.02, 200001)
    b = mg.gaussian(1, 0.02, 200001)
    np.testing.assert_array_equal(a, b)
    assert abs(float(a.mean())) < 3e-4
    assert abs(float(a.std()) - 0.02) < 3e-4
    assert not np.array_equal(a[:1000], mg.gaussian(2, 0.02, 1000))


@pytest.mark.parametrize("fmt", [Q4_K, IQ4_XS])
def test_encoder_round_trip_error_is_small(fmt):
    """Encode N(0, 0.02) weights, decode with the oracle: the reconstruction
    error is a small fraction of the weights' spread and the encoder uses
    the formats' full structure (nonzero mins for Q4_K, signed scales)."""
    w = mg.gaussian(5, 0.02, 64 * 1024).reshape(64, 1024)
    enc = mg.quantize(fmt, w)
    assert enc.shape == (64, 1024 // 256 * (144 if fmt == Q4_K else 136))
    dec = oracle.dequantize(fmt, enc, 64, 1024)
    rms = float(np.sqrt(np.mean((dec - w) ** 2)))
    assert rms < 0.004, rms
    if fmt == Q4_K:
        assert np.any(enc.reshape(-1, 144)[:, 2:4])  # dmin != 0
        scales = enc.reshape(-1, 144)[:, 4:16]
        assert len(np.unique(scales)) > 100          # all scale bit positions used


BASELINE_SHA256 = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "workload_sha256.json")


def test_workload_weights_hash_matches_fixture():
    """The full-size workload weights are regenerated, not stored: their
    encoded bytes must hash to the committed values."""
    import json

    from magnetar_gpu import workloads

    expected = json.load(open(BASELINE_SHA256))
    for name, digest in expected.items():
        spec = workloads.WEIGHTS[name]
        data = workloads.weight_bytes(name)
        assert hashlib.sha256(data.tobytes()).hexdigest() == digest, (name, spec)
