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


@pytest.mark.parametrize("fmt", [Q4_K, IQ4_XS])
@pytest.mark.parametrize("variant", [0, 1, 2, 3])
@pytest.mark.parametrize("m", [1, 4, 8])
def test_gemv_wave_override_clamps_to_the_launch_bound(fmt, variant, m):
    """A 16-wave override (MQ_GEMV_SPLITS=16) never launches more than the
    512 threads every GEMV kernel is built for (__launch_bounds__(512), 8
    reduction slots): the launch that once faulted with 1024 threads."""
    for rows, cols in ((14336, 4096), (4096, 14336), (64, 256), (1000, 512)):
        for ksplit in (0, 1, 4, 16):
            g = mg.gemv_launch_shape(fmt, rows, cols, m, waves=16, variant=variant, ksplit=ksplit)
            assert 1 <= g.waves <= 8, (rows, cols, ksplit, g.form, g.waves)
            assert g.form != mg.GEMV_FORM_WAVE  # an override keeps the forms it sweeps
            assert g.lds_bytes <= 65536
            if variant in (1, 2):
                assert g.form in (mg.GEMV_FORM_LANES8, mg.GEMV_FORM_ROWS)
            if g.form == mg.GEMV_FORM_ROWS:
                assert m <= 4 and g.grid_x == -(-rows // 64)
            if g.form == mg.GEMV_FORM_LANES8:
                assert g.grid_x == -(-rows // 8)


def test_gemv_default_launch_shapes():
    """The defaults the measured shapes take: one super-block per wave for
    the 14336 x 4096 up projection at every m <= 8 (224 work-groups of 16
    waves, no K split; with a waves override the two-blocks-per-wave LDS
    form), the 16-row form for the 4096 x 14336 down projection (256
    work-groups)."""
    g = mg.gemv_launch_shape(Q4_K, 14336, 4096, 1)
    assert (g.form, g.grid_x, g.grid_y, g.waves) == (mg.GEMV_FORM_WAVE, 224, 1, 16)
    assert g.lds_bytes <= 65536
    g = mg.gemv_launch_shape(Q4_K, 14336, 4096, 4)
    assert (g.form, g.waves) == (mg.GEMV_FORM_WAVE, 16)
    g = mg.gemv_launch_shape(Q4_K, 14336, 4096, 1, waves=8)
    assert (g.form, g.grid_x, g.grid_y, g.waves) == (mg.GEMV_FORM_LDS, 224, 1, 8)
    g = mg.gemv_launch_shape(Q4_K, 14336, 4096, 8)
    assert (g.form, g.waves) == (mg.GEMV_FORM_WAVE, 16)
    assert g.lds_bytes <= 65536
    g = mg.gemv_launch_shape(IQ4_XS, 4096, 14336, 1)
    assert (g.form, g.grid_x, g.grid_y, g.waves) == (mg.GEMV_FORM_NARROW, 256, 1, 8)
    with pytest.raises(mg.GpuError):
        mg.gemv_launch_shape(Q4_K, 14336, 4096, 9)
