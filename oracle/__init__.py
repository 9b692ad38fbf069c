"""CPU oracle for the GGUF block-quantized matmul path.

TEST INFRASTRUCTURE ONLY. This package is the checker: ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg use it. The
product library (``magnetar-provider-cpu_amd``) never imports it.

``liboracle.so`` (built from ``oracle.c`` and ``cpu_baseline.c`` by the
Makefile here) restates, in C, the reference's
 - packed decode of Q8_0, Q4_0, IQ4_NL, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K,
   IQ4_XS and the IQ2 / IQ3 grid formats (src/native/quant.rs:46-57,
   96-279, 284-338), the grids set by the caller (`set_iq_grids`),
 - dequantization (quant.rs:1702-1711),
 - int8 activation quantizer and scalar dot (quant.rs:340-388),
 - scalar int8 / f32 column kernel (quant.rs:559-597),
 - dense f32 matmul (src/lib.rs:262-318),
 - the decoder-layer operators rmsnorm, rope, kv-write, attention, silu-mul
   and add (src/lib.rs:348-402, 427-687, 740-990, 993-1133, 2592-2596),
 - and, as the timed CPU baseline, the AVX2 Q4_K / IQ4_XS column kernels
   with the column chunking and worker pool (quant.rs:666-744, 956-984,
   1364-1433; src/native/mod.rs:110-152; src/native/pool.rs:58-155).
"""

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

Q4_0 = 2
Q8_0 = 8
Q2_K = 10
Q3_K = 11
Q4_K = 12
Q5_K = 13
Q6_K = 14
IQ4_NL = 20
IQ4_XS = 23
IQ2_XXS = 16
IQ2_XS = 17
IQ3_XXS = 18
IQ3_S = 21
IQ2_S = 22
GRID_FORMATS = (IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S)
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18, IQ4_NL: 18, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210, IQ4_XS: 136,
               IQ2_XXS: 66, IQ2_XS: 74, IQ2_S: 82, IQ3_XXS: 98, IQ3_S: 110}
BLOCK_ELEMENTS = {Q8_0: 32, Q4_0: 32, IQ4_NL: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256,
                  IQ4_XS: 256, IQ2_XXS: 256, IQ2_XS: 256, IQ2_S: 256, IQ3_XXS: 256, IQ3_S: 256}
# entries and entry dtype of each grid table, in the order set_iq_grids takes them
GRID_TABLES = ((IQ2_XXS, 256, np.uint64), (IQ2_XS, 512, np.uint64), (IQ2_S, 1024, np.uint64),
               (IQ3_XXS, 256, np.uint32), (IQ3_S, 512, np.uint32))

_lib = None


def build():
    """Compiles liboracle.so with the Makefile beside this file."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        u8p = ctypes.POINTER(ctypes.c_uint8)
        f32p = ctypes.POINTER(ctypes.c_float)
        i8p = ctypes.POINTER(ctypes.c_int8)
        i32p = ctypes.POINTER(ctypes.c_int32)
        u64 = ctypes.c_uint64
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_scale_min_k4.argtypes = [ctypes.c_int, u8p, u8p, u8p]
        L.or_iq4_xs_scales.argtypes = [u8p, i8p]
        L.or_q3_k_scales.argtypes = [u8p, i8p]
        L.or_q3_k_scales.restype = None
        L.or_decode_run.argtypes = [ctypes.c_int, u8p, ctypes.c_int, i8p, f32p, f32p]
        L.or_dequantize_rows.argtypes = [ctypes.c_int, u8p, u64, u64, f32p]
        L.or_quantize_rows.argtypes = [f32p, u64, i8p, f32p, i32p]
        L.or_int8_rounded.argtypes = [f32p, u64, f32p]
        L.or_dot_halves.argtypes = [i8p, i8p, i32p]
        L.or_columns_scalar.argtypes = [ctypes.c_int, u8p, u64, u64, f32p, u64,
                                        ctypes.c_int, u64, u64, f32p]
        L.or_matmul_dense.argtypes = [f32p, u64, u64, f32p, u64, u64,
                                      ctypes.c_int, ctypes.c_int, f32p]
        L.bl_half_f16c.restype = ctypes.c_float
        L.bl_half_f16c.argtypes = [ctypes.c_uint16]
        L.bl_packed_matmul.argtypes = [ctypes.c_int, u8p, u64, u64, f32p, u64,
                                       ctypes.c_int, f32p]
        f32 = ctypes.c_float
        L.or_rmsnorm.argtypes = [f32p, u64, u64, f32p, u64, f32, f32p]
        L.or_rope.argtypes = [f32p, u64, u64, f32, f32, u64, u64, u64, ctypes.c_int, f32p]
        L.or_kv_write.argtypes = [f32p, u64, u64, f32p, u64, u64]
        L.or_attention.argtypes = [f32p, u64, f32p, f32p, u64, u64, u64, u64, ctypes.c_int, f32, f32p, f32p]
        L.or_silu_mul.argtypes = [f32p, f32p, u64, f32p]
        L.or_silu_mul.restype = None
        L.or_add.argtypes = [f32p, u64, f32p, u64, f32p]
        u64p = ctypes.POINTER(ctypes.c_uint64)
        u32p = ctypes.POINTER(ctypes.c_uint32)
        L.or_set_iq_grids.argtypes = [u64p, u64p, u64p, u32p, u32p]
        L.or_iq_signs.restype = ctypes.c_uint8
        L.or_iq_signs.argtypes = [ctypes.c_uint32]
        _lib = L
    return _lib


def _p(a, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def f16_to_f32(bits):
    return lib().or_f16_to_f32(int(bits))


def half_f16c(bits):
    return lib().bl_half_f16c(int(bits))


def scale_min_k4(j, twelve):
    q = np.ascontiguousarray(twelve, dtype=np.uint8)
    sc = np.zeros(1, np.uint8)
    m = np.zeros(1, np.uint8)
    lib().or_scale_min_k4(j, _p(q, ctypes.c_uint8), _p(sc, ctypes.c_uint8), _p(m, ctypes.c_uint8))
    return int(sc[0]), int(m[0])


def iq4_xs_scales(six):
    b = np.ascontiguousarray(six, dtype=np.uint8)
    out = np.zeros(8, np.int8)
    lib().or_iq4_xs_scales(_p(b, ctypes.c_uint8), _p(out, ctypes.c_int8))
    return out


def q3_k_scales(twelve):
    b = np.ascontiguousarray(twelve, dtype=np.uint8)
    out = np.zeros(16, np.int8)
    lib().or_q3_k_scales(_p(b, ctypes.c_uint8), _p(out, ctypes.c_int8))
    return out


def set_iq_grids(tables):
    """The IQ2 / IQ3 grid tables the grid formats decode with: a sequence
    of five arrays in GRID_TABLES order (IQ2_XXS, IQ2_XS, IQ2_S u64;
    IQ3_XXS, IQ3_S u32)."""
    arrs = []
    for (fmt, n, dt), t in zip(GRID_TABLES, tables):
        a = np.ascontiguousarray(t, dtype=dt)
        if a.shape != (n,):
            raise ValueError(f"grid table of format {fmt} must hold {n} entries")
        arrs.append(a)
    lib().or_set_iq_grids(*(_p(a, ctypes.c_uint64 if a.dtype == np.uint64 else ctypes.c_uint32) for a in arrs))
    global _grids_keepalive
    _grids_keepalive = arrs


_grids_keepalive = None


def iq_signs(index):
    return int(lib().or_iq_signs(int(index)))


def decode_run(fmt, block, run):
    b = np.ascontiguousarray(block, dtype=np.uint8)
    q = np.zeros(32, np.int8)
    scale = np.zeros(2, np.float32)
    mn = np.zeros(2, np.float32)
    lib().or_decode_run(fmt, _p(b, ctypes.c_uint8), run, _p(q, ctypes.c_int8),
                        _p(scale, ctypes.c_float), _p(mn, ctypes.c_float))
    return q, scale, mn


def dequantize(fmt, data, rows, cols):
    """Stored rows x cols f32 (the stored layout, `dequantize_stored`)."""
    b = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty((rows, cols), np.float32)
    rc = lib().or_dequantize_rows(fmt, _p(b, ctypes.c_uint8), rows, cols, _p(out, ctypes.c_float))
    if rc:
        raise ValueError("oracle dequantize: unsupported format or shape")
    return out


def quantize_rows(x):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    n = x.size
    values = np.empty(n, np.int8)
    scales = np.empty(n // 32, np.float32)
    sums = np.empty((n // 32, 2), np.int32)
    lib().or_quantize_rows(_p(x, ctypes.c_float), n, _p(values, ctypes.c_int8),
                           _p(scales, ctypes.c_float), _p(sums, ctypes.c_int32))
    return values, scales, sums


def int8_rounded(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().or_int8_rounded(_p(x, ctypes.c_float), x.size, _p(out, ctypes.c_float))
    return out


def dot_halves(q, a):
    q = np.ascontiguousarray(q, dtype=np.int8)
    a = np.ascontiguousarray(a, dtype=np.int8)
    out = np.zeros(2, np.int32)
    lib().or_dot_halves(_p(q, ctypes.c_int8), _p(a, ctypes.c_int8), _p(out, ctypes.c_int32))
    return out


def columns_scalar(fmt, data, n, k, x, int8, first=0, count=None):
    """The scalar column kernel over columns first..first+count: [m, count]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = x.shape[0]
    count = n - first if count is None else count
    b = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty((m, count), np.float32)
    rc = lib().or_columns_scalar(fmt, _p(b, ctypes.c_uint8), n, k, _p(x, ctypes.c_float), m,
                                 1 if int8 else 0, first, count, _p(out, ctypes.c_float))
    if rc:
        raise ValueError("oracle columns: bad arguments")
    return out


def matmul_dense(a, b, transpose_a=False, transpose_b=False):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    m = a.shape[1] if transpose_a else a.shape[0]
    n = b.shape[0] if transpose_b else b.shape[1]
    out = np.empty((m, n), np.float32)
    rc = lib().or_matmul_dense(_p(a, ctypes.c_float), a.shape[0], a.shape[1],
                               _p(b, ctypes.c_float), b.shape[0], b.shape[1],
                               int(transpose_a), int(transpose_b), _p(out, ctypes.c_float))
    if rc:
        raise ValueError("matmul inner dimension mismatch")
    return out


def baseline_packed_matmul(fmt, data, n, k, x, threads):
    """The AVX2 CPU path with `threads` pool threads: [m, n]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty((x.shape[0], n), np.float32)
    rc = lib().bl_packed_matmul(fmt, _p(b, ctypes.c_uint8), n, k, _p(x, ctypes.c_float),
                                x.shape[0], threads, _p(out, ctypes.c_float))
    if rc:
        raise RuntimeError(f"baseline packed matmul failed ({rc})")
    return out


# ---- decoder-layer operators ----------------------------------------------------

def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def rmsnorm(x, w, epsilon):
    """`rmsnorm` (src/lib.rs:348-402): x [rows, cols], w [cols] or [rows, cols]."""
    x, w = _f32(x), _f32(w)
    cols = x.shape[-1]
    rows = x.size // cols
    out = np.empty_like(x)
    rc = lib().or_rmsnorm(_p(x, ctypes.c_float), rows, cols, _p(w, ctypes.c_float), w.size // cols,
                          float(epsilon), _p(out, ctypes.c_float))
    if rc:
        raise ValueError("rmsnorm: unsupported shape or epsilon")
    return out


def rope(x, base, scale, dimension, position_offset, head_count, half_split=False):
    """`rope` with unscaled frequencies (src/lib.rs:427-447, 616-687)."""
    x = _f32(x)
    rows, cols = x.shape
    out = np.empty_like(x)
    rc = lib().or_rope(_p(x, ctypes.c_float), rows, cols, float(base), float(scale), dimension, position_offset,
                       head_count, int(half_split), _p(out, ctypes.c_float))
    if rc:
        raise ValueError("rope: unsupported arguments")
    return out


def kv_write(store, rows, row_offset):
    """`kv-write` in place (src/lib.rs:740-768); returns the store."""
    assert store.dtype == np.float32 and store.flags.c_contiguous
    rows = _f32(rows)
    capacity, width = store.shape
    rc = lib().or_kv_write(_p(store, ctypes.c_float), capacity, width, _p(rows, ctypes.c_float), rows.shape[0],
                           row_offset)
    if rc:
        raise ValueError("kv-write exceeds the store")
    return store


def attention(q, k, v, head_count, head_dimension, kv_head_count, causal=True, scale=None):
    """`attention` (src/lib.rs:780-990): q [seq, heads*dim], k/v [kv_seq, kv_heads*dim]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    seq, kv_seq = q.shape[0], k.shape[0]
    out = np.empty_like(q)
    scores = np.empty(kv_seq, np.float32)
    rc = lib().or_attention(_p(q, ctypes.c_float), seq, _p(k, ctypes.c_float), _p(v, ctypes.c_float), kv_seq,
                            head_count, head_dimension, kv_head_count, int(causal),
                            float("nan") if scale is None else float(scale), _p(scores, ctypes.c_float),
                            _p(out, ctypes.c_float))
    if rc:
        raise ValueError("attention: unsupported shape")
    return out


def silu_mul(gate, up):
    """`silu-mul` (src/lib.rs:2592-2596)."""
    gate, up = _f32(gate), _f32(up)
    out = np.empty_like(gate)
    lib().or_silu_mul(_p(gate, ctypes.c_float), _p(up, ctypes.c_float), gate.size, _p(out, ctypes.c_float))
    return out


def add(a, b):
    """`add` / `residual-add` (src/lib.rs:1019-1075, 1128-1133)."""
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    rc = lib().or_add(_p(a, ctypes.c_float), a.size, _p(b, ctypes.c_float), b.size, _p(out, ctypes.c_float))
    if rc:
        raise ValueError("add: shapes do not broadcast")
    return out
