"""ctypes binding of the gfx950 packed-weight matmul library.

``libmagnetar_gpu.so`` (C ABI in ``include/magnetar_gpu.h``) is the product:
packed-weight upload, the int8-activation decode GEMV, the MFMA prefill
GEMM and the bit-exact dequantizer. ``libmagnetar_gguf.so``
(``include/magnetar_gguf.h``) holds host-side GGUF encoders and the seeded
Gaussian generator. Loading fails loudly when a library is missing: there
is no CPU fallback anywhere in this package.
"""

import ctypes
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GPU_LIB = os.path.join(PKG_DIR, "libmagnetar_gpu.so")
GGUF_LIB = os.path.join(PKG_DIR, "libmagnetar_gguf.so")
EXECUTOR_LIB = os.path.join(PKG_DIR, "libmagnetar_executor.so")
PROBE_LIB = os.path.join(PKG_DIR, "libmagnetar_probe.so")

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
BLOCK_VALUES = {Q8_0: 32, Q4_0: 32, IQ4_NL: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256,
                IQ4_XS: 256, IQ2_XXS: 256, IQ2_XS: 256, IQ2_S: 256, IQ3_XXS: 256, IQ3_S: 256}
FORMAT_NAMES = {Q8_0: "Q8_0", Q4_0: "Q4_0", IQ4_NL: "IQ4_NL", Q2_K: "Q2_K", Q3_K: "Q3_K", Q4_K: "Q4_K",
                Q5_K: "Q5_K", Q6_K: "Q6_K", IQ4_XS: "IQ4_XS", IQ2_XXS: "IQ2_XXS", IQ2_XS: "IQ2_XS", IQ2_S: "IQ2_S",
                IQ3_XXS: "IQ3_XXS", IQ3_S: "IQ3_S"}
# the grid tables mq_set_iq_grids takes, in order: (entries, dtype)
GRID_TABLES = ((256, np.uint64), (512, np.uint64), (1024, np.uint64), (256, np.uint32), (512, np.uint32))

OK = 0
ERR_SHAPE = 1
ERR_DTYPE = 2
DECLINED = 3
ERR_HIP = 4
ERR_OOM = 5
ERR_ARGUMENT = 6
INT8_ACTIVATIONS = 1
TRANSPOSE_B = 2
EPILOGUE_NONE = 0
EPILOGUE_ROPE_KV = 1
EPILOGUE_SILU_PAIRS = 2


class GemvShape(ctypes.Structure):
    """mq_gemv_shape (include/magnetar_gpu.h)."""
    _fields_ = [("form", ctypes.c_uint32), ("waves", ctypes.c_uint32), ("grid_x", ctypes.c_uint32),
                ("grid_y", ctypes.c_uint32), ("lds_bytes", ctypes.c_uint64)]


GEMV_FORM_LANES8, GEMV_FORM_ROWS, GEMV_FORM_LDS, GEMV_FORM_NARROW, GEMV_FORM_WAVE = 1, 2, 3, 4, 5


class DecodeFusion(ctypes.Structure):
    """mq_decode_fusion (include/magnetar_gpu.h)."""
    _fields_ = [("norm_weight", ctypes.c_void_p), ("norm_epsilon", ctypes.c_float), ("epilogue", ctypes.c_uint32),
                ("rope_rows", ctypes.c_uint64), ("rope_dim", ctypes.c_uint64), ("rope_offset", ctypes.c_uint64),
                ("rope_base", ctypes.c_float), ("rope_scale", ctypes.c_float),
                ("seg_begin", ctypes.c_uint64 * 3), ("seg_out", ctypes.c_void_p * 3)]

_u8p = ctypes.POINTER(ctypes.c_uint8)
_f32p = ctypes.POINTER(ctypes.c_float)
_i8p = ctypes.POINTER(ctypes.c_int8)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u64 = ctypes.c_uint64
_vp = ctypes.c_void_p

_gpu = None
_gguf = None
_probe = None


class GpuError(RuntimeError):
    def __init__(self, code, reason):
        super().__init__(f"[{code}] {reason}")
        self.code = code
        self.reason = reason


class Declined(GpuError):
    """PackedWeightWrite::Declined: the caller keeps the f32 path."""


def _load(path):
    if not os.path.exists(path):
        raise ImportError(f"{path} is not built: run `make -C {PKG_DIR}` (or __graft_entry__.build())")
    return ctypes.CDLL(path)


def gpu_lib():
    global _gpu
    if _gpu is None:
        L = _load(GPU_LIB)
        L.mq_create.argtypes = [ctypes.c_int, ctypes.POINTER(_vp)]
        L.mq_destroy.argtypes = [_vp]
        L.mq_destroy.restype = None
        L.mq_last_error.argtypes = [_vp]
        L.mq_last_error.restype = ctypes.c_char_p
        L.mq_version.restype = ctypes.c_char_p
        L.mq_gemv_launch_shape.argtypes = [ctypes.c_uint32, _u64, _u64, _u64, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_int, ctypes.POINTER(GemvShape)]
        L.mq_weight_upload.argtypes = [_vp, ctypes.c_uint32, _u64, _u64, ctypes.c_int, _u8p,
                                       ctypes.c_size_t, ctypes.POINTER(_u64)]
        L.mq_weight_release.argtypes = [_vp, _u64]
        L.mq_set_iq_grids.argtypes = [_vp, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64),
                                      ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint32),
                                      ctypes.POINTER(ctypes.c_uint32)]
        L.mq_weight_info.argtypes = [_vp, _u64, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(_u64),
                                     ctypes.POINTER(_u64), ctypes.POINTER(ctypes.c_int), ctypes.POINTER(_u64)]
        L.mq_matmul.argtypes = [_vp, _u64, _f32p, _u64, _u64, ctypes.c_uint32, _f32p]
        L.mq_matmul_dev.argtypes = [_vp, _u64, _vp, _u64, _u64, ctypes.c_uint32, _vp, _vp]
        L.mq_matmul_noalloc_dev.argtypes = [_vp, _u64, _vp, _u64, _u64, ctypes.c_uint32, _vp, _vp]
        L.mq_quantize_activations_dev.argtypes = [_vp, _vp, _u64, _u64, _vp, _vp, _vp, _vp]
        L.mq_matmul_prequantized_dev.argtypes = [_vp, _u64, _vp, _vp, _vp, _u64, _u64, _vp, _vp]
        L.mq_prepare_activations_f16_dev.argtypes = [_vp, _vp, _u64, _u64, ctypes.c_uint32, _vp, _vp]
        L.mq_matmul_f16_dev.argtypes = [_vp, _u64, _vp, _u64, _u64, _vp, _vp]
        L.mq_dequantize.argtypes = [_vp, _u64, ctypes.c_int, _f32p]
        L.mq_dequantize_dev.argtypes = [_vp, _u64, ctypes.c_int, _vp, _vp]
        L.mq_embedding.argtypes = [_vp, _u64, _f32p, _u64, ctypes.c_float, _f32p]
        L.mq_decode_matmul_dev.argtypes = [_vp, _u64, _vp, _u64, ctypes.POINTER(DecodeFusion), _vp, _vp]
        L.mq_embedding_dev.argtypes = [_vp, _u64, _f32p, _u64, ctypes.c_float, _vp, _vp]
        L.mq_matmul_add_dev.argtypes = [_vp, _u64, _vp, _u64, _u64, ctypes.c_uint32, _vp, _u64, _vp, _vp]
        f32 = ctypes.c_float
        L.mq_rmsnorm_dev.argtypes = [_vp, _vp, _u64, _u64, _vp, _u64, f32, _vp, _vp]
        L.mq_rope_dev.argtypes = [_vp, _vp, _u64, _u64, f32, f32, _u64, _u64, _u64, ctypes.c_int, _vp, _vp]
        L.mq_kv_write_dev.argtypes = [_vp, _vp, _u64, _u64, _vp, _u64, _u64, _vp]
        L.mq_attention_dev.argtypes = [_vp, _vp, _u64, _vp, _vp, _u64, _u64, _u64, _u64, _u64, ctypes.c_int, f32,
                                       _vp, _vp]
        L.mq_silu_mul_dev.argtypes = [_vp, _vp, _vp, _u64, _vp, _vp]
        L.mq_add_dev.argtypes = [_vp, _vp, _u64, _vp, _u64, _vp, _vp]
        _gpu = L
    return _gpu


def gguf_lib():
    global _gguf
    if _gguf is None:
        L = _load(GGUF_LIB)
        L.gg_f32_to_f16.argtypes = [ctypes.c_float]
        L.gg_f32_to_f16.restype = ctypes.c_uint16
        L.gg_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.gg_f16_to_f32.restype = ctypes.c_float
        L.gg_gaussian_f32.argtypes = [_u64, ctypes.c_float, _f32p, _u64]
        L.gg_gaussian_f32.restype = None
        L.gg_row_bytes.argtypes = [ctypes.c_uint32, _u64]
        L.gg_row_bytes.restype = _u64
        L.gg_quantize.argtypes = [ctypes.c_uint32, _f32p, _u64, _u64, _u8p]
        _gguf = L
    return _gguf


def gemv_launch_shape(gguf_type, rows, cols, m, waves=0, variant=0, ksplit=0):
    """The launch the pre-quantized decode GEMV takes (mq_gemv_launch_shape),
    computed on the host: a GemvShape."""
    out = GemvShape()
    rc = gpu_lib().mq_gemv_launch_shape(gguf_type, rows, cols, m, waves, variant, ksplit, ctypes.byref(out))
    if rc:
        raise GpuError(rc, gpu_lib().mq_last_error(None).decode())
    return out


def probe_lib():
    """The streaming-read probe (libmagnetar_probe.so), a measurement aid of
    the benchmark: mqp_stream_read reads a device buffer once, nothing else."""
    global _probe
    if _probe is None:
        L = _load(PROBE_LIB)
        L.mqp_stream_read.argtypes = [_vp, _u64, ctypes.c_int, ctypes.c_int, _vp, _vp]
        L.mqp_stream_groups.argtypes = [_u64, ctypes.c_int, ctypes.c_int]
        L.mqp_stream_groups.restype = _u64
        _probe = L
    return _probe


def _p(a, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


# ---- host GGUF helpers -----------------------------------------------------

def gaussian(seed, sigma, n):
    out = np.empty(n, np.float32)
    gguf_lib().gg_gaussian_f32(seed, sigma, _p(out, ctypes.c_float), n)
    return out


def row_bytes(gguf_type, cols):
    return int(gguf_lib().gg_row_bytes(gguf_type, cols))


def quantize(gguf_type, w):
    """Encodes f32 weights [rows, cols] into GGUF blocks (uint8 [rows, row_bytes])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    rb = row_bytes(gguf_type, cols)
    if rb == 0:
        raise ValueError(f"type {gguf_type} cannot encode {cols} columns")
    out = np.empty((rows, rb), np.uint8)
    if gguf_lib().gg_quantize(gguf_type, _p(w, ctypes.c_float), rows, cols, _p(out, ctypes.c_uint8)):
        raise ValueError("gg_quantize failed")
    return out


# ---- device context --------------------------------------------------------

class Weight:
    def __init__(self, ctx, handle, gguf_type, rows, cols, transposed):
        self.ctx = ctx
        self.handle = handle
        self.gguf_type = gguf_type
        self.stored_rows = rows
        self.stored_cols = cols
        self.transposed = transposed

    @property
    def logical_shape(self):
        return (self.stored_cols, self.stored_rows) if self.transposed else (self.stored_rows, self.stored_cols)

    def release(self):
        if self.handle:
            self.ctx._check(gpu_lib().mq_weight_release(self.ctx.ptr, self.handle))
            self.handle = 0


class Context:
    """One device context (mq_ctx): a stream, a workspace, uploaded weights."""

    def __init__(self, device=0):
        L = gpu_lib()
        ptr = _vp()
        rc = L.mq_create(device, ctypes.byref(ptr))
        if rc:
            raise GpuError(rc, L.mq_last_error(None).decode())
        self.ptr = ptr

    def close(self):
        if self.ptr:
            gpu_lib().mq_destroy(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def last_error(self):
        return gpu_lib().mq_last_error(self.ptr).decode()

    def _check(self, rc):
        if rc == DECLINED:
            raise Declined(rc, self.last_error())
        if rc:
            raise GpuError(rc, self.last_error())

    def set_iq_grids(self, tables):
        """The IQ2 / IQ3 grid tables (five arrays in GRID_TABLES order:
        IQ2_XXS, IQ2_XS, IQ2_S u64; IQ3_XXS, IQ3_S u32) for this context's
        device (mq_set_iq_grids)."""
        arrs = []
        for (n, dt), t in zip(GRID_TABLES, tables):
            a = np.ascontiguousarray(t, dtype=dt)
            if a.shape != (n,):
                raise ValueError(f"grid table needs {n} entries, got {a.shape}")
            arrs.append(a)
        if len(arrs) != 5:
            raise ValueError("five grid tables")
        ptrs = [_p(a, ctypes.c_uint64 if a.dtype == np.uint64 else ctypes.c_uint32) for a in arrs]
        self._check(gpu_lib().mq_set_iq_grids(self.ptr, *ptrs))

    def upload(self, gguf_type, rows, cols, data, transposed=True):
        b = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
        h = _u64()
        self._check(gpu_lib().mq_weight_upload(self.ptr, gguf_type, rows, cols, int(transposed),
                                               _p(b, ctypes.c_uint8), b.size, ctypes.byref(h)))
        return Weight(self, h.value, gguf_type, rows, cols, transposed)

    def info(self, weight):
        t = ctypes.c_uint32()
        r, c, nbytes = _u64(), _u64(), _u64()
        tr = ctypes.c_int()
        self._check(gpu_lib().mq_weight_info(self.ptr, weight.handle, ctypes.byref(t), ctypes.byref(r),
                                             ctypes.byref(c), ctypes.byref(tr), ctypes.byref(nbytes)))
        return {"type": t.value, "stored_rows": r.value, "stored_cols": c.value,
                "transposed": tr.value, "device_bytes": nbytes.value}

    def matmul(self, weight, x, int8=True, transpose_b=False):
        """x . W on host arrays (synchronous), W the logical weight read as
        the reference reads it: the stored rows are the outputs when
        weight.transposed != transpose_b, else the input rows (axpy)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim != 2:
            raise ValueError("x must be [m, k]")
        m, k = x.shape
        n = weight.stored_rows if bool(weight.transposed) != bool(transpose_b) else weight.stored_cols
        y = np.empty((m, n), np.float32)
        flags = (INT8_ACTIVATIONS if int8 else 0) | (TRANSPOSE_B if transpose_b else 0)
        self._check(gpu_lib().mq_matmul(self.ptr, weight.handle, _p(x, ctypes.c_float), m, k, flags,
                                        _p(y, ctypes.c_float)))
        return y

    def matmul_dev(self, weight, x_ptr, m, k, y_ptr, int8=True, stream=None, transpose_b=False):
        flags = (INT8_ACTIVATIONS if int8 else 0) | (TRANSPOSE_B if transpose_b else 0)
        self._check(gpu_lib().mq_matmul_dev(self.ptr, weight.handle, x_ptr, m, k, flags, y_ptr, stream))

    def decode_matmul_dev(self, weight, x_ptr, k, y_ptr=None, norm_weight_ptr=None, norm_epsilon=0.0,
                          epilogue=EPILOGUE_NONE, rope_rows=0, rope_dim=2, rope_offset=0, rope_base=1.0,
                          rope_scale=1.0, segments=(), stream=None):
        """One decode row through mq_decode_matmul_dev. segments: up to three
        (first row, device pointer) pairs for EPILOGUE_ROPE_KV."""
        f = DecodeFusion()
        f.norm_weight = norm_weight_ptr
        f.norm_epsilon = norm_epsilon
        f.epilogue = epilogue
        f.rope_rows, f.rope_dim, f.rope_offset = rope_rows, rope_dim, rope_offset
        f.rope_base, f.rope_scale = rope_base, rope_scale
        segs = list(segments) + [(weight.stored_rows, None)] * (3 - len(segments))
        for i, (begin, ptr) in enumerate(segs):
            f.seg_begin[i] = begin
            f.seg_out[i] = ptr
        self._check(gpu_lib().mq_decode_matmul_dev(self.ptr, weight.handle, x_ptr, k, ctypes.byref(f), y_ptr,
                                                   stream))

    def embedding(self, weight, ids, scale=None):
        """The `embedding` Kernel on a packed table: [len(ids), dim]."""
        ids = np.ascontiguousarray(ids, dtype=np.float32).reshape(-1)
        dim = weight.logical_shape[1]
        out = np.empty((ids.size, dim), np.float32)
        self._check(gpu_lib().mq_embedding(self.ptr, weight.handle, _p(ids, ctypes.c_float), ids.size,
                                           float("nan") if scale is None else float(scale),
                                           _p(out, ctypes.c_float)))
        return out

    def embedding_dev(self, weight, ids, out_ptr, scale=None, stream=None):
        ids = np.ascontiguousarray(ids, dtype=np.float32).reshape(-1)
        self._check(gpu_lib().mq_embedding_dev(self.ptr, weight.handle, _p(ids, ctypes.c_float), ids.size,
                                               float("nan") if scale is None else float(scale), out_ptr, stream))

    def quantize_activations_dev(self, x_ptr, m, k, values_ptr, scales_ptr, sums_ptr, stream=None):
        self._check(gpu_lib().mq_quantize_activations_dev(self.ptr, x_ptr, m, k, values_ptr, scales_ptr,
                                                          sums_ptr, stream))

    def matmul_prequantized_dev(self, weight, values_ptr, scales_ptr, sums_ptr, m, k, y_ptr, stream=None):
        self._check(gpu_lib().mq_matmul_prequantized_dev(self.ptr, weight.handle, values_ptr, scales_ptr,
                                                         sums_ptr, m, k, y_ptr, stream))

    def prepare_activations_f16_dev(self, x_ptr, m, k, a16_ptr, int8=True, stream=None):
        self._check(gpu_lib().mq_prepare_activations_f16_dev(self.ptr, x_ptr, m, k,
                                                             INT8_ACTIVATIONS if int8 else 0, a16_ptr, stream))

    def matmul_f16_dev(self, weight, a16_ptr, m, k, y_ptr, stream=None):
        self._check(gpu_lib().mq_matmul_f16_dev(self.ptr, weight.handle, a16_ptr, m, k, y_ptr, stream))

    def dequantize(self, weight, logical=False):
        shape = weight.logical_shape if logical else (weight.stored_rows, weight.stored_cols)
        out = np.empty(shape, np.float32)
        self._check(gpu_lib().mq_dequantize(self.ptr, weight.handle, int(logical), _p(out, ctypes.c_float)))
        return out

    def dequantize_dev(self, weight, out_ptr, logical=False, stream=None):
        self._check(gpu_lib().mq_dequantize_dev(self.ptr, weight.handle, int(logical), out_ptr, stream))

    def matmul_add_dev(self, weight, x_ptr, m, k, addend_ptr, addend_rows, y_ptr, int8=True, stream=None):
        """y = x . W^T + addend (addend_rows 1: a bias row; m: a residual)."""
        self._check(gpu_lib().mq_matmul_add_dev(self.ptr, weight.handle, x_ptr, m, k,
                                                INT8_ACTIVATIONS if int8 else 0, addend_ptr, addend_rows, y_ptr,
                                                stream))

    # ---- decoder-layer operators (device pointers) ----------------------------

    def rmsnorm_dev(self, x_ptr, rows, cols, w_ptr, w_rows, epsilon, out_ptr, stream=None):
        self._check(gpu_lib().mq_rmsnorm_dev(self.ptr, x_ptr, rows, cols, w_ptr, w_rows, epsilon, out_ptr, stream))

    def rope_dev(self, x_ptr, rows, cols, base, scale, dimension, position_offset, head_count, out_ptr,
                 half_split=False, stream=None):
        self._check(gpu_lib().mq_rope_dev(self.ptr, x_ptr, rows, cols, base, scale, dimension, position_offset,
                                          head_count, 1 if half_split else 0, out_ptr, stream))

    def kv_write_dev(self, store_ptr, capacity, width, rows_ptr, count, row_offset, stream=None):
        self._check(gpu_lib().mq_kv_write_dev(self.ptr, store_ptr, capacity, width, rows_ptr, count, row_offset,
                                              stream))

    def attention_dev(self, q_ptr, seq, k_ptr, v_ptr, kv_rows, key_count, heads, head_dim, kv_heads, out_ptr,
                      causal=True, scale=None, stream=None):
        self._check(gpu_lib().mq_attention_dev(self.ptr, q_ptr, seq, k_ptr, v_ptr, kv_rows, key_count, heads,
                                               head_dim, kv_heads, 1 if causal else 0,
                                               float("nan") if scale is None else float(scale), out_ptr, stream))

    def silu_mul_dev(self, gate_ptr, up_ptr, n, out_ptr, stream=None):
        self._check(gpu_lib().mq_silu_mul_dev(self.ptr, gate_ptr, up_ptr, n, out_ptr, stream))

    def add_dev(self, a_ptr, n, b_ptr, b_n, out_ptr, stream=None):
        self._check(gpu_lib().mq_add_dev(self.ptr, a_ptr, n, b_ptr, b_n, out_ptr, stream))
