"""ctypes binding of libmagnetar_executor.so (include/magnetar_executor.h):
the Provider side of the GPU path, with device-resident tensors."""

import ctypes
import json

import numpy as np

from . import EXECUTOR_LIB, _load

OK = 0
KERNEL_EXECUTION_FAILED = 1
KERNEL_DTYPE_UNSUPPORTED = 2
KERNEL_ATTRIBUTE_UNSUPPORTED = 3
KERNEL_NOT_FOUND = 4
KERNEL_TIMEOUT = 5
MEMORY_DENIED = 6
UNKNOWN = 7
ERR_ARGUMENT = 8
ERR_DEVICE = 9
ERR_OOM = 10
KV_F32 = 0

_lib = None


class Attribute(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("value", ctypes.c_char_p)]


def lib():
    global _lib
    if _lib is None:
        L = _load(EXECUTOR_LIB)
        vp, u64 = ctypes.c_void_p, ctypes.c_uint64
        L.mg_executor_create.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, u64, ctypes.POINTER(vp)]
        L.mg_executor_destroy.argtypes = [vp]
        L.mg_executor_destroy.restype = None
        L.mg_executor_last_error.argtypes = [vp]
        L.mg_executor_last_error.restype = ctypes.c_char_p
        L.mg_write_packed_weight_tensor.argtypes = [vp, ctypes.c_char_p, ctypes.c_uint32, u64, u64, ctypes.c_int,
                                                    ctypes.POINTER(ctypes.c_uint8), ctypes.c_size_t,
                                                    ctypes.POINTER(ctypes.c_int)]
        L.mg_write_tensor.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(u64), ctypes.c_uint32,
                                      ctypes.POINTER(ctypes.c_float)]
        L.mg_write_tensor_admitted.argtypes = L.mg_write_tensor.argtypes
        L.mg_resident_shape.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(u64), ctypes.POINTER(ctypes.c_uint32)]
        L.mg_read_tensor.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float), u64]
        L.mg_is_packed.argtypes = [vp, ctypes.c_char_p]
        L.mg_read_tensor_value_is_opaque.argtypes = [vp, ctypes.c_char_p]
        L.mg_release_tensor.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int)]
        L.mg_submit_kernel.argtypes = [vp, ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p),
                                       ctypes.c_uint32, ctypes.c_char_p, ctypes.POINTER(Attribute), ctypes.c_uint32,
                                       ctypes.c_int64, ctypes.c_char_p, ctypes.c_size_t]
        L.mg_complete_kernel.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int), ctypes.c_char_p,
                                         ctypes.c_size_t]
        L.mg_observation_count.argtypes = [vp]
        L.mg_observation_count.restype = u64
        L.mg_observation.argtypes = [vp, u64, ctypes.c_char_p, ctypes.c_size_t, ctypes.c_char_p, ctypes.c_size_t]
        L.mg_kernel_advertisement_count.restype = ctypes.c_uint32
        L.mg_kernel_advertisement_json.argtypes = [ctypes.c_uint32]
        L.mg_kernel_advertisement_json.restype = ctypes.c_char_p
        L.mg_materialization_count.argtypes = [vp]
        L.mg_materialization_count.restype = u64
        L.mg_memory_used.argtypes = [vp]
        L.mg_memory_used.restype = u64
        L.mg_write_tensor_value.argtypes = [vp, ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(u64), ctypes.c_uint32,
                                            ctypes.POINTER(ctypes.c_float)]
        L.mg_write_tensor_value_admitted.argtypes = L.mg_write_tensor_value.argtypes
        L.mg_copy_tensor_admitted.argtypes = [vp, ctypes.c_char_p, ctypes.c_char_p]
        L.mg_write_zeroed_kv_store.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(u64), ctypes.c_uint32,
                                               ctypes.c_uint32, u64, u64, ctypes.POINTER(ctypes.c_int)]
        L.mg_allocate_workspace.argtypes = [vp, u64, ctypes.c_char_p, ctypes.c_size_t]
        L.mg_release_workspace.argtypes = [vp, ctypes.c_char_p]
        L.mg_release_admitted_tensor.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int)]
        L.mg_synchronize.argtypes = [vp]
        L.mg_profile_count.argtypes = [vp]
        L.mg_profile_count.restype = ctypes.c_uint32
        L.mg_profile_entry.argtypes = [vp, ctypes.c_uint32, ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(u64),
                                       ctypes.POINTER(ctypes.c_double)]
        _lib = L
    return _lib


def kernel_advertisements():
    L = lib()
    return [json.loads(L.mg_kernel_advertisement_json(i)) for i in range(L.mg_kernel_advertisement_count())]


class ExecutorError(RuntimeError):
    def __init__(self, code, reason):
        super().__init__(f"[{code}] {reason}")
        self.code = code
        self.reason = reason


class KernelResult:
    def __init__(self, error, reason):
        self.error = error
        self.reason = reason

    @property
    def succeeded(self):
        return self.error == OK


class GpuExecutor:
    """`NativeCpuExecutor`-shaped executor over the GPU path."""

    def __init__(self, device=0, packed_weights=True, int8_activations=True, memory_capacity=1 << 40):
        p = ctypes.c_void_p()
        rc = lib().mg_executor_create(device, int(packed_weights), int(int8_activations), memory_capacity,
                                      ctypes.byref(p))
        if rc:
            raise ExecutorError(rc, lib().mg_executor_last_error(None).decode())
        self.ptr = p

    def close(self):
        if self.ptr:
            lib().mg_executor_destroy(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _err(self):
        return lib().mg_executor_last_error(self.ptr).decode()

    def _check(self, rc):
        if rc:
            raise ExecutorError(rc, self._err())

    def write_packed_weight_tensor(self, rid, gguf_type, rows, cols, data, transposed=True):
        """Returns True (Stored) or False (Declined)."""
        b = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
        stored = ctypes.c_int()
        self._check(lib().mg_write_packed_weight_tensor(self.ptr, rid.encode(), gguf_type, rows, cols,
                                                        int(transposed),
                                                        b.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)),
                                                        b.size, ctypes.byref(stored)))
        return bool(stored.value)

    @staticmethod
    def _tensor_args(tensor):
        t = np.ascontiguousarray(tensor, dtype=np.float32)
        shape = (ctypes.c_uint64 * max(1, t.ndim))(*t.shape)
        return t, shape

    def write_tensor(self, rid, tensor):
        t, shape = self._tensor_args(tensor)
        self._check(lib().mg_write_tensor(self.ptr, rid.encode(), shape, t.ndim,
                                          t.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))

    def write_tensor_admitted(self, rid, tensor):
        t, shape = self._tensor_args(tensor)
        self._check(lib().mg_write_tensor_admitted(self.ptr, rid.encode(), shape, t.ndim,
                                                   t.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))

    def resident_shape(self, rid):
        shape = (ctypes.c_uint64 * 8)()
        rank = ctypes.c_uint32(8)
        rc = lib().mg_resident_shape(self.ptr, rid.encode(), shape, ctypes.byref(rank))
        if rc == UNKNOWN:
            return None
        self._check(rc)
        return [shape[i] for i in range(rank.value)]

    def read_tensor(self, rid):
        shape = self.resident_shape(rid)
        if shape is None:
            return None
        out = np.empty(shape, np.float32)
        self._check(lib().mg_read_tensor(self.ptr, rid.encode(), out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                         out.size))
        return out

    def write_tensor_value(self, rid, tensor=None, admitted=False):
        """`write_tensor_value(_admitted)`: tensor None writes back the Opaque
        value (stores nothing); an array is a Host value that replaces."""
        f = lib().mg_write_tensor_value_admitted if admitted else lib().mg_write_tensor_value
        if tensor is None:
            self._check(f(self.ptr, rid.encode(), 1, None, 0, None))
            return
        t, shape = self._tensor_args(tensor)
        self._check(f(self.ptr, rid.encode(), 0, shape, t.ndim, t.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))

    def copy_tensor_admitted(self, src, dst):
        self._check(lib().mg_copy_tensor_admitted(self.ptr, src.encode(), dst.encode()))

    def write_zeroed_kv_store(self, rid, shape, head_dimension, precision=KV_F32, exact_rows=0):
        """Returns True when the store was created."""
        s = (ctypes.c_uint64 * max(1, len(shape)))(*shape)
        created = ctypes.c_int()
        self._check(lib().mg_write_zeroed_kv_store(self.ptr, rid.encode(), s, len(shape), precision, head_dimension,
                                                   exact_rows, ctypes.byref(created)))
        return bool(created.value)

    def allocate_workspace(self, nbytes):
        out = ctypes.create_string_buffer(128)
        self._check(lib().mg_allocate_workspace(self.ptr, nbytes, out, 128))
        return out.value.decode()

    def release_workspace(self, allocation):
        self._check(lib().mg_release_workspace(self.ptr, allocation.encode()))

    def release_admitted_tensor(self, rid):
        r = ctypes.c_int()
        self._check(lib().mg_release_admitted_tensor(self.ptr, rid.encode(), ctypes.byref(r)))
        return bool(r.value)

    def synchronize(self):
        self._check(lib().mg_synchronize(self.ptr))

    def profile(self):
        """[(kernel, calls, seconds)], most time first (MAGNETAR_GPU_PROFILE=1)."""
        out = []
        name = ctypes.create_string_buffer(128)
        calls, secs = ctypes.c_uint64(), ctypes.c_double()
        for i in range(lib().mg_profile_count(self.ptr)):
            self._check(lib().mg_profile_entry(self.ptr, i, name, 128, ctypes.byref(calls), ctypes.byref(secs)))
            out.append((name.value.decode(), calls.value, secs.value))
        return out

    def is_packed(self, rid):
        return bool(lib().mg_is_packed(self.ptr, rid.encode()))

    def read_tensor_value_is_opaque(self, rid):
        return bool(lib().mg_read_tensor_value_is_opaque(self.ptr, rid.encode()))

    def release_tensor(self, rid):
        r = ctypes.c_int()
        self._check(lib().mg_release_tensor(self.ptr, rid.encode(), ctypes.byref(r)))
        return bool(r.value)

    def submit_kernel(self, kernel, invocation_id, inputs, output, attributes=None, deadline_millis=-1):
        attributes = attributes or {}
        ins = (ctypes.c_char_p * max(1, len(inputs)))(*[i.encode() for i in inputs])
        attrs = (Attribute * max(1, len(attributes)))(*[Attribute(k.encode(), str(v).encode())
                                                        for k, v in attributes.items()])
        handle = ctypes.create_string_buffer(512)
        self._check(lib().mg_submit_kernel(self.ptr, kernel.encode(), invocation_id.encode(), ins, len(inputs),
                                           output.encode() if output else None, attrs, len(attributes),
                                           deadline_millis, handle, 512))
        return handle.value.decode()

    def complete_kernel(self, handle):
        err = ctypes.c_int()
        reason = ctypes.create_string_buffer(1024)
        self._check(lib().mg_complete_kernel(self.ptr, handle.encode(), ctypes.byref(err), reason, 1024))
        return KernelResult(err.value, reason.value.decode())

    def observations(self):
        out = []
        kind = ctypes.create_string_buffer(128)
        kern = ctypes.create_string_buffer(128)
        for i in range(lib().mg_observation_count(self.ptr)):
            self._check(lib().mg_observation(self.ptr, i, kind, 128, kern, 128))
            out.append((kind.value.decode(), kern.value.decode()))
        return out

    def materializations(self):
        return int(lib().mg_materialization_count(self.ptr))

    def memory_used(self):
        return int(lib().mg_memory_used(self.ptr))
