"""ctypes view of the ggml API that libggml_mi355x.so carries (the restated ggml core:
tensors, graphs, backend vtables), so tests can drive the backend the way llama.cpp's
loader and scheduler do: allocate weights in a backend buffer, upload them with
ggml_backend_tensor_set, ask supports_op, run graph_compute."""
import ctypes

import numpy as np

GGML_TYPE_F32, GGML_TYPE_F16, GGML_TYPE_Q4_0, GGML_TYPE_Q8_0, GGML_TYPE_I32 = 0, 1, 2, 8, 26
GGML_PREC_F32 = 10
GGML_TENSOR_FLAG_OUTPUT = 2

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t


class Tensor(ctypes.Structure):
    """struct ggml_tensor (member order of ggml.h)"""
    _fields_ = [("type", ctypes.c_int), ("buffer", _P), ("ne", _I64 * 4), ("nb", _SZ * 4), ("op", ctypes.c_int),
                ("op_params", ctypes.c_int32 * 16), ("flags", ctypes.c_int32), ("src", _P * 10), ("view_src", _P),
                ("view_offs", _SZ), ("data", _P), ("name", ctypes.c_char * 64), ("extra", _P),
                ("padding", ctypes.c_char * 8)]


class InitParams(ctypes.Structure):
    _fields_ = [("mem_size", _SZ), ("mem_buffer", _P), ("no_alloc", ctypes.c_bool)]


TP = ctypes.POINTER(Tensor)

_SIGS = {
    "ggml_init": (_P, [InitParams]),
    "ggml_free": (None, [_P]),
    "ggml_new_tensor_1d": (TP, [_P, ctypes.c_int, _I64]),
    "ggml_new_tensor_2d": (TP, [_P, ctypes.c_int, _I64, _I64]),
    "ggml_new_tensor_3d": (TP, [_P, ctypes.c_int, _I64, _I64, _I64]),
    "ggml_new_tensor_4d": (TP, [_P, ctypes.c_int, _I64, _I64, _I64, _I64]),
    "ggml_set_name": (TP, [TP, ctypes.c_char_p]),
    "ggml_set_output": (None, [TP]),
    "ggml_nbytes": (_SZ, [TP]),
    "ggml_mul_mat": (TP, [_P, TP, TP]),
    "ggml_flash_attn_ext": (TP, [_P, TP, TP, TP, TP, ctypes.c_float, ctypes.c_float, ctypes.c_float]),
    "ggml_flash_attn_ext_add_kv_lengths": (None, [TP, TP]),
    "ggml_rms_norm": (TP, [_P, TP, ctypes.c_float]),
    "ggml_mul": (TP, [_P, TP, TP]),
    "ggml_add": (TP, [_P, TP, TP]),
    "ggml_new_graph": (_P, [_P]),
    "ggml_build_forward_expand": (None, [_P, TP]),
    "ggml_backend_cpu_buffer_type": (_P, []),
    "ggml_backend_buft_get_alloc_size": (_SZ, [_P, TP]),
    "ggml_backend_alloc_ctx_tensors_from_buft": (_P, [_P, _P]),
    "ggml_backend_buffer_free": (None, [_P]),
    "ggml_backend_tensor_set": (None, [TP, _P, _SZ, _SZ]),
    "ggml_backend_tensor_get": (None, [TP, _P, _SZ, _SZ]),
    "ggml_backend_supports_op": (ctypes.c_bool, [_P, TP]),
    "ggml_backend_graph_compute": (ctypes.c_int, [_P, _P]),
    "ggml_gallocr_new": (_P, [_P]),
    "ggml_gallocr_free": (None, [_P]),
    "ggml_gallocr_alloc_graph": (ctypes.c_bool, [_P, _P]),
    "ggml_backend_get_default_buffer_type": (_P, [_P]),
    "ggml_backend_mi355x_init": (_P, [ctypes.c_int]),
    "ggml_backend_mi355x_buffer_type": (_P, [ctypes.c_int]),
    "ggml_backend_mi355x_set_smooth_factors": (ctypes.c_bool, [TP, _P, _I64]),
    "ggml_backend_free": (None, [_P]),
}


def bind(lib):
    if not getattr(lib, "_ggml_declared", False):
        for name, (res, args) in _SIGS.items():
            f = getattr(lib, name)
            f.restype = res
            f.argtypes = args
        lib._ggml_declared = True
    return lib


class Context:
    """a no_alloc ggml context: tensor headers only, data from backend buffers"""

    def __init__(self, lib):
        self.L = bind(lib)
        self.ctx = self.L.ggml_init(InitParams(0, None, True))
        self.buffers = []

    def tensor(self, type_, *ne, name=None):
        fn = {1: self.L.ggml_new_tensor_1d, 2: self.L.ggml_new_tensor_2d, 3: self.L.ggml_new_tensor_3d,
              4: self.L.ggml_new_tensor_4d}[len(ne)]
        t = fn(self.ctx, type_, *ne)
        if name:
            self.L.ggml_set_name(t, name.encode())
        return t

    def alloc(self, buft):
        """allocate every tensor of the context without data in one buffer of buft"""
        b = self.L.ggml_backend_alloc_ctx_tensors_from_buft(self.ctx, buft)
        assert b, "buffer allocation failed"
        self.buffers.append(b)
        return b

    def set(self, t, arr, offset=0):
        a = np.ascontiguousarray(arr)
        self.L.ggml_backend_tensor_set(t, a.ctypes.data, offset, a.nbytes)

    def get(self, t, dtype, count=None):
        n = self.L.ggml_nbytes(t)
        out = np.empty(n // np.dtype(dtype).itemsize if count is None else count, dtype)
        self.L.ggml_backend_tensor_get(t, out.ctypes.data, 0, out.nbytes)
        return out

    def free(self):
        for b in self.buffers:
            self.L.ggml_backend_buffer_free(b)
        self.buffers = []
        if self.ctx:
            self.L.ggml_free(self.ctx)
            self.ctx = None
