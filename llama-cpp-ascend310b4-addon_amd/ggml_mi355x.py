"""Python host binding of libggml_mi355x.so (ctypes + numpy, no torch).

The library carries its own HIP runtime link (/opt/rocm), so the host side
here uses the library's device-memory, stream and event wrappers instead of a
second HIP runtime.  Every entry point raises MiError on a non-zero status;
nothing falls back to a CPU path: a missing library is an ImportError-like
failure at load time.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libggml_mi355x.so")

MI_OK = 0
MI_ERR_ARG = -1
MI_ERR_ALIGN = -2
MI_ERR_WORKSPACE = -3
MI_ERR_NODEVICE = -4
MI_ERR_UNSUPPORTED = -5

Q8_ROUND_REF = 0
Q8_ROUND_X86 = 1


class MiError(RuntimeError):
    def __init__(self, fn, code, msg):
        super().__init__(f"{fn} failed with status {code}: {msg}")
        self.code = code


_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t
_F = ctypes.c_float
_I = ctypes.c_int

_SIGS = {
    "mi_last_error": (ctypes.c_char_p, []),
    "mi_device_count": (_I, [ctypes.POINTER(_I)]),
    "mi_set_device": (_I, [_I]),
    "mi_device_name": (_I, [_I, ctypes.c_char_p, _SZ]),
    "mi_malloc": (_I, [ctypes.POINTER(_P), _SZ]),
    "mi_free": (_I, [_P]),
    "mi_memcpy_h2d": (_I, [_P, _P, _SZ, _P]),
    "mi_memcpy_d2h": (_I, [_P, _P, _SZ, _P]),
    "mi_memcpy_d2d": (_I, [_P, _P, _SZ, _P]),
    "mi_memset": (_I, [_P, _I, _SZ, _P]),
    "mi_stream_create": (_I, [ctypes.POINTER(_P)]),
    "mi_stream_destroy": (_I, [_P]),
    "mi_stream_sync": (_I, [_P]),
    "mi_device_sync": (_I, []),
    "mi_event_create": (_I, [ctypes.POINTER(_P)]),
    "mi_event_destroy": (_I, [_P]),
    "mi_event_record": (_I, [_P, _P]),
    "mi_event_elapsed_ms": (_I, [ctypes.POINTER(_F), _P, _P]),
    "mi_graph_capture_begin": (_I, [_P]),
    "mi_graph_capture_end": (_I, [_P, ctypes.POINTER(_P)]),
    "mi_graph_launch": (_I, [_P, _P]),
    "mi_graph_destroy": (_I, [_P]),
    "mi_q8_0_packed_size": (_SZ, [_I64, _I64]),
    "mi_q4_0_packed_size": (_SZ, [_I64, _I64]),
    "mi_prepack_q8_0": (_I, [_P, _P, _P, _I64, _I64]),
    "mi_prepack_q4_0": (_I, [_P, _P, _P, _I64, _I64]),
    "mi_prepack_q8_0_host": (_I, [_P, _P, _I64, _I64]),
    "mi_prepack_q4_0_host": (_I, [_P, _P, _I64, _I64]),
    "mi_unpack_q8_0_host": (_I, [_P, _P, _I64, _I64]),
    "mi_unpack_q4_0_host": (_I, [_P, _P, _I64, _I64]),
    "mi_quantize_f16_q8_0": (_I, [_P, _P, _P, _P, _I64, _I64]),
    "mi_xq_size": (_SZ, [_I64, _I64]),
    "mi_xq_d_offset": (_SZ, [_I64, _I64]),
    "mi_act_quant_q8_0": (_I, [_P, _P, _P, _I64, _I64, _P, _I]),
    "mi_gemv_q8_0": (_I, [_P, _P, _P, _P, _I64, _I64, _I64]),
    "mi_mul_mat_q8_0_workspace_size": (_SZ, [_I64, _I64]),
    "mi_mul_mat_q8_0_f32": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _P, _SZ]),
    "mi_q8_0_block_dots": (_I, [_P, _P, _P, _P, _I64, _I64]),
    "mi_gemv_q4_0_f16": (_I, [_P, _P, _P, _P, _I64, _I64, _I64]),
    "mi_mul_mat_q4_0_f32": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _P, _SZ]),
    "mi_mul_mat_q4_0_workspace_size": (_SZ, [_I64, _I64]),
    "mi_gemv_q4_0_f16_add": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64]),
    "mi_cast_f32_f16": (_I, [_P, _P, _P, _I64]),
    "mi_gemv_f16": (_I, [_P, _P, _I64, _P, _P, _I64, _I64, _I64]),
    "mi_fa_decode_workspace_size": (_SZ, [_I64, _I64, _I64, _I64]),
    "mi_fa_decode": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _SZ, _SZ, _SZ, _SZ, _F, _P, _P, _SZ]),
    "mi_kv_lengths": (_I, [_P, _P, _I, _I64, _I64, _P]),
    "mi_fa_decode_batch_workspace_size": (_SZ, [_I64, _I64, _I64, _I64, _I64]),
    "mi_fa_decode_batch": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _SZ, _SZ, _SZ, _SZ, _F, _P, _I64, _SZ,
                                _SZ, _SZ, _SZ, _SZ, _P, _SZ]),
    "mi_fa_decode_rows": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _SZ, _SZ, _SZ, _SZ, _F, _P, _I64, _SZ,
                               _SZ, _SZ, _P, _SZ]),
    "mi_fa_decode_num_splits": (_I64, [_I64, _I64, _I64, _I64]),
    "mi_fa_decode_partials": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _SZ, _SZ, _SZ, _SZ, _F, _P, _SZ]),
    "mi_fa_decode_noalloc_max_workspace": (_SZ, []),
    "mi_fa_decode_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _SZ, _SZ, _SZ, _SZ, _F, _P]),
    "mi_mul_mat_q8_0_f32_multi": (_I, [_P, _I, _P, _P, _P, _I64, _P, _P, _I, _P, _SZ]),
    "mi_rms_norm": (_I, [_P, _P, _P, _P, _I64, _I64, _F]),
    "mi_head_f16_argmax_workspace_size": (_SZ, [_I64, _I64]),
    "mi_head_f16_argmax": (_I, [_P, _P, _I64, _P, _P, _F, _P, _P, _I64, _I64, _P, _SZ]),
    "mi_add_bcast": (_I, [_P, _P, _P, _P, _I64, _I64]),
    "mi_mul_bcast": (_I, [_P, _P, _P, _P, _I64, _I64]),
    "mi_rope_neox": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _F, _F, _F, _SZ, _SZ, _SZ, _SZ]),
    "mi_set_rows_f16": (_I, [_P, _P, _P, _I, _P, _I64, _I64, _SZ, _SZ, _I64]),
    "mi_get_rows": (_I, [_P, _P, _I, _P, _P, _I64, _I64, _SZ, _I64]),
    "mi_swiglu": (_I, [_P, _P, _P, _P, _I64]),
    "mi_argmax_workspace_size": (_SZ, [_I64, _I64]),
    "mi_argmax": (_I, [_P, _P, _P, _I64, _I64, _P, _SZ]),
    "mi_mul_mat_q8_0_f32_fused": (_I, [_P, _I, _P, _P, _P, _P, _I64, _P, _P, _F, _P, _I]),
    "mi_mul_mat_q8_0_f32_batch": (_I, [_P, _I, _P, _P, _P, _P, _P, _I64, _I64, _P, _P, _P, _F, _P, _I, _P, _SZ]),
    "mi_mul_mat_q8_0_f32_lse": (_I, [_P, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _P, _I]),
    "mi_gate_up_swiglu_q8_0": (_I, [_P, _P, _P, _I64, _I64, _P, _P, _F, _P, _P, _I, _P]),
    "mi_gate_up_swiglu_f32_q8_0": (_I, [_P, _P, _P, _I64, _I64, _P, _P, _F, _P, _P, _I, _P]),
    "mi_gate_up_pair_q8_0": (_I, [_P, _P, _P, _I64, _I64, _P, _P, _F, _P, _P, _I, _P, _P, _P]),
    "mi_mul_mat_q4_0_f32_batch": (_I, [_P, _I, _P, _P, _P, _P, _P, _I64, _I64, _P, _P, _P, _F, _P, _SZ]),
    "mi_mul_mat_q4_0_batch_xp": (_I, [_P, _I, _P, _P, _P, _P, _P, _I64, _I64, _P]),
    "mi_mul_mat_q4_0_gate_up_glu_batch": (_I, [_P, _P, _P, _I64, _I64, _I64, _P, _P, _F, _P, _SZ, _P]),
    "mi_qkv_rope_kv_q4_0_batch": (_I, [_P, _P, _P, _P, _I64, _I64, _P, _P, _F, _P, _SZ, _I64, _P, _F, _F, _F, _P, _P, _SZ,
                                       _P, _SZ, _P, _I, _I64]),
    "mi_fa_decode_batch_q4act": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _SZ, _SZ, _SZ, _SZ, _F, _P, _I64,
                                      _SZ, _SZ, _SZ, _SZ, _P, _SZ]),
    "mi_rope_kv_rows": (_I, [_P, _P, _P, _P, _P, _P, _SZ, _P, _SZ, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _F,
                             _F, _F]),
    "mi_mul_mat_q4_0_f32_fused": (_I, [_P, _I, _P, _P, _P, _P, _I64, _P, _P, _F]),
    "mi_gate_up_swiglu_q4_0": (_I, [_P, _P, _P, _I64, _I64, _P, _P, _F, _P]),
    "mi_qkv_rope_kv_q4_0": (_I, [_P, _P, _P, _P, _I64, _P, _P, _F, _I64, _P, _F, _F, _F, _P, _P, _SZ, _P, _SZ,
                                 _P, _I, _I64, _P]),
    "mi_rope_table": (_I, [_P, _P, _I64, _F, _F, _F, _P]),
    "mi_qkv_rope_kv_q8_0": (_I, [_P, _P, _P, _P, _I64, _P, _P, _F, _P, _I, _I64, _P, _F, _F, _F, _P, _P, _SZ, _P, _SZ,
                                 _P, _I, _I64, _P]),
    "mi_swiglu_quant_q8_0": (_I, [_P, _P, _P, _P, _I64, _P, _I]),
    "mi_gemv_q8_0_add": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64]),
    "mi_fill_mask_f16": (_I, [_P, _P, _P, _I64]),
    "mi_fill_f16_uniform": (_I, [_P, _P, _I64, _I64, _SZ, ctypes.c_uint64, _F]),
    "mi_persist_create": (_I, [_P, _I, _I, _I, _I, _I, _I, _I]),
    "mi_persist_destroy": (None, [_P]),
    "mi_persist_set_layers": (_I, [_P, _P, _P, _I]),
    "mi_persist_supported": (_I, [_I64, _I, _I, _I, _I, _I]),
    "mi_persist_decode_q8_0": (_I, [_P, _P, _P]),
    "mi_persist_status": (_I, [_P]),
    "mi_persist_enable_trace": (_I, [_P]),
    "mi_persist_read_trace": (_I, [_P, _P, _SZ, _P, _P, _P, _P]),
}

# every symbol the C ABI header declares (checked by the CPU tests)
EXPORTED = tuple(_SIGS)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OSError(f"libggml_mi355x.so is not built at {LIB_PATH}; run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def last_error():
    return lib().mi_last_error().decode(errors="replace")


def _call(name, *args):
    r = getattr(lib(), name)(*args)
    if r != MI_OK:
        raise MiError(name, r, last_error())
    return r


def device_count():
    n = _I(0)
    lib().mi_device_count(ctypes.byref(n))
    return n.value


def device_name(dev=0):
    buf = ctypes.create_string_buffer(256)
    _call("mi_device_name", dev, buf, 256)
    return buf.value.decode()


# ---------------------------------------------------------------- memory

class DeviceBuffer:
    """A hipMalloc'd buffer; .ptr is the device address."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = _P()
        _call("mi_malloc", ctypes.byref(p), max(self.nbytes, 1))
        self.ptr = p.value

    def free(self):
        if self.ptr:
            lib().mi_free(_P(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def upload(self, arr, stream=None, offset=0):
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes
        _call("mi_memcpy_h2d", _P(self.ptr + offset), arr.ctypes.data, arr.nbytes, _P(stream))
        return self

    def download(self, dtype, count=None, stream=None, offset=0):
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        _call("mi_memcpy_d2h", out.ctypes.data, _P(self.ptr + offset), out.nbytes, _P(stream))
        return out

    def zero(self, stream=None):
        _call("mi_memset", _P(self.ptr), 0, self.nbytes, _P(stream))
        return self


def to_device(arr, stream=None):
    arr = np.ascontiguousarray(arr)
    return DeviceBuffer(arr.nbytes).upload(arr, stream)


class Stream:
    def __init__(self):
        p = _P()
        _call("mi_stream_create", ctypes.byref(p))
        self.ptr = p.value

    def sync(self):
        _call("mi_stream_sync", _P(self.ptr))

    def destroy(self):
        if self.ptr:
            lib().mi_stream_destroy(_P(self.ptr))
            self.ptr = None


class Event:
    def __init__(self):
        p = _P()
        _call("mi_event_create", ctypes.byref(p))
        self.ptr = p.value

    def record(self, stream=None):
        _call("mi_event_record", _P(self.ptr), _P(stream))

    def elapsed_ms(self, end):
        ms = _F(0)
        _call("mi_event_elapsed_ms", ctypes.byref(ms), _P(self.ptr), _P(end.ptr))
        return ms.value

    def destroy(self):
        if self.ptr:
            lib().mi_event_destroy(_P(self.ptr))
            self.ptr = None


def device_sync():
    _call("mi_device_sync")


class Graph:
    """Captures every launch issued on `stream` inside the with-block into a HIP graph."""

    def __init__(self, stream):
        assert stream is not None and stream.ptr, "graph capture needs a created (non-null) stream"
        self.stream = stream
        self.exec = None

    def __enter__(self):
        _call("mi_graph_capture_begin", _P(self.stream.ptr))
        return self

    def __exit__(self, et, ev, tb):
        p = _P()
        r = lib().mi_graph_capture_end(_P(self.stream.ptr), ctypes.byref(p))
        if et is None:
            if r != MI_OK:
                raise MiError("mi_graph_capture_end", r, last_error())
            self.exec = p.value
        return False

    def launch(self):
        _call("mi_graph_launch", _P(self.exec), _P(self.stream.ptr))

    def destroy(self):
        if self.exec:
            lib().mi_graph_destroy(_P(self.exec))
            self.exec = None


# ---------------------------------------------------------------- prepack

def q8_0_packed_size(n, k):
    return lib().mi_q8_0_packed_size(n, k)


def q4_0_packed_size(n, k):
    return lib().mi_q4_0_packed_size(n, k)


def prepack_q8_0_host(blocks, n, k):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(q8_0_packed_size(n, k), dtype=np.uint8)
    _call("mi_prepack_q8_0_host", blocks.ctypes.data, out.ctypes.data, n, k)
    return out


def unpack_q8_0_host(packed, n, k):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty(n * (k // 32) * 34, dtype=np.uint8)
    _call("mi_unpack_q8_0_host", packed.ctypes.data, out.ctypes.data, n, k)
    return out.reshape(n, -1)


def prepack_q4_0_host(blocks, n, k):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(q4_0_packed_size(n, k), dtype=np.uint8)
    _call("mi_prepack_q4_0_host", blocks.ctypes.data, out.ctypes.data, n, k)
    return out


def unpack_q4_0_host(packed, n, k):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty(n * (k // 32) * 18, dtype=np.uint8)
    _call("mi_unpack_q4_0_host", packed.ctypes.data, out.ctypes.data, n, k)
    return out.reshape(n, -1)


def quantize_f16_q8_0(w_f16_dev, s_dev, dst_dev, n, k, stream=None):
    """A8W8 weight quantization: F16 [n][k] times s[k] (None = 1) to the Q8_0 packed layout"""
    _call("mi_quantize_f16_q8_0", _P(stream), _P(w_f16_dev), _P(s_dev), _P(dst_dev), n, k)


def prepack_q8_0(src_dev, dst_dev, n, k, stream=None):
    _call("mi_prepack_q8_0", _P(stream), _P(src_dev), _P(dst_dev), n, k)


def prepack_q4_0(src_dev, dst_dev, n, k, stream=None):
    _call("mi_prepack_q4_0", _P(stream), _P(src_dev), _P(dst_dev), n, k)


# ---------------------------------------------------------------- kernels (device pointers)

def xq_size(m, k):
    return lib().mi_xq_size(m, k)


def xq_d_offset(m, k):
    return lib().mi_xq_d_offset(m, k)


def act_quant_q8_0(x, inv_s, m, k, xq, rounding=Q8_ROUND_X86, stream=None):
    _call("mi_act_quant_q8_0", _P(stream), _P(x), _P(inv_s), m, k, _P(xq), rounding)


def gemv_q8_0(w_packed, xq, y, n, k, m=1, stream=None):
    _call("mi_gemv_q8_0", _P(stream), _P(w_packed), _P(xq), _P(y), n, k, m)


def mul_mat_q8_0_workspace_size(m, k):
    return lib().mi_mul_mat_q8_0_workspace_size(m, k)


def mul_mat_q8_0_f32(w_packed, x, inv_s, y, n, k, m=1, rounding=Q8_ROUND_X86, ws=None, ws_bytes=0, stream=None):
    _call("mi_mul_mat_q8_0_f32", _P(stream), _P(w_packed), _P(x), _P(inv_s), _P(y), n, k, m, rounding, _P(ws),
          ws_bytes)


def mul_mat_q8_0_f32_multi(w_packed, n, y, k, x, inv_s=None, rounding=Q8_ROUND_X86, ws=None, ws_bytes=0,
                           stream=None):
    """up to four Q8_0 matrices (device pointers w_packed[i], n[i] rows, outputs y[i]) on one activation row"""
    cnt = len(w_packed)
    wa = (ctypes.c_void_p * cnt)(*w_packed)
    na = (ctypes.c_int64 * cnt)(*n)
    ya = (ctypes.c_void_p * cnt)(*y)
    _call("mi_mul_mat_q8_0_f32_multi", _P(stream), cnt, ctypes.cast(wa, ctypes.c_void_p), ctypes.cast(na, ctypes.c_void_p),
          ctypes.cast(ya, ctypes.c_void_p), k, _P(x), _P(inv_s), rounding, _P(ws), ws_bytes)


def q8_0_block_dots(w_packed, xq, out, n, k, stream=None):
    _call("mi_q8_0_block_dots", _P(stream), _P(w_packed), _P(xq), _P(out), n, k)


def gemv_q4_0_f16(w_packed, x16, y, n, k, m=1, stream=None):
    _call("mi_gemv_q4_0_f16", _P(stream), _P(w_packed), _P(x16), _P(y), n, k, m)


def mul_mat_q4_0_workspace_size(m, k):
    return lib().mi_mul_mat_q4_0_workspace_size(m, k)


def mul_mat_q4_0_f32(w_packed, x, y, n, k, m=1, ws=None, ws_bytes=0, stream=None):
    _call("mi_mul_mat_q4_0_f32", _P(stream), _P(w_packed), _P(x), _P(y), n, k, m, _P(ws), ws_bytes)


def gemv_f16(w, ldw, x, y, n, k, m=1, stream=None):
    _call("mi_gemv_f16", _P(stream), _P(w), ldw, _P(x), _P(y), n, k, m)


def fa_decode_workspace_size(n_kv, n_q_heads, n_kv_heads, d):
    return lib().mi_fa_decode_workspace_size(n_kv, n_q_heads, n_kv_heads, d)


def fa_decode(q, k, v, mask, kv_len, n_kv, n_q_heads, n_kv_heads, d, k_nb1, k_nb2, v_nb1, v_nb2, scale, out,
              ws, ws_bytes, stream=None):
    _call("mi_fa_decode", _P(stream), _P(q), _P(k), _P(v), _P(mask), _P(kv_len), n_kv, n_q_heads, n_kv_heads, d,
          k_nb1, k_nb2, v_nb1, v_nb2, scale, _P(out), _P(ws), ws_bytes)


def fa_decode_batch_workspace_size(n_kv, n_q_heads, n_kv_heads, d, n_seq):
    return lib().mi_fa_decode_batch_workspace_size(n_kv, n_q_heads, n_kv_heads, d, n_seq)


def fa_decode_batch(q, k, v, mask, kv_len, n_kv, n_q_heads, n_kv_heads, d, k_nb1, k_nb2, v_nb1, v_nb2, scale, out,
                    n_seq, q_seq, k_seq, v_seq, mask_seq, out_seq, ws, ws_bytes, stream=None):
    _call("mi_fa_decode_batch", _P(stream), _P(q), _P(k), _P(v), _P(mask), _P(kv_len), n_kv, n_q_heads, n_kv_heads,
          d, k_nb1, k_nb2, v_nb1, v_nb2, scale, _P(out), n_seq, q_seq, k_seq, v_seq, mask_seq, out_seq, _P(ws),
          ws_bytes)


def fa_decode_rows(q, k, v, mask, kv_len, n_kv, n_q_heads, n_kv_heads, d, k_nb1, k_nb2, v_nb1, v_nb2, scale, out,
                   n_rows, q_row, mask_row, out_row, ws, ws_bytes, stream=None):
    _call("mi_fa_decode_rows", _P(stream), _P(q), _P(k), _P(v), _P(mask), _P(kv_len), n_kv, n_q_heads, n_kv_heads,
          d, k_nb1, k_nb2, v_nb1, v_nb2, scale, _P(out), n_rows, q_row, mask_row, out_row, _P(ws), ws_bytes)


def fa_decode_noalloc(q, k, v, mask, kv_len, n_kv, n_q_heads, n_kv_heads, d, k_nb1, k_nb2, v_nb1, v_nb2, scale,
                      out, stream=None):
    """mi_fa_decode on the library's fixed per-device scratch (allocates nothing)"""
    _call("mi_fa_decode_noalloc", _P(stream), _P(q), _P(k), _P(v), _P(mask), _P(kv_len), n_kv, n_q_heads, n_kv_heads,
          d, k_nb1, k_nb2, v_nb1, v_nb2, scale, _P(out))


def kv_lengths(mask, is_f16, n_kv, n_rows, out, stream=None):
    _call("mi_kv_lengths", _P(stream), _P(mask), 1 if is_f16 else 0, n_kv, n_rows, _P(out))


# ---------------------------------------------------------------- Qwen2 decode driver (mi_qwen2.h)

class _QwenHP(ctypes.Structure):
    _fields_ = [("n_layer", ctypes.c_int32), ("n_embd", ctypes.c_int32), ("n_head", ctypes.c_int32),
                ("n_head_kv", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("n_ff", ctypes.c_int32),
                ("n_vocab", ctypes.c_int32), ("n_ctx", ctypes.c_int32), ("rms_eps", ctypes.c_float),
                ("rope_theta", ctypes.c_float), ("wtype", ctypes.c_int32), ("use_bias", ctypes.c_int32),
                ("n_seq", ctypes.c_int32)]


_QWEN_SIGS = {
    "mi_qwen2_create": (_P, [ctypes.POINTER(_QwenHP), _I]),
    "mi_qwen2_free": (None, [_P]),
    "mi_qwen2_last_error": (ctypes.c_char_p, []),
    "mi_qwen2_set_tensor": (_I, [_P, ctypes.c_char_p, _P, _SZ]),
    "mi_qwen2_set_smooth": (_I, [_P, ctypes.c_char_p, _P, _I64]),
    "mi_qwen2_tensor_nbytes": (_I64, [_P, ctypes.c_char_p, _P]),
    "mi_qwen2_decode": (_I, [_P, ctypes.c_int32, ctypes.c_int32, _P, _P]),
    "mi_qwen2_generate": (_I, [_P, _P, ctypes.c_int32, ctypes.c_int32, _P, ctypes.POINTER(ctypes.c_double)]),
    "mi_qwen2_decode_steps": (_I, [_P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _P,
                                  ctypes.POINTER(ctypes.c_double)]),
    "mi_qwen2_n_seq": (ctypes.c_int32, [_P]),
    "mi_qwen2_decode_batch": (_I, [_P, _P, _P, _P, _P]),
    "mi_qwen2_decode_steps_batch": (_I, [_P, _P, _P, ctypes.c_int32, _P, ctypes.POINTER(ctypes.c_double)]),
    "mi_qwen2_get_cache_seq": (_I, [_P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _P, _SZ]),
    "mi_qwen2_persist_timing": (_I, [_P, ctypes.POINTER(_I64), ctypes.POINTER(ctypes.c_double)]),
    "mi_qwen2_prefill": (_I, [_P, ctypes.c_int32, _P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _P, _P,
                              ctypes.POINTER(ctypes.c_double)]),
    "mi_qwen2_set_cache_seq": (_I, [_P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _P, _SZ]),
    "mi_qwen2_fill_cache": (_I, [_P, ctypes.c_int32, ctypes.c_uint64, ctypes.c_float]),
    "mi_qwen2_get_cache": (_I, [_P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _P, _SZ]),
    "mi_qwen2_reset": (_I, [_P]),
    "mi_smooth_scales_read": (_I, [ctypes.c_char_p, _I64, _I64, _P]),
    "mi_qwen2_load_smooth_file": (_I, [_P, ctypes.c_char_p, _I]),
    "mi_qwen2_set_layer_dump": (_I, [_P, _I]),
    "mi_qwen2_dump_layers": (_I, [_P, ctypes.c_char_p, _I]),
}
EXPORTED = EXPORTED + tuple(_QWEN_SIGS)


def read_smooth_scales(path, n_layer, n_embd):
    """Host-side read of a SmoothQuant scale file through the library's own parser."""
    out = np.empty((n_layer, n_embd), np.float32)
    r = _qlib().mi_smooth_scales_read(str(path).encode(), n_layer, n_embd, out.ctypes.data)
    if r != 0:
        raise MiError("mi_smooth_scales_read", r, _qlib().mi_qwen2_last_error().decode())
    return out


def _qlib():
    L = lib()
    if not getattr(L, "_qwen_declared", False):
        for name, (res, args) in _QWEN_SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        L._qwen_declared = True
    return L


class Qwen2Model:
    """A Qwen2 model run through the ggml backend (ggml_backend_mi355x) one token per step."""

    def __init__(self, hp, device=0):
        L = _qlib()
        h = _QwenHP()
        for f, _ in _QwenHP._fields_:
            setattr(h, f, hp.get(f, 1 if f == "n_seq" else 0))
        self.hp = dict(hp)
        self.ptr = L.mi_qwen2_create(ctypes.byref(h), device)
        if not self.ptr:
            raise MiError("mi_qwen2_create", -1, L.mi_qwen2_last_error().decode())
        self.n_seq = int(L.mi_qwen2_n_seq(self.ptr))
        self.logits = np.empty(hp["n_vocab"] * self.n_seq, np.float32)

    def _chk(self, name, r):
        if r != 0:
            raise MiError(name, r, _qlib().mi_qwen2_last_error().decode())

    def set_tensor(self, name, arr):
        arr = np.ascontiguousarray(arr)
        self._chk("mi_qwen2_set_tensor", _qlib().mi_qwen2_set_tensor(self.ptr, name.encode(), arr.ctypes.data,
                                                                    arr.nbytes))

    def set_smooth(self, weight_name, s):
        s = np.ascontiguousarray(s, np.float32)
        self._chk("mi_qwen2_set_smooth", _qlib().mi_qwen2_set_smooth(self.ptr, weight_name.encode(), s.ctypes.data,
                                                                    s.size))

    def load_smooth_file(self, path, weights_presmoothed=False):
        """SmoothQuant factors of every layer's ffn_gate / ffn_up from a scale file
        (little-endian fp32 [n_layer][n_embd]).  F16 weights on the A8W8 path get s
        folded in by the backend; Q8_0 weights are refused unless weights_presmoothed
        asserts that their blocks already hold W*diag(s)."""
        self._chk("mi_qwen2_load_smooth_file", _qlib().mi_qwen2_load_smooth_file(self.ptr, str(path).encode(),
                                                                                1 if weights_presmoothed else 0))

    def set_layer_dump(self, on=True):
        """keep ffn_norm-<layer> / ffn_out-<layer> as graph outputs in later steps"""
        self._chk("mi_qwen2_set_layer_dump", _qlib().mi_qwen2_set_layer_dump(self.ptr, 1 if on else 0))

    def dump_layers(self, path, append=False):
        """The latest step's layer tensors as LLDUMP1 records (see lldump.py): per layer
        ffn_norm-<layer> and ffn_out-<layer> with the layer dump on, then l_out-<layer>."""
        self._chk("mi_qwen2_dump_layers", _qlib().mi_qwen2_dump_layers(self.ptr, str(path).encode(),
                                                                      1 if append else 0))

    def load(self, tensors, smooth=None):
        for name, arr in tensors.items():
            self.set_tensor(name, arr)
        for name, s in (smooth or {}).items():
            self.set_smooth(name, s)

    def decode(self, token, pos, want_logits=False):
        nxt = ctypes.c_int32(0)
        self._chk("mi_qwen2_decode", _qlib().mi_qwen2_decode(self.ptr, int(token), int(pos), ctypes.byref(nxt),
                                                             self.logits.ctypes.data if want_logits else None))
        return (nxt.value, self.logits.copy()) if want_logits else nxt.value

    def generate(self, prompt, n_gen):
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(max(n_gen, 1), np.int32)
        secs = ctypes.c_double(0.0)
        self._chk("mi_qwen2_generate", _qlib().mi_qwen2_generate(self.ptr, prompt.ctypes.data, prompt.size, n_gen,
                                                                 out.ctypes.data, ctypes.byref(secs)))
        return out[:n_gen], secs.value

    def decode_steps(self, token, pos, n_steps):
        """greedy continuation from (token, pos) -> (tokens[n_steps], seconds)"""
        out = np.empty(max(n_steps, 1), np.int32)
        secs = ctypes.c_double(0.0)
        self._chk("mi_qwen2_decode_steps", _qlib().mi_qwen2_decode_steps(self.ptr, int(token), int(pos), int(n_steps),
                                                                         out.ctypes.data, ctypes.byref(secs)))
        return out[:n_steps], secs.value

    def decode_batch(self, tokens, pos, want_logits=False):
        """one step of all sequences -> next tokens [n_seq] (and logits [n_seq, n_vocab])"""
        t = np.ascontiguousarray(tokens, np.int32)
        p = np.ascontiguousarray(pos, np.int32)
        assert t.size == self.n_seq and p.size == self.n_seq
        nxt = np.empty(self.n_seq, np.int32)
        self._chk("mi_qwen2_decode_batch", _qlib().mi_qwen2_decode_batch(
            self.ptr, t.ctypes.data, p.ctypes.data, nxt.ctypes.data, self.logits.ctypes.data if want_logits else None))
        if want_logits:
            return nxt, self.logits.reshape(self.n_seq, -1).copy()
        return nxt

    def decode_steps_batch(self, tokens, pos, n_steps):
        """greedy continuation of all sequences -> (tokens [n_steps, n_seq], seconds)"""
        t = np.ascontiguousarray(tokens, np.int32)
        p = np.ascontiguousarray(pos, np.int32)
        out = np.empty((max(n_steps, 1), self.n_seq), np.int32)
        secs = ctypes.c_double(0.0)
        self._chk("mi_qwen2_decode_steps_batch", _qlib().mi_qwen2_decode_steps_batch(
            self.ptr, t.ctypes.data, p.ctypes.data, int(n_steps), out.ctypes.data, ctypes.byref(secs)))
        return out[:n_steps], secs.value

    def get_cache_seq(self, layer, is_v, seq, n_pos):
        out = np.empty((n_pos, self.hp["n_head_kv"] * self.hp["head_dim"]), np.uint16)
        self._chk("mi_qwen2_get_cache_seq", _qlib().mi_qwen2_get_cache_seq(
            self.ptr, int(layer), int(is_v), int(seq), int(n_pos), out.ctypes.data, out.nbytes))
        return out

    def set_cache_seq(self, layer, is_v, seq, data):
        data = np.ascontiguousarray(data, np.uint16)
        self._chk("mi_qwen2_set_cache_seq", _qlib().mi_qwen2_set_cache_seq(
            self.ptr, int(layer), int(is_v), int(seq), int(data.shape[0]), data.ctypes.data, data.nbytes))

    def prefill(self, tokens, pos0=0, n_ubatch=8, seq=0, want_logits=False):
        """prompt tokens in ubatches of n_ubatch -> (next token, logits or None, seconds)"""
        t = np.ascontiguousarray(tokens, np.int32)
        nxt = ctypes.c_int32(0)
        lg = np.empty(self.hp["n_vocab"], np.float32) if want_logits else None
        secs = ctypes.c_double(0.0)
        self._chk("mi_qwen2_prefill", _qlib().mi_qwen2_prefill(
            self.ptr, int(seq), t.ctypes.data, int(t.size), int(pos0), int(n_ubatch), ctypes.byref(nxt),
            lg.ctypes.data if want_logits else None, ctypes.byref(secs)))
        return int(nxt.value), lg, secs.value

    def persist_timing(self):
        """(launches, total ms) of the persistent layer-stack launches timed so far
        (GGML_MI355X_PERSIST_TIMING=1 at creation)"""
        n, ms = _I64(0), ctypes.c_double(0.0)
        self._chk("mi_qwen2_persist_timing", _qlib().mi_qwen2_persist_timing(self.ptr, ctypes.byref(n), ctypes.byref(ms)))
        return int(n.value), float(ms.value)

    def fill_cache(self, n_pos, seed=0, scale=1.0):
        self._chk("mi_qwen2_fill_cache", _qlib().mi_qwen2_fill_cache(self.ptr, int(n_pos), int(seed), float(scale)))

    def get_cache(self, layer, is_v, n_pos):
        """fp16 bits [n_pos, n_head_kv*head_dim] of one layer's K or V cache"""
        out = np.empty((n_pos, self.hp["n_head_kv"] * self.hp["head_dim"]), np.uint16)
        self._chk("mi_qwen2_get_cache", _qlib().mi_qwen2_get_cache(self.ptr, int(layer), int(is_v), int(n_pos),
                                                                   out.ctypes.data, out.nbytes))
        return out

    def reset(self):
        self._chk("mi_qwen2_reset", _qlib().mi_qwen2_reset(self.ptr))

    def free(self):
        if self.ptr:
            _qlib().mi_qwen2_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
