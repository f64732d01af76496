"""ctypes wrapper of the CPU oracle (oracle/libggml_oracle.so).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, by __graft_entry__.smoke() as
the checker, and by bench.py's cpu_baseline leg; never by the product.

Array conventions (numpy):
  Q8_0 weights : uint8 [n_rows, K/32*34]  (ggml block_q8_0 bytes)
  Q4_0 weights : uint8 [n_rows, K/32*18]  (ggml block_q4_0 bytes)
  fp16 data    : uint16 bit patterns
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libggml_oracle.so")

Q8_ROUND_REF = 0
Q8_ROUND_X86 = 1

_lib = None


def build():
    """Compile the oracle with its Makefile (gcc)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F = ctypes.c_float
_I = ctypes.c_int
_SZ = ctypes.c_size_t


def _declare(L):
    sig = {
        "orc_fp32_to_fp16": (ctypes.c_uint16, [_F]),
        "orc_fp16_to_fp32": (_F, [ctypes.c_uint16]),
        "orc_fp32_to_fp16_row": (None, [_P, _P, _I64]),
        "orc_fp16_to_fp32_row": (None, [_P, _P, _I64]),
        "orc_quantize_row_q8_0": (None, [_P, _P, _P, _I64, _I]),
        "orc_dequantize_row_q8_0": (None, [_P, _P, _I64]),
        "orc_vec_dot_q8_0_q8_0": (_F, [_I64, _P, _P]),
        "orc_q8_0_block_dots": (None, [_P, _P, _I64, _I64, _P]),
        "orc_mul_mat_q8_0": (None, [_P, _P, _P, _P, _I64, _I64, _I]),
        "orc_mul_mat_q8_0_batch": (None, [_P, _P, _P, _P, _I64, _I64, _I64, _I]),
        "orc_quantize_weight_q8_0": (None, [_P, _P, _P, _I64, _I64]),
        "orc_dequantize_row_q4_0": (None, [_P, _P, _I64]),
        "orc_mul_mat_q4_0_f16": (None, [_P, _P, _P, _I64, _I64]),
        "orc_mul_mat_q4_0_f16_f64": (None, [_P, _P, _P, _I64, _I64]),
        "orc_mul_mat_f16": (None, [_P, _P, _P, _I64, _I64]),
        "orc_mul_mat_f16_f64": (None, [_P, _P, _P, _I64, _I64]),
        "orc_flash_attn_ext_1tok": (None, [_P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                           _SZ, _SZ, _SZ, _SZ, _F, _P, _I]),
        "orc_kv_lengths": (None, [_P, _I, _I64, _I64, _P]),
        "orc_quantize_a8w8_per_channel": (None, [_P, _I64, _I64, _P, _P]),
        "orc_quantize_per_token_i8": (None, [_P, _I64, _P, _P]),
        "orc_simd_isa": (ctypes.c_char_p, []),
        "orc_mul_mat_q8_0_mt": (None, [_P, _P, _P, _P, _I64, _I64, _I]),
        "orc_mul_mat_q4_0_f16_mt": (None, [_P, _P, _P, _I64, _I64, _I]),
        "orc_mul_mat_f16_mt": (None, [_P, _P, _P, _I64, _I64, _I]),
        "orc_flash_attn_ext_1tok_mt": (None, [_P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                              _SZ, _SZ, _SZ, _SZ, _F, _P, _I]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


# ---------------------------------------------------------------- fp16

def f32_to_f16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().orc_fp32_to_fp16_row(_p(x), _p(y), x.size)
    return y


def f16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib().orc_fp16_to_fp32_row(_p(h), _p(y), h.size)
    return y


# ---------------------------------------------------------------- Q8_0

def quantize_row_q8_0(x, inv_s=None, variant=Q8_ROUND_X86):
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.size
    assert k % 32 == 0
    y = np.empty(k // 32 * 34, dtype=np.uint8)
    s = None if inv_s is None else np.ascontiguousarray(inv_s, dtype=np.float32)
    lib().orc_quantize_row_q8_0(_p(x), _p(s), _p(y), k, variant)
    return y


def q8_0_block_dots(w, xq, n_rows, k):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.uint8)
    out = np.empty((n_rows, k // 32), dtype=np.int32)
    lib().orc_q8_0_block_dots(_p(w), _p(xq), n_rows, k, _p(out))
    return out


def vec_dot_q8_0(k, x, y):
    return lib().orc_vec_dot_q8_0_q8_0(k, _p(np.ascontiguousarray(x, np.uint8)), _p(np.ascontiguousarray(y, np.uint8)))


def mul_mat_q8_0(w, x, n_rows, k, inv_s=None, variant=Q8_ROUND_X86):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    s = None if inv_s is None else np.ascontiguousarray(inv_s, dtype=np.float32)
    m = x.size // k
    y = np.empty((m, n_rows), dtype=np.float32)
    lib().orc_mul_mat_q8_0_batch(_p(w), _p(x), _p(s), _p(y), n_rows, k, m, variant)
    return y.reshape(n_rows) if x.ndim == 1 else y


def mul_mat_q8_0_mt(w, x, n_rows, k, inv_s=None, n_threads=1):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    s = None if inv_s is None else np.ascontiguousarray(inv_s, dtype=np.float32)
    y = np.empty(n_rows, dtype=np.float32)
    lib().orc_mul_mat_q8_0_mt(_p(w), _p(x), _p(s), _p(y), n_rows, k, n_threads)
    return y


def quantize_weight_q8_0(w, s=None):
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    sv = None if s is None else np.ascontiguousarray(s, dtype=np.float32)
    y = np.empty((n, k // 32 * 34), dtype=np.uint8)
    lib().orc_quantize_weight_q8_0(_p(w), _p(sv), _p(y), n, k)
    return y


def dequantize_q8_0(w, k):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    n = w.size // (k // 32 * 34)
    y = np.empty((n, k), dtype=np.float32)
    lib().orc_dequantize_row_q8_0(_p(w), _p(y), n * k)
    return y


# ---------------------------------------------------------------- Q4_0

def dequantize_q4_0(w, k):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    n = w.size // (k // 32 * 18)
    y = np.empty((n, k), dtype=np.float32)
    lib().orc_dequantize_row_q4_0(_p(w), _p(y), n * k)
    return y


def mul_mat_q4_0_f16(w, x_f16, n_rows, k):
    y = np.empty(n_rows, dtype=np.float32)
    lib().orc_mul_mat_q4_0_f16(_p(np.ascontiguousarray(w, np.uint8)), _p(np.ascontiguousarray(x_f16, np.uint16)),
                               _p(y), n_rows, k)
    return y


def mul_mat_q4_0_f16_f64(w, x_f16, n_rows, k):
    y = np.empty(n_rows, dtype=np.float64)
    lib().orc_mul_mat_q4_0_f16_f64(_p(np.ascontiguousarray(w, np.uint8)),
                                   _p(np.ascontiguousarray(x_f16, np.uint16)), _p(y), n_rows, k)
    return y


def mul_mat_q4_0_f16_mt(w, x_f16, n_rows, k, n_threads=1):
    y = np.empty(n_rows, dtype=np.float32)
    lib().orc_mul_mat_q4_0_f16_mt(_p(np.ascontiguousarray(w, np.uint8)),
                                  _p(np.ascontiguousarray(x_f16, np.uint16)), _p(y), n_rows, k, n_threads)
    return y


# ---------------------------------------------------------------- F16

def mul_mat_f16(w_f16, x, n_rows, k):
    y = np.empty(n_rows, dtype=np.float32)
    lib().orc_mul_mat_f16(_p(np.ascontiguousarray(w_f16, np.uint16)), _p(np.ascontiguousarray(x, np.float32)),
                          _p(y), n_rows, k)
    return y


def mul_mat_f16_f64(w_f16, x, n_rows, k):
    y = np.empty(n_rows, dtype=np.float64)
    lib().orc_mul_mat_f16_f64(_p(np.ascontiguousarray(w_f16, np.uint16)), _p(np.ascontiguousarray(x, np.float32)),
                              _p(y), n_rows, k)
    return y


def mul_mat_f16_mt(w_f16, x, n_rows, k, n_threads=1):
    y = np.empty(n_rows, dtype=np.float32)
    lib().orc_mul_mat_f16_mt(_p(np.ascontiguousarray(w_f16, np.uint16)), _p(np.ascontiguousarray(x, np.float32)),
                             _p(y), n_rows, k, n_threads)
    return y


# ---------------------------------------------------------------- attention

def flash_attn_ext_1tok(q, k_cache, v_cache, n_kv_heads, scale, mask=None, kv_len=None, mode=0,
                        n_threads=None):
    """q: fp32 [nq, d]; k_cache/v_cache: uint16 [n_kv, n_kv_heads, d] (the ggml KV view layout
    ne=[d, n_kv, n_kv_heads] with nb1 = n_kv_heads*d*2, nb2 = d*2); mask: uint16 [>= n_kv] or None."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k_cache = np.ascontiguousarray(k_cache, dtype=np.uint16)
    v_cache = np.ascontiguousarray(v_cache, dtype=np.uint16)
    nq, d = q.shape
    n_kv = k_cache.shape[0]
    if kv_len is None:
        kv_len = n_kv
    nb1 = n_kv_heads * d * 2
    nb2 = d * 2
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint16)
    out = np.empty((nq, d), dtype=np.float32)
    if n_threads is None:
        lib().orc_flash_attn_ext_1tok(_p(q), _p(k_cache), _p(v_cache), _p(m), kv_len, nq, n_kv_heads, d,
                                      nb1, nb2, nb1, nb2, scale, _p(out), mode)
    else:
        lib().orc_flash_attn_ext_1tok_mt(_p(q), _p(k_cache), _p(v_cache), _p(m), kv_len, nq, n_kv_heads, d,
                                         nb1, nb2, nb1, nb2, scale, _p(out), n_threads)
    return out


def kv_lengths(mask, is_f16=True):
    mask = np.ascontiguousarray(mask)
    if mask.ndim == 1:
        mask = mask.reshape(1, -1)
    n_rows, n_kv = mask.shape
    out = np.empty(n_rows, dtype=np.int32)
    lib().orc_kv_lengths(_p(mask), 1 if is_f16 else 0, n_kv, n_rows, _p(out))
    return out


# ---------------------------------------------------------------- reference A8W8 scheme

def quantize_a8w8_per_channel(w_f16, k, n):
    q = np.zeros(k * n, dtype=np.int8)
    s = np.empty(n, dtype=np.uint16)
    lib().orc_quantize_a8w8_per_channel(_p(np.ascontiguousarray(w_f16, np.uint16)), k, n, _p(q), _p(s))
    return q, s


def quantize_per_token_i8(x_f16):
    x_f16 = np.ascontiguousarray(x_f16, dtype=np.uint16)
    xq = np.empty(x_f16.size, dtype=np.int8)
    s = np.empty(1, dtype=np.uint16)
    lib().orc_quantize_per_token_i8(_p(x_f16), x_f16.size, _p(xq), _p(s))
    return xq, s[0]


def simd_isa():
    return lib().orc_simd_isa().decode()


# ---------------------------------------------------------------- whole model (qwen2_oracle.c)

class _Layer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "attn_norm", "ffn_norm", "wq", "wk", "wv", "wo", "wgate", "wup", "wdown", "bq", "bk", "bv",
        "inv_s_attn", "inv_s_o", "inv_s_ffn", "inv_s_down")]


class _Model(ctypes.Structure):
    _fields_ = [("n_layer", ctypes.c_int), ("n_embd", ctypes.c_int), ("n_head", ctypes.c_int),
                ("n_head_kv", ctypes.c_int), ("head_dim", ctypes.c_int), ("n_ff", ctypes.c_int),
                ("n_vocab", ctypes.c_int), ("n_ctx", ctypes.c_int), ("rms_eps", ctypes.c_float),
                ("rope_theta", ctypes.c_float), ("wtype", ctypes.c_int), ("fa_mode", ctypes.c_int),
                ("n_threads", ctypes.c_int), ("tok_embd", ctypes.c_void_p), ("output_norm", ctypes.c_void_p),
                ("layers", ctypes.POINTER(_Layer)), ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p),
                ("q8_variant", ctypes.c_int), ("q8_generic", ctypes.c_int)]


class Qwen2:
    """CPU Qwen2 decode with ggml-CPU op semantics over a dict of ggml-format arrays
    (GGUF tensor names) and optional SmoothQuant factors per projection input."""

    def __init__(self, hp, tensors, smooth=None, fa_mode=0, n_threads=1, q8_variant=Q8_ROUND_X86, q8_generic=False):
        L = lib()
        if not hasattr(L, "_qwen2_declared"):
            L.orc_qwen2_decode.restype = ctypes.c_int
            L.orc_qwen2_decode.argtypes = [ctypes.POINTER(_Model), ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
            L._qwen2_declared = True
        self.hp = hp
        self._keep = []

        def ptr(a):
            if a is None:
                return None
            a = np.ascontiguousarray(a)
            self._keep.append(a)
            return a.ctypes.data

        nkv = hp["n_head_kv"] * hp["head_dim"]
        layers = (_Layer * hp["n_layer"])()
        smooth = smooth or {}
        for il in range(hp["n_layer"]):
            p = f"blk.{il}."
            inv = {}
            for key, wname in (("attn", "attn_q"), ("o", "attn_output"), ("ffn", "ffn_gate"), ("down", "ffn_down")):
                s = smooth.get(p + wname + ".weight")
                inv[key] = None if s is None else (np.float32(1.0) / np.asarray(s, np.float32)).astype(np.float32)
            lay = layers[il]
            lay.attn_norm = ptr(tensors[p + "attn_norm.weight"])
            lay.ffn_norm = ptr(tensors[p + "ffn_norm.weight"])
            for f, n in (("wq", "attn_q"), ("wk", "attn_k"), ("wv", "attn_v"), ("wo", "attn_output"),
                         ("wgate", "ffn_gate"), ("wup", "ffn_up"), ("wdown", "ffn_down")):
                setattr(lay, f, ptr(tensors[p + n + ".weight"]))
            for f, n in (("bq", "attn_q"), ("bk", "attn_k"), ("bv", "attn_v")):
                setattr(lay, f, ptr(tensors.get(p + n + ".bias")))
            lay.inv_s_attn, lay.inv_s_o = ptr(inv["attn"]), ptr(inv["o"])
            lay.inv_s_ffn, lay.inv_s_down = ptr(inv["ffn"]), ptr(inv["down"])
        self._layers = layers
        self.k_cache = np.zeros((hp["n_layer"], hp["n_ctx"], nkv), np.uint16)
        self.v_cache = np.zeros((hp["n_layer"], hp["n_ctx"], nkv), np.uint16)
        m = _Model()
        for f in ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_ff", "n_vocab", "n_ctx"):
            setattr(m, f, int(hp[f]))
        m.rms_eps, m.rope_theta = float(hp["rms_eps"]), float(hp["rope_theta"])
        m.wtype, m.fa_mode, m.n_threads = int(hp["wtype"]), int(fa_mode), int(n_threads)
        m.q8_variant, m.q8_generic = int(q8_variant), int(bool(q8_generic))
        m.tok_embd = ptr(tensors["token_embd.weight"])
        m.output_norm = ptr(tensors["output_norm.weight"])
        m.layers = layers
        m.k_cache, m.v_cache = self.k_cache.ctypes.data, self.v_cache.ctypes.data
        self._m = m
        self.logits = np.empty(hp["n_vocab"], np.float32)

    def decode(self, token, pos):
        """returns (argmax, logits copy)"""
        best = lib().orc_qwen2_decode(ctypes.byref(self._m), int(token), int(pos), self.logits.ctypes.data)
        return best, self.logits.copy()
