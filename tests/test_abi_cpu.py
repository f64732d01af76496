"""CPU-side checks of the C ABI library: it loads, exports every symbol that
include/ggml_mi355x_kernels.h declares, validates arguments before touching a
device, and its host prepack layouts round-trip byte for byte."""
import os
import re

import numpy as np
import pytest

from synth import q4_0_weights, q8_0_weights

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header):
    txt = open(os.path.join(ROOT, "include", header)).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", txt)))


def _declared_prefix(header, prefix):
    txt = open(os.path.join(ROOT, "include", header)).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(" + prefix + r"[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_declared_symbol(mi):
    L = mi.lib()
    declared = _declared("ggml_mi355x_kernels.h")
    assert declared, "header parse found no declarations"
    missing = [s for s in declared if not hasattr(L, s)]
    assert not missing, missing
    assert set(declared) <= set(mi.EXPORTED)
    for header, prefix in (("ggml-mi355x.h", "ggml_backend_mi355x_"), ("mi_qwen2.h", "mi_qwen2_")):
        syms = _declared_prefix(header, prefix)
        assert syms, header
        missing = [s for s in syms if not hasattr(L, s)]
        assert not missing, (header, missing)
    assert hasattr(L, "ggml_backend_is_mi355x")


def test_argument_validation_without_device(mi):
    with pytest.raises(mi.MiError) as e:
        mi.gemv_q8_0(0x1000, 0x1000, 0x1000, 16, 33)
    assert e.value.code == mi.MI_ERR_ARG
    with pytest.raises(mi.MiError) as e:
        mi.gemv_q8_0(0x1001, 0x1000, 0x1000, 16, 64)  # packed weight must be 256-byte aligned
    assert e.value.code == mi.MI_ERR_ARG
    with pytest.raises(mi.MiError) as e:
        mi.fa_decode(0x1000, 0x1000, 0x1000, None, None, 64, 12, 2, 96, 512, 256, 512, 256, 0.1, 0x1000, 0, 0)
    assert e.value.code == mi.MI_ERR_ARG  # head dim 96 unsupported
    with pytest.raises(mi.MiError) as e:
        mi.fa_decode(0x1000, 0x1000, 0x1000, None, None, 64, 12, 5, 128, 512, 256, 512, 256, 0.1, 0x1000, 0, 0)
    assert e.value.code == mi.MI_ERR_ARG  # 12 % 5 != 0
    with pytest.raises(mi.MiError) as e:
        mi.fa_decode(0x1000, 0x1000, 0x1000, None, None, 64, 12, 2, 128, 520, 256, 512, 256, 0.1, 0x1000, 0, 0)
    assert e.value.code == mi.MI_ERR_ARG  # stride not 16-byte aligned
    with pytest.raises(mi.MiError) as e:
        mi.gemv_f16(0x1000, 100, 0x1000, 0x1000, 16, 128)  # ldw < k
    assert e.value.code == mi.MI_ERR_ARG


def test_fa_workspace_size_is_monotone(mi):
    sizes = [mi.fa_decode_workspace_size(L, 12, 2, 128) for L in (64, 512, 4096, 32768)]
    assert all(s % 16 == 0 for s in sizes)
    assert sizes == sorted(sizes)


@pytest.mark.parametrize("n,k", [(1, 32), (7, 96), (256, 1536), (33, 8960)])
def test_q8_0_prepack_roundtrip(mi, n, k):
    w = q8_0_weights(np.random.default_rng(n), n, k)
    packed = mi.prepack_q8_0_host(w, n, k)
    assert packed.size == mi.q8_0_packed_size(n, k)
    assert packed.size % 256 == 0
    assert np.array_equal(mi.unpack_q8_0_host(packed, n, k), w)
    # the planes hold exactly the ggml bytes: qs[0:16] | qs[16:32] | d
    nb = k // 32
    plane = (n * nb * 16 + 255) // 256 * 256
    b = w.reshape(n * nb, 34)
    assert np.array_equal(packed[: n * nb * 16].reshape(-1, 16), b[:, 2:18])
    assert np.array_equal(packed[plane: plane + n * nb * 16].reshape(-1, 16), b[:, 18:34])
    assert np.array_equal(packed[2 * plane: 2 * plane + n * nb * 2].reshape(-1, 2), b[:, 0:2])


@pytest.mark.parametrize("n,k", [(1, 32), (5, 64), (1536, 8960)])
def test_q4_0_prepack_roundtrip(mi, n, k):
    w = q4_0_weights(np.random.default_rng(n), n, k)
    packed = mi.prepack_q4_0_host(w, n, k)
    assert packed.size == mi.q4_0_packed_size(n, k)
    assert np.array_equal(mi.unpack_q4_0_host(packed, n, k), w)


def test_smooth_factors_refuse_a_foreign_weight(mi):
    """A Q8_0 weight in another backend's buffer whose extra holds that backend's data (as
    the CPU repack buffer types do) is not this backend's: no factors, nothing written."""
    import ctypes

    import ggml_api as ga
    ctx = ga.Context(mi.lib())
    L = ctx.L
    w = ctx.tensor(ga.GGML_TYPE_Q8_0, 64, 16, name="blk.0.ffn_up.weight")
    ctx.alloc(L.ggml_backend_cpu_buffer_type())
    foreign = ctypes.create_string_buffer(b"\x5a" * 64)
    w.contents.extra = ctypes.addressof(foreign)
    s = np.full(64, 2.0, np.float32)
    assert not L.ggml_backend_mi355x_set_smooth_factors(w, s.ctypes.data, 64)
    assert foreign.raw[:64] == b"\x5a" * 64
    ctx.free()
