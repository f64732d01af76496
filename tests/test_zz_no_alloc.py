"""mi_fa_decode_noalloc, the flash-decoding entry point that allocates nothing (its split
partials live in the library's per-device scratch array), against mi_fa_decode with a
caller workspace: bit-identical outputs on two calls in a row, the second smaller, so the
scratch's leftovers from the first call cannot leak into the second."""
import numpy as np
import pytest

from synth import f16_bits

pytestmark = pytest.mark.gpu


def _inputs(rng, L, nq, nkv, d):
    q = rng.standard_normal((nq, d)).astype(np.float32)
    kc = f16_bits(rng.standard_normal((L, nkv, d)))
    vc = f16_bits(rng.standard_normal((L, nkv, d)))
    return q, kc, vc


def _both(mi, q, kc, vc, nkv, mask=None, kv_len=None):
    nq, d = q.shape
    L = kc.shape[0]
    dq, dk, dv = mi.to_device(q), mi.to_device(kc), mi.to_device(vc)
    dm = mi.to_device(mask) if mask is not None else None
    dl = mi.to_device(np.array([kv_len], np.int32)) if kv_len is not None else None
    nb1, nb2 = nkv * d * 2, d * 2
    scale = 1 / np.sqrt(d)
    a, b = mi.DeviceBuffer(nq * d * 4), mi.DeviceBuffer(nq * d * 4)
    wsb = mi.fa_decode_workspace_size(L, nq, nkv, d)
    ws = mi.DeviceBuffer(wsb).zero()
    mi.fa_decode(dq.ptr, dk.ptr, dv.ptr, dm.ptr if dm else None, dl.ptr if dl else None, L, nq, nkv, d, nb1, nb2,
                 nb1, nb2, scale, a.ptr, ws.ptr, wsb)
    mi.fa_decode_noalloc(dq.ptr, dk.ptr, dv.ptr, dm.ptr if dm else None, dl.ptr if dl else None, L, nq, nkv, d,
                         nb1, nb2, nb1, nb2, scale, b.ptr)
    mi.device_sync()
    return a.download(np.float32).reshape(nq, d), b.download(np.float32).reshape(nq, d), wsb


def test_noalloc_matches_workspace_entry_point_twice(gpu, orc):
    mi = gpu
    rng = np.random.default_rng(4242)
    cap = mi.lib().mi_fa_decode_noalloc_max_workspace()
    assert cap == 4 << 20
    # first call: 12q/2kv at 5000 positions (79 splits); second: a smaller one (700 positions,
    # 28q/4kv) that reuses a prefix of the scratch the first call filled
    for L, nq, nkv in ((5000, 12, 2), (700, 28, 4)):
        q, kc, vc = _inputs(rng, L, nq, nkv, 128)
        ref, got, wsb = _both(mi, q, kc, vc, nkv)
        assert 0 < wsb <= cap
        assert np.array_equal(ref, got), f"L={L}"
        exact = orc.flash_attn_ext_1tok(q, kc, vc, nkv, 1 / np.sqrt(128), mode=1)
        assert float(np.abs(got - exact).max()) < 5e-5
    # a masked call with a kv_lengths input through the same scratch
    L = 3000
    q, kc, vc = _inputs(rng, L, 12, 2, 128)
    mask = np.zeros(L, np.float32)
    mask[2100:] = -np.inf
    ref, got, _ = _both(mi, q, kc, vc, 2, mask=f16_bits(mask), kv_len=2100)
    assert np.array_equal(ref, got)


def test_noalloc_refuses_more_than_its_scratch(gpu):
    """a request whose partials exceed the scratch fails before any launch, with the sizes"""
    mi = gpu
    L, nq, nkv, d = 1 << 20, 28, 4, 128
    assert mi.fa_decode_workspace_size(L, nq, nkv, d) > mi.lib().mi_fa_decode_noalloc_max_workspace()
    with pytest.raises(mi.MiError) as e:
        mi.fa_decode_noalloc(0x1000, 0x1000, 0x1000, None, None, L, nq, nkv, d, nkv * d * 2, d * 2, nkv * d * 2, d * 2,
                             0.088, 0x1000)
    assert e.value.code == mi.MI_ERR_WORKSPACE and "scratch" in str(e.value)
