"""GPU parity of the decode-graph glue kernels and of the fused decode chains, called
through the C ABI, against numpy restatements of the ggml-CPU ops (ggml/src/ggml-cpu/ops.cpp
of llama.cpp @ 37b3a9e0) composed with the oracle's Q8_0 matmul.

Bars: RMSNorm within 1 ulp (the double sum's order differs); RoPE within 2e-6 relative
(device cosf/sinf against the host's); ARGMAX exact (first maximum); SwiGLU+quantize
with Q8_0 scales exact and at most one int8 step on <0.1% of the elements (device expf
is not the host's); fused GEMV chains within the GEMV bar (1e-3 relative); fp16 cache
rows within 2 fp16 ulps of the reference; cache rows other than the target untouched.
"""
import numpy as np
import pytest

from synth import f16_bits, q4_0_weights, q8_0_weights, rel_err, xq_to_blocks

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3
F32 = np.float32


def rms_norm_ref(x, w, eps):
    """ggml rms_norm then mul: (float)(sum of (double)(x*x) / n), y = (x * scale) * w"""
    x = np.asarray(x, F32)
    sq = (x * x).astype(np.float64)
    mean = F32(np.sum(sq) / x.size)
    scale = F32(1.0) / np.sqrt(F32(mean + F32(eps)))
    y = (x * scale).astype(F32)
    return (y * w).astype(F32) if w is not None else y


def _powf(a, b):
    """the C library powf, as the host code forms theta_scale"""
    import ctypes
    libm = ctypes.CDLL("libm.so.6")
    libm.powf.restype = ctypes.c_float
    libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    return F32(libm.powf(F32(a), F32(b)))


def rope_neox_ref(x, pos, hd, base):
    """x [heads, hd] fp32; theta_i = pos * theta_scale^i by repeated float multiplication"""
    ts = _powf(base, F32(-2.0) / F32(hd))
    th = np.empty(hd // 2, F32)
    t = F32(pos)
    for i in range(hd // 2):
        th[i] = t
        t = F32(t * ts)
    c = np.cos(th.astype(np.float64)).astype(F32)
    s = np.sin(th.astype(np.float64)).astype(F32)
    x0, x1 = x[:, : hd // 2], x[:, hd // 2:]
    return np.concatenate([(x0 * c - x1 * s).astype(F32), (x0 * s + x1 * c).astype(F32)], axis=1)


def _packed_q8(mi, w, n, k):
    src = mi.to_device(w)
    dst = mi.DeviceBuffer(mi.q8_0_packed_size(n, k)).zero()
    mi.prepack_q8_0(src.ptr, dst.ptr, n, k)
    mi.device_sync()
    src.free()
    return dst


def _ptrs(*bufs):
    import ctypes
    return (ctypes.c_void_p * len(bufs))(*[b.ptr if b is not None else None for b in bufs])


def _i64s(*v):
    import ctypes
    return (ctypes.c_int64 * len(v))(*v)


def ulp_diff(a, b):
    ai = np.asarray(a, F32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, F32).view(np.int32).astype(np.int64)
    return np.abs(ai - bi)


# ---------------------------------------------------------------- glue kernels

@pytest.mark.parametrize("ne0,nrows", [(1536, 1), (3584, 2), (96, 3)])
def test_rms_norm(gpu, ne0, nrows):
    mi = gpu
    rng = np.random.default_rng(ne0)
    x = (rng.standard_normal((nrows, ne0)) * 0.3).astype(F32)
    w = rng.uniform(0.8, 1.2, ne0).astype(F32)
    dx, dw, dy = mi.to_device(x), mi.to_device(w), mi.DeviceBuffer(x.nbytes)
    mi._call("mi_rms_norm", None, mi._P(dx.ptr), mi._P(dw.ptr), mi._P(dy.ptr), ne0, nrows, F32(1e-6))
    mi.device_sync()
    y = dy.download(F32).reshape(nrows, ne0)
    for r in range(nrows):
        assert ulp_diff(y[r], rms_norm_ref(x[r], w, 1e-6)).max() <= 1


@pytest.mark.parametrize("hd,heads,pos", [(128, 12, 0), (128, 2, 517), (64, 4, 32767)])
def test_rope_neox(gpu, hd, heads, pos):
    mi = gpu
    rng = np.random.default_rng(pos + hd)
    x = rng.standard_normal((heads, hd)).astype(F32)
    dx, dy = mi.to_device(x), mi.DeviceBuffer(x.nbytes)
    dp = mi.to_device(np.array([pos], np.int32))
    mi._call("mi_rope_neox", None, mi._P(dx.ptr), mi._P(dy.ptr), mi._P(dp.ptr), hd, heads, 1, hd, F32(1e6), F32(1.0),
             F32(1.0), hd * 4, hd * heads * 4, hd * 4, hd * heads * 4)
    mi.device_sync()
    y = dy.download(F32).reshape(heads, hd)
    ref = rope_neox_ref(x, pos, hd, 1e6)
    assert rel_err(y, ref) < 2e-6


def _rope_table(mi, dpos, hd, base, freq_scale=1.0, attn_factor=1.0):
    tab = mi.DeviceBuffer(4 * hd)
    mi._call("mi_rope_table", None, mi._P(dpos.ptr), hd, F32(base), F32(freq_scale), F32(attn_factor),
             mi._P(tab.ptr))
    return tab


@pytest.mark.parametrize("hd,pos,base,fs,af", [(128, 0, 1e6, 1.0, 1.0), (128, 32767, 1e6, 1.0, 1.0),
                                               (64, 517, 1e4, 0.5, 1.1), (1024, 77, 1e6, 1.0, 1.0)])
def test_rope_table(gpu, hd, pos, base, fs, af):
    """cos/sin of theta_p = freq_scale * (pos * theta_scale^p), the power by repeated float
    multiplication; within 2 ulps of the host's double-precision cos/sin of the same angle"""
    mi = gpu
    dpos = mi.to_device(np.array([pos], np.int32))
    tab = _rope_table(mi, dpos, hd, base, fs, af)
    mi.device_sync()
    got = tab.download(F32).reshape(2, hd // 2)
    ts = _powf(base, F32(-2.0) / F32(hd))
    th = np.empty(hd // 2, F32)
    t = F32(pos)
    for i in range(hd // 2):
        th[i] = F32(F32(fs) * t)
        t = F32(t * ts)
    ref_c = (np.cos(th.astype(np.float64)).astype(F32) * F32(af)).astype(F32)
    ref_s = (np.sin(th.astype(np.float64)).astype(F32) * F32(af)).astype(F32)
    tol = 2 * np.spacing(np.float32(1.0)) * af + 1e-7
    assert np.max(np.abs(got[0] - ref_c)) <= tol and np.max(np.abs(got[1] - ref_s)) <= tol


@pytest.mark.parametrize("idx_i64", [False, True])
@pytest.mark.parametrize("m,hd,nhq,nhk,nv", [(8, 128, 28, 4, 512), (3, 64, 4, 2, 128), (1, 128, 12, 2, 256)])
def test_rope_kv_rows(gpu, m, hd, nhq, nhk, nv, idx_i64):
    """ROPE q, ROPE k, SET_ROWS k, SET_ROWS v of a ubatch in one launch: bit-identical to
    mi_rope_neox + mi_set_rows_f16, within 2e-6 of the host rotation; a cache index outside
    the cache is skipped and no other cache row changes."""
    mi = gpu
    P = mi._P
    rng = np.random.default_rng(m * 1000 + hd + nhq + idx_i64)
    n_rows_cache = 64
    q = rng.standard_normal((m, nhq * hd)).astype(F32)
    k = rng.standard_normal((m, nhk * hd)).astype(F32)
    v = rng.standard_normal((m, nv)).astype(F32)
    pos = rng.integers(0, 40000, m).astype(np.int32)
    idx = rng.permutation(n_rows_cache)[:m].astype(np.int64 if idx_i64 else np.int32)
    if m > 2:
        idx[1] = n_rows_cache + 5  # outside the cache: not written
    kc0 = f16_bits(rng.standard_normal((n_rows_cache, nhk * hd)))
    vc0 = f16_bits(rng.standard_normal((n_rows_cache, nv)))
    dq, dk, dv, dp, di = (mi.to_device(a) for a in (q, k, v, pos, idx))
    dkc, dvc = mi.to_device(kc0), mi.to_device(vc0)
    dqo = mi.DeviceBuffer(q.nbytes)
    mi._call("mi_rope_kv_rows", None, P(dq.ptr), P(dk.ptr), P(dv.ptr), P(dqo.ptr), P(dkc.ptr), nhk * hd * 2,
             P(dvc.ptr), nv * 2, P(dp.ptr), P(di.ptr), int(idx_i64), n_rows_cache, m, hd, nhq, nhk, nv, F32(1e6),
             F32(1.0), F32(1.0))
    # node-by-node on the device
    dq2, dk2 = mi.DeviceBuffer(q.nbytes), mi.DeviceBuffer(k.nbytes)
    dkc2, dvc2 = mi.to_device(kc0), mi.to_device(vc0)
    for src, dst, nh in ((dq, dq2, nhq), (dk, dk2, nhk)):
        mi._call("mi_rope_neox", None, P(src.ptr), P(dst.ptr), P(dp.ptr), hd, nh, m, hd, F32(1e6), F32(1.0), F32(1.0),
                 hd * 4, nh * hd * 4, hd * 4, nh * hd * 4)
    mi._call("mi_set_rows_f16", None, P(dk2.ptr), P(di.ptr), int(idx_i64), P(dkc2.ptr), nhk * hd, m, nhk * hd * 4,
             nhk * hd * 2, n_rows_cache)
    mi._call("mi_set_rows_f16", None, P(dv.ptr), P(di.ptr), int(idx_i64), P(dvc2.ptr), nv, m, nv * 4, nv * 2,
             n_rows_cache)
    mi.device_sync()
    qo, kc, vc = dqo.download(F32).reshape(m, -1), dkc.download(np.uint16).reshape(n_rows_cache, -1), \
        dvc.download(np.uint16).reshape(n_rows_cache, -1)
    assert np.array_equal(qo, dq2.download(F32).reshape(m, -1))
    assert np.array_equal(kc, dkc2.download(np.uint16).reshape(n_rows_cache, -1))
    assert np.array_equal(vc, dvc2.download(np.uint16).reshape(n_rows_cache, -1))
    written = [int(i) for i in idx if 0 <= i < n_rows_cache]
    untouched = [r for r in range(n_rows_cache) if r not in written]
    assert np.array_equal(kc[untouched], kc0[untouched]) and np.array_equal(vc[untouched], vc0[untouched])
    for r in range(m):
        ref_q = rope_neox_ref(q[r].reshape(nhq, hd), int(pos[r]), hd, 1e6).reshape(-1)
        assert rel_err(qo[r], ref_q) < 2e-6
        if 0 <= idx[r] < n_rows_cache:
            ref_k = rope_neox_ref(k[r].reshape(nhk, hd), int(pos[r]), hd, 1e6).reshape(-1)
            kf = kc[idx[r]].view(np.float16).astype(F32)
            assert np.max(np.abs(kf - ref_k) / np.maximum(np.abs(ref_k), 1e-3)) < 2e-3
            assert np.array_equal(vc[idx[r]], f16_bits(v[r]))


@pytest.mark.parametrize("ne0,nrows", [(151936, 1), (1000, 3), (2049, 2), (4096 * 300 + 7, 1)])
def test_argmax_first_maximum(gpu, ne0, nrows):
    mi = gpu
    rng = np.random.default_rng(ne0 + nrows)
    x = rng.standard_normal((nrows, ne0)).astype(F32)
    if nrows >= 2:
        x[1, :] = -np.inf                      # all -inf: index 0
    x[0, ne0 // 3] = 50.0                      # tie of the maximum: the lower index wins
    x[0, ne0 - 1] = 50.0
    x[0, 5] = np.nan                           # NaN is never the maximum
    if nrows >= 3:
        x[2, 0] = 99.0                         # maximum at the first element
    ws_bytes = mi.lib().mi_argmax_workspace_size(ne0, nrows)
    dx, do, dws = mi.to_device(x), mi.DeviceBuffer(4 * nrows), mi.DeviceBuffer(ws_bytes)
    mi._call("mi_argmax", None, mi._P(dx.ptr), mi._P(do.ptr), ne0, nrows, mi._P(dws.ptr), ws_bytes)
    mi.device_sync()
    got = do.download(np.int32)
    ref = [int(np.argmax(np.where(np.isnan(r), -np.inf, r))) for r in x]
    assert list(got) == ref


def test_argmax_rejects_small_workspace(gpu):
    mi = gpu
    dx, do = mi.DeviceBuffer(4 * 5000), mi.DeviceBuffer(4)
    with pytest.raises(mi.MiError):
        mi._call("mi_argmax", None, mi._P(dx.ptr), mi._P(do.ptr), 5000, 1, None, 0)


# ---------------------------------------------------------------- fused chains

def _q8_ref(orc, blocks, x, n, k, inv):
    return orc.mul_mat_q8_0(blocks, x, n, k, inv_s=inv, variant=orc.Q8_ROUND_X86)


@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("ns,k", [((8960, 8960), 1536), ((1536,), 1536), ((3584, 512, 512), 3584)])
def test_fused_norm_matmuls_add(gpu, orc, norm, ns, k):
    mi = gpu
    rng = np.random.default_rng(sum(ns) + k + norm)
    x = (rng.standard_normal(k) * 0.5).astype(F32)
    nw = rng.uniform(0.8, 1.2, k).astype(F32)
    inv = (1.0 / rng.uniform(0.5, 2.0, k)).astype(F32)
    ws = [q8_0_weights(rng, n, k) for n in ns]
    adds = [rng.standard_normal(n).astype(F32) if i % 2 == 0 else None for i, n in enumerate(ns)]
    pw = [_packed_q8(mi, w, n, k) for w, n in zip(ws, ns)]
    ys = [mi.DeviceBuffer(4 * n) for n in ns]
    da = [mi.to_device(a) if a is not None else None for a in adds]
    dx, dnw, dinv = mi.to_device(x), mi.to_device(nw), mi.to_device(inv)
    mi._call("mi_mul_mat_q8_0_f32_fused", None, len(ns), _ptrs(*pw), _i64s(*ns), _ptrs(*ys), _ptrs(*da), k,
             mi._P(dx.ptr), mi._P(dnw.ptr if norm else None), F32(1e-6), mi._P(dinv.ptr), mi.Q8_ROUND_X86)
    mi.device_sync()
    xin = rms_norm_ref(x, nw, 1e-6) if norm else x
    for i, n in enumerate(ns):
        ref = _q8_ref(orc, ws[i], xin, n, k, inv)
        if adds[i] is not None:
            ref = (ref + adds[i]).astype(F32)
        assert rel_err(ys[i].download(F32), ref) < GEMV_TOL, f"matrix {i}"


@pytest.mark.parametrize("table", [False, True])
@pytest.mark.parametrize("idx_i64", [False, True])
@pytest.mark.parametrize("cfg", [dict(k=1536, hq=12, hkv=2, hd=128, pos=517, row=517, bias=True),
                                 dict(k=3584, hq=28, hkv=4, hd=128, pos=3, row=9, bias=True),
                                 dict(k=256, hq=4, hkv=2, hd=64, pos=0, row=0, bias=False),
                                 dict(k=512, hq=64, hkv=8, hd=128, pos=40, row=1, bias=True)])
def test_qkv_rope_kv(gpu, orc, cfg, idx_i64, table):
    """the shapes cover 64, 32 and 16 lanes per row (the launch picks the width from the row count);
    the angles formed in the launch or read from mi_rope_table"""
    mi = gpu
    k, hq, hkv, hd = cfg["k"], cfg["hq"], cfg["hkv"], cfg["hd"]
    nq, nkv = hq * hd, hkv * hd
    n_cache = 640
    rng = np.random.default_rng(k + hq + cfg["pos"] + idx_i64)
    x = (rng.standard_normal(k) * 0.5).astype(F32)
    nw = rng.uniform(0.8, 1.2, k).astype(F32)
    inv = (1.0 / rng.uniform(0.5, 2.0, k)).astype(F32)
    ns = (nq, nkv, nkv)
    ws = [q8_0_weights(rng, n, k) for n in ns]
    bs = [(rng.standard_normal(n) * 0.02).astype(F32) if cfg["bias"] else None for n in ns]
    pw = [_packed_q8(mi, w, n, k) for w, n in zip(ws, ns)]
    db = [mi.to_device(b) if b is not None else None for b in bs]
    dx, dnw, dinv = mi.to_device(x), mi.to_device(nw), mi.to_device(inv)
    dq = mi.DeviceBuffer(4 * nq)
    kc = mi.DeviceBuffer(n_cache * nkv * 2).zero()
    vc = mi.DeviceBuffer(n_cache * nkv * 2).zero()
    dpos = mi.to_device(np.array([cfg["pos"]], np.int32))
    didx = mi.to_device(np.array([cfg["row"]], np.int64 if idx_i64 else np.int32))
    tab = _rope_table(mi, dpos, hd, 1e6) if table else None
    mi._call("mi_qkv_rope_kv_q8_0", None, _ptrs(*pw), _i64s(*ns), _ptrs(*db), k, mi._P(dx.ptr), mi._P(dnw.ptr),
             F32(1e-6), mi._P(dinv.ptr), mi.Q8_ROUND_X86, hd, mi._P(dpos.ptr), F32(1e6), F32(1.0), F32(1.0),
             mi._P(dq.ptr), mi._P(kc.ptr), nkv * 2, mi._P(vc.ptr), nkv * 2, mi._P(didx.ptr), int(idx_i64), n_cache,
             mi._P(tab.ptr if tab is not None else None))
    mi.device_sync()
    xn = rms_norm_ref(x, nw, 1e-6)
    proj = []
    for i, n in enumerate(ns):
        y = _q8_ref(orc, ws[i], xn, n, k, inv)
        proj.append((y + bs[i]).astype(F32) if bs[i] is not None else y)
    q_ref = rope_neox_ref(proj[0].reshape(hq, hd), cfg["pos"], hd, 1e6).reshape(-1)
    k_ref = rope_neox_ref(proj[1].reshape(hkv, hd), cfg["pos"], hd, 1e6).reshape(-1)
    assert rel_err(dq.download(F32), q_ref) < GEMV_TOL
    kcache = kc.download(np.uint16).reshape(n_cache, nkv)
    vcache = vc.download(np.uint16).reshape(n_cache, nkv)
    for name, cache, ref in (("k", kcache, k_ref), ("v", vcache, proj[2])):
        got = cache[cfg["row"]].view(np.float16).astype(np.float64)
        tol = 2 * np.abs(ref.astype(np.float16).astype(np.float64)) * 2.0 ** -10 + 1e-7
        assert np.all(np.abs(got - ref) <= tol + GEMV_TOL * np.sqrt(np.mean(ref.astype(np.float64) ** 2))), name
        others = np.delete(cache, cfg["row"], axis=0)
        assert not others.any(), f"{name} cache rows other than {cfg['row']} were written"


def test_qkv_rope_kv_skips_out_of_range_row(gpu):
    mi = gpu
    rng = np.random.default_rng(7)
    k, hd, ns = 256, 64, (256, 128, 128)
    ws = [q8_0_weights(rng, n, k) for n in ns]
    pw = [_packed_q8(mi, w, n, k) for w, n in zip(ws, ns)]
    dx = mi.to_device(rng.standard_normal(k).astype(F32))
    dq = mi.DeviceBuffer(4 * ns[0])
    kc = mi.DeviceBuffer(8 * 128 * 2).zero()
    vc = mi.DeviceBuffer(8 * 128 * 2).zero()
    dpos = mi.to_device(np.array([3], np.int32))
    didx = mi.to_device(np.array([8], np.int32))   # one past the last cache row
    mi._call("mi_qkv_rope_kv_q8_0", None, _ptrs(*pw), _i64s(*ns), _ptrs(None, None, None), k, mi._P(dx.ptr), None,
             F32(1e-6), None, mi.Q8_ROUND_X86, hd, mi._P(dpos.ptr), F32(1e4), F32(1.0), F32(1.0), mi._P(dq.ptr),
             mi._P(kc.ptr), 256, mi._P(vc.ptr), 256, mi._P(didx.ptr), 0, 8, None)
    mi.device_sync()
    assert not kc.download(np.uint16).any() and not vc.download(np.uint16).any()


@pytest.mark.parametrize("k", [8960, 18944, 512])
def test_swiglu_quant(gpu, orc, k):
    mi = gpu
    rng = np.random.default_rng(k)
    g = (rng.standard_normal(k) * 2).astype(F32)
    u = rng.standard_normal(k).astype(F32)
    inv = (1.0 / rng.uniform(0.5, 2.0, k)).astype(F32)
    dg, du, dinv = mi.to_device(g), mi.to_device(u), mi.to_device(inv)
    dq = mi.DeviceBuffer(mi.xq_size(1, k))
    mi._call("mi_swiglu_quant_q8_0", None, mi._P(dg.ptr), mi._P(du.ptr), mi._P(dinv.ptr), k, mi._P(dq.ptr),
             mi.Q8_ROUND_X86)
    mi.device_sync()
    silu = (g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))).astype(F32)
    v = (silu * u).astype(F32)
    ref = orc.quantize_row_q8_0(v, inv_s=inv, variant=orc.Q8_ROUND_X86).reshape(k // 32, 34)
    qs = dq.download(np.int8, k)
    d = dq.download(np.uint16, k // 32, offset=mi.xq_d_offset(1, k))
    got = xq_to_blocks(qs, d, k).reshape(k // 32, 34)
    d_same = np.mean(np.all(got[:, :2] == ref[:, :2], axis=1))
    dq_ = np.abs(got[:, 2:].view(np.int8).astype(int) - ref[:, 2:].view(np.int8).astype(int))
    assert d_same >= 0.99 and dq_.max() <= 1 and np.mean(dq_ > 0) < 1e-3


@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("nff,k", [(8960, 1536), (4864, 896), (11008, 2048), (512, 256)])
def test_gate_up_swiglu_q8_0(gpu, orc, nff, k, norm):
    """Normed gate+up with the swiglu and the down projection's activation quantization in
    the epilogue: the quantized activation is byte-identical to the fused gate/up GEMV
    followed by the swiglu-quantize kernel, and its blocks follow the oracle's quantizer
    of the oracle's gate/up (scales exact on >= 99% of blocks, int8 within one step)."""
    mi = gpu
    P = mi._P
    rng = np.random.default_rng(nff + k + norm)
    x = (rng.standard_normal(k) * 0.5).astype(F32)
    nw = rng.uniform(0.8, 1.2, k).astype(F32)
    inv = (1.0 / rng.uniform(0.5, 2.0, k)).astype(F32)
    inv_d = (1.0 / rng.uniform(0.5, 2.0, nff)).astype(F32)
    wg, wu = q8_0_weights(rng, nff, k), q8_0_weights(rng, nff, k)
    pg, pu = _packed_q8(mi, wg, nff, k), _packed_q8(mi, wu, nff, k)
    dx, dnw, dinv, dinvd = mi.to_device(x), mi.to_device(nw), mi.to_device(inv), mi.to_device(inv_d)
    xq = mi.DeviceBuffer(mi.xq_size(1, nff))
    mi._call("mi_gate_up_swiglu_q8_0", None, P(pg.ptr), P(pu.ptr), nff, k, P(dx.ptr), P(dnw.ptr if norm else None),
             F32(1e-6), P(dinv.ptr), P(dinvd.ptr), mi.Q8_ROUND_X86, P(xq.ptr))
    yg, yu = mi.DeviceBuffer(4 * nff), mi.DeviceBuffer(4 * nff)
    mi._call("mi_mul_mat_q8_0_f32_fused", None, 2, _ptrs(pg, pu), _i64s(nff, nff), _ptrs(yg, yu), None, k,
             P(dx.ptr), P(dnw.ptr if norm else None), F32(1e-6), P(dinv.ptr), mi.Q8_ROUND_X86)
    xq2 = mi.DeviceBuffer(mi.xq_size(1, nff))
    mi._call("mi_swiglu_quant_q8_0", None, P(yg.ptr), P(yu.ptr), P(dinvd.ptr), nff, P(xq2.ptr), mi.Q8_ROUND_X86)
    mi.device_sync()
    doff = mi.xq_d_offset(1, nff)
    qs, d = xq.download(np.int8, nff), xq.download(np.uint16, nff // 32, offset=doff)
    assert np.array_equal(qs, xq2.download(np.int8, nff))
    assert np.array_equal(d, xq2.download(np.uint16, nff // 32, offset=doff))
    xin = rms_norm_ref(x, nw, 1e-6) if norm else x
    g = _q8_ref(orc, wg, xin, nff, k, inv)
    u = _q8_ref(orc, wu, xin, nff, k, inv)
    v = ((g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))).astype(F32) * u).astype(F32)
    ref = orc.quantize_row_q8_0(v, inv_s=inv_d, variant=orc.Q8_ROUND_X86).reshape(nff // 32, 34)
    got = xq_to_blocks(qs, d, nff).reshape(nff // 32, 34)
    d_same = np.mean(np.all(got[:, :2] == ref[:, :2], axis=1))
    dq_ = np.abs(got[:, 2:].view(np.int8).astype(int) - ref[:, 2:].view(np.int8).astype(int))
    assert d_same >= 0.99 and dq_.max() <= 1 and np.mean(dq_ > 0) < 1e-2


@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("nff,k", [(8960, 1536), (4864, 896), (11008, 2048), (512, 256)])
def test_gate_up_pair_then_down_q8_0(gpu, orc, nff, k, norm):
    """The two-launch FFN forms: gate/up rows paired per workgroup with the swiglu (times
    the down divisor) kept in fp32, then the down projection quantizing it in its prologue
    (+ residual); and the pair launch quantizing each 32-block in the last of its four
    workgroups.  Bit-identical to the three launches they replace (fused gate/up GEMV,
    swiglu-quantize, down GEMV + residual), and within the GEMV bar of the oracle's
    gate/up -> swiglu -> quantized down."""
    mi = gpu
    P = mi._P
    rng = np.random.default_rng(nff + 3 * k + norm)
    n = k  # the down projection maps back to the embedding width
    x = (rng.standard_normal(k) * 0.5).astype(F32)
    nw = rng.uniform(0.8, 1.2, k).astype(F32)
    inv = (1.0 / rng.uniform(0.5, 2.0, k)).astype(F32)
    inv_d = (1.0 / rng.uniform(0.5, 2.0, nff)).astype(F32)
    wg, wu, wd = q8_0_weights(rng, nff, k), q8_0_weights(rng, nff, k), q8_0_weights(rng, n, nff)
    pg, pu, pd = _packed_q8(mi, wg, nff, k), _packed_q8(mi, wu, nff, k), _packed_q8(mi, wd, n, nff)
    res = rng.standard_normal(n).astype(F32)
    dx, dnw, dinv, dinvd, dres = (mi.to_device(a) for a in (x, nw, inv, inv_d, res))
    h = mi.DeviceBuffer(4 * nff)
    y = mi.DeviceBuffer(4 * n)
    mi._call("mi_gate_up_swiglu_f32_q8_0", None, P(pg.ptr), P(pu.ptr), nff, k, P(dx.ptr),
             P(dnw.ptr if norm else None), F32(1e-6), P(dinv.ptr), P(dinvd.ptr), mi.Q8_ROUND_X86, P(h.ptr))
    mi._call("mi_mul_mat_q8_0_f32_fused", None, 1, _ptrs(pd), _i64s(n), _ptrs(y), _ptrs(dres), nff, P(h.ptr), None,
             F32(0.0), None, mi.Q8_ROUND_X86)
    # the three launches
    yg, yu = mi.DeviceBuffer(4 * nff), mi.DeviceBuffer(4 * nff)
    mi._call("mi_mul_mat_q8_0_f32_fused", None, 2, _ptrs(pg, pu), _i64s(nff, nff), _ptrs(yg, yu), None, k,
             P(dx.ptr), P(dnw.ptr if norm else None), F32(1e-6), P(dinv.ptr), mi.Q8_ROUND_X86)
    xq = mi.DeviceBuffer(mi.xq_size(1, nff))
    mi._call("mi_swiglu_quant_q8_0", None, P(yg.ptr), P(yu.ptr), P(dinvd.ptr), nff, P(xq.ptr), mi.Q8_ROUND_X86)
    y3 = mi.DeviceBuffer(4 * n)
    mi._call("mi_gemv_q8_0_add", None, P(pd.ptr), P(xq.ptr), P(dres.ptr), P(y3.ptr), n, nff, 1)
    # the last-arrival form: quantized row written by the pair launch itself, twice on the
    # same counters (each call leaves them zero)
    xqp = mi.DeviceBuffer(mi.xq_size(1, nff))
    ht = mi.DeviceBuffer(4 * nff)
    ctr = mi.DeviceBuffer(4 * (nff // 32)).zero()
    for _ in range(2):
        mi._call("mi_gate_up_pair_q8_0", None, P(pg.ptr), P(pu.ptr), nff, k, P(dx.ptr), P(dnw.ptr if norm else None),
                 F32(1e-6), P(dinv.ptr), P(dinvd.ptr), mi.Q8_ROUND_X86, P(xqp.ptr), P(ht.ptr), P(ctr.ptr))
    mi.device_sync()
    got, three = y.download(F32), y3.download(F32)
    assert np.array_equal(got, three), f"max |diff| {np.abs(got - three).max():.3e}"
    doff = mi.xq_d_offset(1, nff)
    assert np.array_equal(xqp.download(np.int8, nff), xq.download(np.int8, nff))
    assert np.array_equal(xqp.download(np.uint16, nff // 32, offset=doff), xq.download(np.uint16, nff // 32, offset=doff))
    assert not ctr.download(np.uint32, nff // 32).any()
    xin = rms_norm_ref(x, nw, 1e-6) if norm else x
    g = _q8_ref(orc, wg, xin, nff, k, inv)
    u = _q8_ref(orc, wu, xin, nff, k, inv)
    v = ((g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))).astype(F32) * u).astype(F32)
    ref = (_q8_ref(orc, wd, v, n, nff, inv_d) + res).astype(F32)
    err = rel_err(got, ref)
    print(f"gate/up pair + down {nff}x{k}: rel vs oracle {err:.2e}")
    assert err < GEMV_TOL


def test_gemv_q8_0_add_equals_gemv_plus_vector(gpu):
    mi = gpu
    rng = np.random.default_rng(11)
    n, k = 1536, 8960
    w = q8_0_weights(rng, n, k)
    pw = _packed_q8(mi, w, n, k)
    x = rng.standard_normal(k).astype(F32)
    add = rng.standard_normal(n).astype(F32)
    dx, da = mi.to_device(x), mi.to_device(add)
    dq = mi.DeviceBuffer(mi.xq_size(1, k))
    y0, y1 = mi.DeviceBuffer(4 * n), mi.DeviceBuffer(4 * n)
    mi.act_quant_q8_0(dx.ptr, None, 1, k, dq.ptr, mi.Q8_ROUND_X86)
    mi.gemv_q8_0(pw.ptr, dq.ptr, y0.ptr, n, k, 1)
    mi._call("mi_gemv_q8_0_add", None, mi._P(pw.ptr), mi._P(dq.ptr), mi._P(da.ptr), mi._P(y1.ptr), n, k, 1)
    mi.device_sync()
    assert np.array_equal(y1.download(F32), (y0.download(F32) + add).astype(F32))


def _fa_splits(mi, n_kv, nq, nkv, d):
    return int(mi.lib().mi_fa_decode_num_splits(n_kv, nq, nkv, d))


# (n_kv, q heads, kv heads, head dim, kv_len, mask): 1, 4, 11 (two empty), 13, 16 splits
@pytest.mark.parametrize("L,nq,nkv,d,kv_len,masked", [(64, 12, 2, 128, None, False), (200, 12, 2, 128, None, False),
                                                      (700, 12, 2, 128, 517, False), (777, 8, 4, 64, None, False),
                                                      (1024, 12, 2, 128, None, True)])
def test_fa_partials_into_q8_projection(gpu, orc, L, nq, nkv, d, kv_len, masked):
    """Attention left in split form, merged in the o projection's prologue (+ residual):
    against the oracle's exact attention through the oracle's Q8_0 matmul (GEMV bar), and
    against the unfused FA + combine + fused GEMV launches of this library."""
    mi = gpu
    S = _fa_splits(mi, L, nq, nkv, d)
    assert 1 <= S <= 16
    k = nq * d
    n = k
    rng = np.random.default_rng(L + nq + d)
    q = rng.standard_normal((nq, d)).astype(F32)
    kc = f16_bits(rng.standard_normal((L, nkv, d)))
    vc = f16_bits(rng.standard_normal((L, nkv, d)))
    mask = None
    if masked:
        mf = np.zeros(L, F32)
        mf[L - 100:] = -np.inf
        mf[10:20] = -np.inf
        mf[33] = -2.5
        mask = f16_bits(mf)
    w = q8_0_weights(rng, n, k)
    inv = (1.0 / rng.uniform(0.5, 2.0, k)).astype(F32)
    add = rng.standard_normal(n).astype(F32)
    pw = _packed_q8(mi, w, n, k)
    dq, dk, dv = mi.to_device(q), mi.to_device(kc), mi.to_device(vc)
    dm = mi.to_device(mask) if mask is not None else None
    dl = mi.to_device(np.array([kv_len], np.int32)) if kv_len is not None else None
    dinv, dadd = mi.to_device(inv), mi.to_device(add)
    wsb = mi.fa_decode_workspace_size(L, nq, nkv, d)
    ws = mi.DeviceBuffer(wsb).zero()
    nb1 = nkv * d * 2
    y = mi.DeviceBuffer(4 * n)
    P = mi._P
    mi._call("mi_fa_decode_partials", None, P(dq.ptr), P(dk.ptr), P(dv.ptr), P(dm.ptr if dm else None),
             P(dl.ptr if dl else None), L, nq, nkv, d, nb1, d * 2, nb1, d * 2, F32(1 / np.sqrt(d)), P(ws.ptr), wsb)
    mi._call("mi_mul_mat_q8_0_f32_lse", None, P(pw.ptr), n, P(y.ptr), P(dadd.ptr), P(ws.ptr), S, nq, d,
             P(dinv.ptr), mi.Q8_ROUND_X86)
    # the unfused launches on the same inputs
    att = mi.DeviceBuffer(4 * k)
    ws2 = mi.DeviceBuffer(wsb).zero()
    y2 = mi.DeviceBuffer(4 * n)
    mi.fa_decode(dq.ptr, dk.ptr, dv.ptr, dm.ptr if dm else None, dl.ptr if dl else None, L, nq, nkv, d, nb1, d * 2,
                 nb1, d * 2, 1 / np.sqrt(d), att.ptr, ws2.ptr, wsb)
    mi._call("mi_mul_mat_q8_0_f32_fused", None, 1, _ptrs(pw), _i64s(n), _ptrs(y2), _ptrs(dadd), k, P(att.ptr),
             P(None), F32(0.0), P(dinv.ptr), mi.Q8_ROUND_X86)
    mi.device_sync()
    got, unfused = y.download(F32), y2.download(F32)
    exact = orc.flash_attn_ext_1tok(q, kc, vc, nkv, F32(1 / np.sqrt(d)), mask=mask, kv_len=kv_len, mode=1)
    ref = (_q8_ref(orc, w, exact.reshape(-1).astype(F32), n, k, inv) + add).astype(F32)
    e_ref, e_unf = rel_err(got, ref), rel_err(got, unfused)
    print(f"lse projection S={S}: rel vs oracle {e_ref:.2e}, vs unfused {e_unf:.2e}")
    assert e_ref < GEMV_TOL
    assert e_unf < GEMV_TOL


def test_q8_lse_projection_rejects_bad_shapes(gpu):
    mi = gpu
    P = mi._P
    with pytest.raises(mi.MiError):  # more splits than the prologue merges
        mi._call("mi_mul_mat_q8_0_f32_lse", None, P(256), 1536, P(256), P(None), P(256), 17, 12, 128, P(None), 0)
    with pytest.raises(mi.MiError):  # k above 2048
        mi._call("mi_mul_mat_q8_0_f32_lse", None, P(256), 3584, P(256), P(None), P(256), 4, 28, 128, P(None), 0)


# ---------------------------------------------------------------- W4A16 chains (one activation row)

def _packed_q4(mi, w, n, k):
    src = mi.to_device(w)
    dst = mi.DeviceBuffer(mi.q4_0_packed_size(n, k)).zero()
    mi.prepack_q4_0(src.ptr, dst.ptr, n, k)
    mi.device_sync()
    src.free()
    return dst


def _q4_ref(orc, w, x, n, k):
    """ggml MUL_MAT of a Q4_0 weight and an fp32 row: src1 converted to fp16 (RNE)"""
    return orc.mul_mat_q4_0_f16(w, f16_bits(x), n, k)


# (rows per matrix, k, activation rows, epilogue): q/k/v + bias, gate/up, down + residual
# after the GLU, o + residual, ragged last matrix, one 4-block group per row (k = 128:
# per-group scale loads), a 4096+-row set whose first matrix is not a whole number of
# 32-row tile pairs (one tile per wave)
@pytest.mark.parametrize("ns,k,m,mode", [((3584, 512, 512), 3584, 8, "bias"), ((18944, 18944), 3584, 5, "none"),
                                         ((3584,), 18944, 8, "glu_add"), ((3584,), 3584, 16, "add"),
                                         ((96, 40), 256, 3, "bias"), ((1536,), 8960, 2, "glu"),
                                         ((3584, 512, 512), 3584, 8, "norm_bias"), ((18944, 18944), 3584, 8, "norm"),
                                         ((256,), 4096, 3, "norm"), ((48, 40), 128, 4, "bias"),
                                         ((4080, 48), 256, 6, "bias"), ((4096,), 128, 2, "add")])
def test_q4_batch_set(gpu, orc, ns, k, m, mode):
    """Several activation rows through up to four Q4_0 matrices in one launch: bit-identical
    to one mi_mul_mat_q4_0_f32 launch per matrix followed by the ADD (the graph's node-by-node
    path), and within the GEMV bar of the oracle's ggml MUL_MAT (src1 rounded to fp16)."""
    mi = gpu
    P = mi._P
    rng = np.random.default_rng(sum(ns) + k + m)
    ws = [q4_0_weights(rng, n, k) for n in ns]
    pw = [_packed_q4(mi, w, n, k) for w, n in zip(ws, ns)]
    x = rng.standard_normal((m, k)).astype(F32)
    up = rng.standard_normal((m, k)).astype(F32) if mode.startswith("glu") else None
    bias = [rng.standard_normal(n).astype(F32) for n in ns] if mode.endswith("bias") else None
    add = [rng.standard_normal((m, n)).astype(F32) for n in ns] if mode.endswith("add") else None
    nw = rng.uniform(0.8, 1.2, k).astype(F32) if mode.startswith("norm") else None
    dx = mi.to_device(x)
    dup = mi.to_device(up) if up is not None else None
    dnw = mi.to_device(nw) if nw is not None else None
    db = [mi.to_device(b) for b in bias] if bias else None
    da = [mi.to_device(a) for a in add] if add else None
    ys = [mi.DeviceBuffer(4 * m * n) for n in ns]
    wsb = mi.mul_mat_q4_0_workspace_size(m, k)
    wbuf = mi.DeviceBuffer(wsb)
    mi._call("mi_mul_mat_q4_0_f32_batch", None, len(ns), _ptrs(*pw), _i64s(*ns), _ptrs(*ys),
             _ptrs(*db) if db else None, _ptrs(*da) if da else None, k, m, P(dx.ptr), P(dup.ptr if dup else None),
             P(dnw.ptr if dnw else None), F32(1e-6), P(wbuf.ptr), wsb)
    # node-by-node: GLU, then one launch per matrix, then the ADD
    act = x
    if up is not None:
        dh = mi.DeviceBuffer(4 * m * k)
        mi._call("mi_swiglu", None, P(dx.ptr), P(dup.ptr), P(dh.ptr), m * k)
        mi.device_sync()
        act_dev = dh
        act = dh.download(F32).reshape(m, k)  # the oracle matmul takes the GLU node's output
    elif nw is not None:
        dh = mi.DeviceBuffer(4 * m * k)
        mi._call("mi_rms_norm", None, P(dx.ptr), P(dnw.ptr), P(dh.ptr), k, m, F32(1e-6))
        mi.device_sync()
        act_dev = dh
        act = dh.download(F32).reshape(m, k)
        for r in range(m):
            assert ulp_diff(act[r], rms_norm_ref(x[r], nw, 1e-6)).max() <= 1
    else:
        act_dev = dx
    plain = []
    for t, n in enumerate(ns):
        yb = mi.DeviceBuffer(4 * m * n)
        mi.mul_mat_q4_0_f32(pw[t].ptr, act_dev.ptr, yb.ptr, n, k, m, ws=wbuf.ptr, ws_bytes=wsb)
        mi.device_sync()
        v = yb.download(F32).reshape(m, n)
        if bias:
            v = (v + bias[t]).astype(F32)
        if add:
            v = (v + add[t]).astype(F32)
        plain.append(v)
    mi.device_sync()
    for t, n in enumerate(ns):
        got = ys[t].download(F32).reshape(m, n)
        assert np.array_equal(got, plain[t]), f"matrix {t}: fused differs from node-by-node"
        for r in range(m):
            ref = _q4_ref(orc, ws[t], act[r], n, k)
            if bias:
                ref = (ref + bias[t]).astype(F32)
            if add:
                ref = (ref + add[t][r]).astype(F32)
            assert rel_err(got[r], ref) < GEMV_TOL, f"matrix {t} row {r}"


@pytest.mark.parametrize("ns,k,m,mode", [((1536, 256, 256), 1536, 8, "norm_bias"), ((8960, 8960), 1536, 8, "norm"),
                                         ((1536,), 8960, 8, "glu_add"), ((1536,), 1536, 3, "add"),
                                         ((96, 40), 256, 2, "bias"), ((256,), 4096, 5, "norm"),
                                         ((512,), 8960, 5, "glu"), ((300, 33, 64, 7), 96, 4, "plain")])
def test_q8_batch_set(gpu, orc, ns, k, m, mode):
    """Several activation rows through up to four Q8_0 matrices (mi_mul_mat_q8_0_f32_batch:
    the activation's quantization with RMSNorm or swiglu folded in, then one launch over the
    stacked matrices with the blocks in LDS): bit-identical to the node-by-node path
    (RMS_NORM+MUL or GLU, one mi_mul_mat_q8_0_f32 per matrix, then the ADD), and within the
    GEMV bar of the oracle's Q8_0 MUL_MAT.  k = 8960 at 8 rows stages 76 KB of LDS."""
    mi = gpu
    P = mi._P
    rng = np.random.default_rng(sum(ns) + k + m + len(mode))
    ws = [q8_0_weights(rng, n, k) for n in ns]
    pw = [_packed_q8(mi, w, n, k) for w, n in zip(ws, ns)]
    x = rng.standard_normal((m, k)).astype(F32)
    up = rng.standard_normal((m, k)).astype(F32) if mode.startswith("glu") else None
    bias = [rng.standard_normal(n).astype(F32) for n in ns] if mode.endswith("bias") else None
    add = [rng.standard_normal((m, n)).astype(F32) for n in ns] if mode.endswith("add") else None
    nw = rng.uniform(0.8, 1.2, k).astype(F32) if mode.startswith("norm") else None
    inv = (1.0 / rng.uniform(0.5, 2.0, k)).astype(F32)
    dx, dinv = mi.to_device(x), mi.to_device(inv)
    dup = mi.to_device(up) if up is not None else None
    dnw = mi.to_device(nw) if nw is not None else None
    db = [mi.to_device(b) for b in bias] if bias else None
    da = [mi.to_device(a) for a in add] if add else None
    ys = [mi.DeviceBuffer(4 * m * n) for n in ns]
    wsb = mi.mul_mat_q8_0_workspace_size(m, k)
    wbuf = mi.DeviceBuffer(wsb)
    mi._call("mi_mul_mat_q8_0_f32_batch", None, len(ns), _ptrs(*pw), _i64s(*ns), _ptrs(*ys),
             _ptrs(*db) if db else None, _ptrs(*da) if da else None, k, m, P(dx.ptr), P(dup.ptr if dup else None),
             P(dnw.ptr if dnw else None), F32(1e-6), P(dinv.ptr), mi.Q8_ROUND_X86, P(wbuf.ptr), wsb)
    mi.device_sync()
    # node-by-node: the GLU or the norm, then one launch per matrix, then the ADD
    act_dev = dx
    if up is not None or nw is not None:
        act_dev = mi.DeviceBuffer(4 * m * k)
        if up is not None:
            mi._call("mi_swiglu", None, P(dx.ptr), P(dup.ptr), P(act_dev.ptr), m * k)
        else:
            mi._call("mi_rms_norm", None, P(dx.ptr), P(dnw.ptr), P(act_dev.ptr), k, m, F32(1e-6))
        mi.device_sync()
    act = act_dev.download(F32).reshape(m, k)
    for t, n in enumerate(ns):
        yb = mi.DeviceBuffer(4 * m * n)
        mi.mul_mat_q8_0_f32(pw[t].ptr, act_dev.ptr, dinv.ptr, yb.ptr, n, k, m, ws=wbuf.ptr, ws_bytes=wsb)
        mi.device_sync()
        plain = yb.download(F32).reshape(m, n)
        if bias:
            plain = (plain + bias[t]).astype(F32)
        if add:
            plain = (plain + add[t]).astype(F32)
        got = ys[t].download(F32).reshape(m, n)
        assert np.array_equal(got, plain), f"matrix {t}: batch launch differs from node-by-node"
        for r in range(m):
            ref = _q8_ref(orc, ws[t], act[r], n, k, inv)
            if bias:
                ref = (ref + bias[t]).astype(F32)
            if add:
                ref = (ref + add[t][r]).astype(F32)
            assert rel_err(got[r], ref) < GEMV_TOL, f"matrix {t} row {r}"


@pytest.mark.parametrize("n,k,case", [(151936, 1536, "random"), (152064, 3584, "random"), (5000, 1536, "ties"),
                                      (333, 256, "nan"), (77, 512, "all_neg_inf")])
def test_head_f16_argmax(gpu, n, k, case):
    """The output head with the norm and the argmax folded in (mi_head_f16_argmax):
    logits bit-identical to mi_rms_norm + mi_gemv_f16, and the same index as mi_argmax
    over them, including equal maxima in different workgroups (the lower row wins), NaN
    rows (never taken) and all-(-inf) logits (index 0)."""
    mi = gpu
    P = mi._P
    rng = np.random.default_rng(n + k)
    w = (rng.standard_normal((n, k), dtype=np.float32) * F32(0.05)).astype(np.float16)
    x = rng.standard_normal(k).astype(F32)
    if case == "ties":  # rows 4321 and 17 (workgroups apart) equal, and far above the others
        w[17] = w[4321] = (np.sign(x) * 0.5).astype(np.float16)
    if case == "nan":
        w[5, :] = np.float16(np.nan)
    if case == "all_neg_inf":
        w[:, :] = np.float16(-np.inf)
    if case == "all_neg_inf":
        x = np.abs(x) + F32(0.5)
    nw = rng.uniform(0.8, 1.2, k).astype(F32)
    dw, dx, dnw = mi.to_device(w.view(np.uint16)), mi.to_device(x), mi.to_device(nw)
    y1, y2 = mi.DeviceBuffer(4 * n), mi.DeviceBuffer(4 * n)
    o1, o2 = mi.DeviceBuffer(4), mi.DeviceBuffer(4)
    h = mi.DeviceBuffer(4 * k)
    wsb = max(mi.lib().mi_head_f16_argmax_workspace_size(n, k), mi.lib().mi_argmax_workspace_size(n, 1))
    ws = mi.DeviceBuffer(wsb)
    mi._call("mi_head_f16_argmax", None, P(dw.ptr), k, P(dx.ptr), P(dnw.ptr), F32(1e-6), P(y1.ptr), P(o1.ptr), n, k,
             P(ws.ptr), wsb)
    mi.device_sync()
    mi._call("mi_rms_norm", None, P(dx.ptr), P(dnw.ptr), P(h.ptr), k, 1, F32(1e-6))
    mi._call("mi_gemv_f16", None, P(dw.ptr), k, P(h.ptr), P(y2.ptr), n, k, 1)
    mi._call("mi_argmax", None, P(y2.ptr), P(o2.ptr), n, 1, P(ws.ptr), wsb)
    mi.device_sync()
    a, b = y1.download(F32), y2.download(F32)
    assert np.array_equal(a.view(np.int32), b.view(np.int32)), f"logits differ at {np.flatnonzero(a != b)[:5]}"
    i1, i2 = int(o1.download(np.int32)[0]), int(o2.download(np.int32)[0])
    assert i1 == i2, (i1, i2)
    if case == "ties":
        assert i1 == 17
    if case == "all_neg_inf":
        assert i1 == 0 and np.all(np.isneginf(a))
    if case == "nan":
        assert np.isnan(a[5]) and i1 != 5


def test_q4_batch_set_rejects_bad_shapes(gpu):
    mi = gpu
    P = mi._P
    w = _ptrs(mi.DeviceBuffer(256))
    y = _ptrs(mi.DeviceBuffer(256))
    with pytest.raises(mi.MiError):  # k not a multiple of 128
        mi._call("mi_mul_mat_q4_0_f32_batch", None, 1, w, _i64s(16), y, None, None, 96, 2, P(256), P(None), P(None),
                 F32(0), P(256), 1 << 20)
    with pytest.raises(mi.MiError):  # 17 activation rows
        mi._call("mi_mul_mat_q4_0_f32_batch", None, 1, w, _i64s(16), y, None, None, 128, 17, P(256), P(None), P(None),
                 F32(0), P(256), 1 << 20)
    with pytest.raises(mi.MiError):  # RMSNorm of a row longer than 4096
        mi._call("mi_mul_mat_q4_0_f32_batch", None, 1, w, _i64s(16), y, None, None, 4224, 2, P(256), P(None), P(256),
                 F32(1e-6), P(256), 1 << 20)


@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("ns,k", [((18944, 18944), 3584), ((3584,), 3584), ((3584, 512, 512), 3584),
                                  ((1536,), 1536), ((7, 9), 256), ((66,), 4096)])
def test_q4_fused_norm_matmuls_add(gpu, orc, norm, ns, k):
    from synth import q4_0_weights
    mi = gpu
    rng = np.random.default_rng(sum(ns) + k + norm)
    x = (rng.standard_normal(k) * 0.5).astype(F32)
    nw = rng.uniform(0.8, 1.2, k).astype(F32)
    ws = [q4_0_weights(rng, n, k) for n in ns]
    adds = [rng.standard_normal(n).astype(F32) if i % 2 == 0 else None for i, n in enumerate(ns)]
    pw = [_packed_q4(mi, w, n, k) for w, n in zip(ws, ns)]
    ys = [mi.DeviceBuffer(4 * n) for n in ns]
    da = [mi.to_device(a) if a is not None else None for a in adds]
    dx, dnw = mi.to_device(x), mi.to_device(nw)
    mi._call("mi_mul_mat_q4_0_f32_fused", None, len(ns), _ptrs(*pw), _i64s(*ns), _ptrs(*ys), _ptrs(*da), k,
             mi._P(dx.ptr), mi._P(dnw.ptr if norm else None), F32(1e-6))
    mi.device_sync()
    xin = rms_norm_ref(x, nw, 1e-6) if norm else x
    for i, n in enumerate(ns):
        ref = _q4_ref(orc, ws[i], xin, n, k)
        if adds[i] is not None:
            ref = (ref + adds[i]).astype(F32)
        err = rel_err(ys[i].download(F32), ref)
        print(f"q4 fused {ns} k={k} norm={norm} matrix {i}: rel_err {err:.2e}")
        assert err < GEMV_TOL, f"matrix {i}"


@pytest.mark.parametrize("n,k", [(18944, 3584), (8960, 1536), (33, 512)])
def test_q4_gate_up_swiglu(gpu, orc, n, k):
    """h = fp16(silu(gate) * up): the GLU output as the down projection's MUL_MAT converts it"""
    from synth import q4_0_weights
    mi = gpu
    rng = np.random.default_rng(n + k)
    x = (rng.standard_normal(k) * 0.5).astype(F32)
    nw = rng.uniform(0.8, 1.2, k).astype(F32)
    wg, wu = q4_0_weights(rng, n, k), q4_0_weights(rng, n, k)
    pg, pu = _packed_q4(mi, wg, n, k), _packed_q4(mi, wu, n, k)
    dx, dnw = mi.to_device(x), mi.to_device(nw)
    dh = mi.DeviceBuffer(2 * n)
    mi._call("mi_gate_up_swiglu_q4_0", None, mi._P(pg.ptr), mi._P(pu.ptr), n, k, mi._P(dx.ptr), mi._P(dnw.ptr),
             F32(1e-6), mi._P(dh.ptr))
    mi.device_sync()
    xn = rms_norm_ref(x, nw, 1e-6)
    g = _q4_ref(orc, wg, xn, n, k)
    u = _q4_ref(orc, wu, xn, n, k)
    h = ((g / (1.0 + np.exp(-g.astype(np.float64)))).astype(F32) * u).astype(F32)
    got = dh.download(np.uint16).view(np.float16).astype(F32)
    err = rel_err(got, h)
    print(f"gate_up_swiglu {n}x{k}: rel_err {err:.2e}")
    assert err < GEMV_TOL


@pytest.mark.parametrize("table", [False, True])
@pytest.mark.parametrize("idx_i64", [False, True])
@pytest.mark.parametrize("cfg", [dict(k=3584, hq=28, hkv=4, hd=128, pos=32767, row=32767, bias=True),
                                 dict(k=1536, hq=12, hkv=2, hd=128, pos=517, row=517, bias=True),
                                 dict(k=256, hq=4, hkv=2, hd=64, pos=0, row=0, bias=False),
                                 dict(k=512, hq=6, hkv=3, hd=32, pos=40, row=1, bias=True)])
def test_q4_qkv_rope_kv(gpu, orc, cfg, idx_i64, table):
    from synth import q4_0_weights
    mi = gpu
    k, hq, hkv, hd = cfg["k"], cfg["hq"], cfg["hkv"], cfg["hd"]
    nq, nkv = hq * hd, hkv * hd
    n_cache = max(640, cfg["row"] + 1)
    rng = np.random.default_rng(k + hq + cfg["pos"] + idx_i64)
    x = (rng.standard_normal(k) * 0.5).astype(F32)
    nw = rng.uniform(0.8, 1.2, k).astype(F32)
    ns = (nq, nkv, nkv)
    ws = [q4_0_weights(rng, n, k) for n in ns]
    bs = [(rng.standard_normal(n) * 0.02).astype(F32) if cfg["bias"] else None for n in ns]
    pw = [_packed_q4(mi, w, n, k) for w, n in zip(ws, ns)]
    db = [mi.to_device(b) if b is not None else None for b in bs]
    dx, dnw = mi.to_device(x), mi.to_device(nw)
    dq = mi.DeviceBuffer(4 * nq)
    kc = mi.DeviceBuffer(n_cache * nkv * 2).zero()
    vc = mi.DeviceBuffer(n_cache * nkv * 2).zero()
    dpos = mi.to_device(np.array([cfg["pos"]], np.int32))
    didx = mi.to_device(np.array([cfg["row"]], np.int64 if idx_i64 else np.int32))
    tab = _rope_table(mi, dpos, hd, 1e6) if table else None
    mi._call("mi_qkv_rope_kv_q4_0", None, _ptrs(*pw), _i64s(*ns), _ptrs(*db), k, mi._P(dx.ptr), mi._P(dnw.ptr),
             F32(1e-6), hd, mi._P(dpos.ptr), F32(1e6), F32(1.0), F32(1.0), mi._P(dq.ptr), mi._P(kc.ptr), nkv * 2,
             mi._P(vc.ptr), nkv * 2, mi._P(didx.ptr), int(idx_i64), n_cache, mi._P(tab.ptr if tab is not None else None))
    mi.device_sync()
    xn = rms_norm_ref(x, nw, 1e-6)
    proj = []
    for i, n in enumerate(ns):
        y = _q4_ref(orc, ws[i], xn, n, k)
        proj.append((y + bs[i]).astype(F32) if bs[i] is not None else y)
    q_ref = rope_neox_ref(proj[0].reshape(hq, hd), cfg["pos"], hd, 1e6).reshape(-1)
    k_ref = rope_neox_ref(proj[1].reshape(hkv, hd), cfg["pos"], hd, 1e6).reshape(-1)
    assert rel_err(dq.download(F32), q_ref) < GEMV_TOL
    kcache = kc.download(np.uint16).reshape(n_cache, nkv)
    vcache = vc.download(np.uint16).reshape(n_cache, nkv)
    for name, cache, ref in (("k", kcache, k_ref), ("v", vcache, proj[2])):
        got = cache[cfg["row"]].view(np.float16).astype(np.float64)
        tol = 2 * np.abs(ref.astype(np.float16).astype(np.float64)) * 2.0 ** -10 + 1e-7
        assert np.all(np.abs(got - ref) <= tol + GEMV_TOL * np.sqrt(np.mean(ref.astype(np.float64) ** 2))), name
        others = np.delete(cache, cfg["row"], axis=0)
        assert not others.any(), f"{name} cache rows other than {cfg['row']} were written"


def test_q4_qkv_rope_kv_skips_out_of_range_row(gpu):
    from synth import q4_0_weights
    mi = gpu
    rng = np.random.default_rng(8)
    k, hd, ns = 256, 64, (256, 128, 128)
    ws = [q4_0_weights(rng, n, k) for n in ns]
    pw = [_packed_q4(mi, w, n, k) for w, n in zip(ws, ns)]
    dx = mi.to_device(rng.standard_normal(k).astype(F32))
    dq = mi.DeviceBuffer(4 * ns[0])
    kc = mi.DeviceBuffer(8 * 128 * 2).zero()
    vc = mi.DeviceBuffer(8 * 128 * 2).zero()
    dpos = mi.to_device(np.array([3], np.int32))
    didx = mi.to_device(np.array([-1], np.int32))   # before the first cache row
    mi._call("mi_qkv_rope_kv_q4_0", None, _ptrs(*pw), _i64s(*ns), _ptrs(None, None, None), k, mi._P(dx.ptr), None,
             F32(1e-6), hd, mi._P(dpos.ptr), F32(1e4), F32(1.0), F32(1.0), mi._P(dq.ptr), mi._P(kc.ptr), 256,
             mi._P(vc.ptr), 256, mi._P(didx.ptr), 0, 8, None)
    mi.device_sync()
    assert not kc.download(np.uint16).any() and not vc.download(np.uint16).any()


# (sequences, KV length, q heads, kv heads, head dim): the 7B shape with several splits and
# with one, and the 1.5B head group
@pytest.mark.parametrize("n_seq,L,nq,nkv,d", [(8, 3000, 28, 4, 128), (3, 40, 28, 4, 128), (2, 700, 12, 2, 128),
                                              (4, 300, 8, 2, 64)])
def test_fa_q4act_into_batch_projection(gpu, n_seq, L, nq, nkv, d):
    """Attention of several sequences written straight into the o projection's permuted fp16
    activation, then the matrix-core projection with its residual, is bit-identical to the
    fp32 attention output followed by the projection that converts it (the node-by-node
    ubatch path); the attention itself is pinned against the oracle by the flash-decoding
    tests."""
    mi = gpu
    P = mi._P
    rng = np.random.default_rng(n_seq * L + nq)
    q = rng.standard_normal((n_seq, nq, d)).astype(F32)
    kc = f16_bits(rng.standard_normal((n_seq, L, nkv, d)))
    vc = f16_bits(rng.standard_normal((n_seq, L, nkv, d)))
    lens = rng.integers(1, L + 1, n_seq).astype(np.int32)
    dq, dk, dv, dl = mi.to_device(q), mi.to_device(kc), mi.to_device(vc), mi.to_device(lens)
    k_in, n_out = nq * d, 3584
    w = q4_0_weights(rng, n_out, k_in)
    pw = _packed_q4(mi, w, n_out, k_in)
    res = rng.standard_normal((n_seq, n_out)).astype(F32)
    dres = mi.to_device(res)
    wsb = mi.fa_decode_batch_workspace_size(L, nq, nkv, d, n_seq)
    ws = mi.DeviceBuffer(wsb).zero()
    nb1 = nkv * d * 2
    seq_bytes = L * nb1
    scale = F32(1 / np.sqrt(d))
    # node by node: fp32 attention output, then the projection converting it
    out = mi.DeviceBuffer(n_seq * k_in * 4)
    mi.fa_decode_batch(dq.ptr, dk.ptr, dv.ptr, None, dl.ptr, L, nq, nkv, d, nb1, d * 2, nb1, d * 2, scale, out.ptr,
                       n_seq, nq * d, seq_bytes, seq_bytes, 0, nq * d, ws.ptr, wsb)
    y1 = mi.DeviceBuffer(4 * n_seq * n_out)
    pws = mi.DeviceBuffer(n_seq * k_in * 2)
    mi._call("mi_mul_mat_q4_0_f32_batch", None, 1, _ptrs(pw), _i64s(n_out), _ptrs(y1), None, _ptrs(dres), k_in,
             n_seq, P(out.ptr), None, None, F32(1e-6), P(pws.ptr), n_seq * k_in * 2)
    # fused: the combine writes the permuted activation
    xp = mi.DeviceBuffer(n_seq * k_in * 2)
    mi._call("mi_fa_decode_batch_q4act", None, P(dq.ptr), P(dk.ptr), P(dv.ptr), None, P(dl.ptr), L, nq, nkv, d, nb1,
             d * 2, nb1, d * 2, scale, P(xp.ptr), n_seq, nq * d, seq_bytes, seq_bytes, 0, P(ws.ptr), wsb)
    y2 = mi.DeviceBuffer(4 * n_seq * n_out)
    mi._call("mi_mul_mat_q4_0_batch_xp", None, 1, _ptrs(pw), _i64s(n_out), _ptrs(y2), None, _ptrs(dres), k_in, n_seq,
             P(xp.ptr))
    mi.device_sync()
    assert np.array_equal(xp.download(np.uint16), pws.download(np.uint16))
    assert np.array_equal(y1.download(F32), y2.download(F32))


def test_q4act_entry_points_reject_bad_arguments(gpu):
    mi = gpu
    P = mi._P
    with pytest.raises(RuntimeError):
        mi._call("mi_mul_mat_q4_0_batch_xp", None, 1, None, None, None, None, None, 128, 2, None)
    with pytest.raises(RuntimeError):
        mi._call("mi_fa_decode_batch_q4act", None, None, None, None, None, None, 64, 2, 1, 64, 128, 128, 128, 128,
                 F32(0.1), None, 2, 128, 0, 0, 0, None, 0)


@pytest.mark.parametrize("n,k,m,norm", [(18944, 3584, 8, True), (512, 256, 3, False), (1024, 4096, 16, True),
                                         (256, 128, 2, False)])
def test_q4_gate_up_glu_batch(gpu, n, k, m, norm):
    """Gate and up of several rows with the swiglu in their epilogue, written as the down
    projection's permuted fp16 activation: bit-identical to the gate/up batch launch
    followed by the down projection's GLU conversion (both checked on the activation and
    on the down projection's output with the residual)."""
    mi = gpu
    P = mi._P
    rng = np.random.default_rng(n + k + m)
    wg, wu = q4_0_weights(rng, n, k), q4_0_weights(rng, n, k)
    pg, pu = _packed_q4(mi, wg, n, k), _packed_q4(mi, wu, n, k)
    nd = 384
    wd = q4_0_weights(rng, nd, n)
    pd = _packed_q4(mi, wd, nd, n)
    x = rng.standard_normal((m, k)).astype(F32)
    nw = rng.uniform(0.8, 1.2, k).astype(F32)
    res = rng.standard_normal((m, nd)).astype(F32)
    dx, dnw, dres = mi.to_device(x), mi.to_device(nw), mi.to_device(res)
    ws = mi.DeviceBuffer(m * k * 2)
    hxp = mi.DeviceBuffer(m * n * 2)
    mi._call("mi_mul_mat_q4_0_gate_up_glu_batch", None, P(pg.ptr), P(pu.ptr), n, k, m, P(dx.ptr),
             P(dnw.ptr if norm else None), F32(1e-6), P(ws.ptr), m * k * 2, P(hxp.ptr))
    y1 = mi.DeviceBuffer(4 * m * nd)
    mi._call("mi_mul_mat_q4_0_batch_xp", None, 1, _ptrs(pd), _i64s(nd), _ptrs(y1), None, _ptrs(dres), n, m,
             P(hxp.ptr))
    # node by node: gate/up batch (fp32 outputs), then the down projection converting the GLU
    yg, yu = mi.DeviceBuffer(4 * m * n), mi.DeviceBuffer(4 * m * n)
    ws2 = mi.DeviceBuffer(m * max(k, n) * 2)
    mi._call("mi_mul_mat_q4_0_f32_batch", None, 2, _ptrs(pg, pu), _i64s(n, n), _ptrs(yg, yu), None, None, k, m,
             P(dx.ptr), None, P(dnw.ptr if norm else None), F32(1e-6), P(ws2.ptr), m * max(k, n) * 2)
    y2 = mi.DeviceBuffer(4 * m * nd)
    mi._call("mi_mul_mat_q4_0_f32_batch", None, 1, _ptrs(pd), _i64s(nd), _ptrs(y2), None, _ptrs(dres), n, m,
             P(yg.ptr), P(yu.ptr), None, F32(0.0), P(ws2.ptr), m * max(k, n) * 2)
    mi.device_sync()
    assert np.array_equal(hxp.download(np.uint16), ws2.download(np.uint16, m * n))
    assert np.array_equal(y1.download(F32), y2.download(F32))


# (activation rows, k, head dim, q heads, kv heads, index type, norm): the 7B ubatch shape,
# a 64-wide head, one sequence, two with 64-bit cache indices
@pytest.mark.parametrize("m,k,hd,nhq,nhk,idx_i64,norm", [(8, 3584, 128, 28, 4, False, True),
                                                         (3, 512, 64, 8, 2, True, False),
                                                         (1, 1024, 128, 4, 2, False, True),
                                                         (2, 256, 32, 4, 1, True, True)])
def test_q4_qkv_rope_kv_batch(gpu, m, k, hd, nhq, nhk, idx_i64, norm):
    """q/k/v of several rows with their biases, the rotation of q and k and the k / v cache
    writes in the projection's epilogue: bit-identical to the q/k/v batch launch followed
    by the rope + cache-write launch (the node-by-node ubatch path); a cache index outside
    the cache is skipped."""
    mi = gpu
    P = mi._P
    rng = np.random.default_rng(m * 100 + k + hd)
    ns = (nhq * hd, nhk * hd, nhk * hd)
    ws_ = [q4_0_weights(rng, n, k) for n in ns]
    pw = [_packed_q4(mi, w, n, k) for w, n in zip(ws_, ns)]
    bias = [rng.standard_normal(n).astype(F32) for n in ns]
    db = [mi.to_device(b) for b in bias]
    x = rng.standard_normal((m, k)).astype(F32)
    nw = rng.uniform(0.8, 1.2, k).astype(F32)
    dx, dnw = mi.to_device(x), mi.to_device(nw)
    n_cache = 48
    pos = rng.integers(0, 40000, m).astype(np.int32)
    idx = rng.permutation(n_cache)[:m].astype(np.int64 if idx_i64 else np.int32)
    if m > 2:
        idx[1] = n_cache + 3  # outside the cache: not written
    kc0 = f16_bits(rng.standard_normal((n_cache, ns[1])))
    vc0 = f16_bits(rng.standard_normal((n_cache, ns[2])))
    dp, di = mi.to_device(pos), mi.to_device(idx)
    wsb = m * k * 2
    # fused
    kc1, vc1, qo1 = mi.to_device(kc0), mi.to_device(vc0), mi.DeviceBuffer(4 * m * ns[0])
    ws1 = mi.DeviceBuffer(wsb)
    mi._call("mi_qkv_rope_kv_q4_0_batch", None, _ptrs(*pw), _i64s(*ns), _ptrs(*db), k, m, P(dx.ptr),
             P(dnw.ptr if norm else None), F32(1e-6), P(ws1.ptr), wsb, hd, P(dp.ptr), F32(1e6), F32(1.0), F32(1.0),
             P(qo1.ptr), P(kc1.ptr), ns[1] * 2, P(vc1.ptr), ns[2] * 2, P(di.ptr), int(idx_i64), n_cache)
    # node by node: the set with biases, then rope + cache writes
    ys = [mi.DeviceBuffer(4 * m * n) for n in ns]
    ws2 = mi.DeviceBuffer(wsb)
    mi._call("mi_mul_mat_q4_0_f32_batch", None, 3, _ptrs(*pw), _i64s(*ns), _ptrs(*ys), _ptrs(*db), None, k, m,
             P(dx.ptr), None, P(dnw.ptr if norm else None), F32(1e-6), P(ws2.ptr), wsb)
    kc2, vc2, qo2 = mi.to_device(kc0), mi.to_device(vc0), mi.DeviceBuffer(4 * m * ns[0])
    mi._call("mi_rope_kv_rows", None, P(ys[0].ptr), P(ys[1].ptr), P(ys[2].ptr), P(qo2.ptr), P(kc2.ptr), ns[1] * 2,
             P(vc2.ptr), ns[2] * 2, P(dp.ptr), P(di.ptr), int(idx_i64), n_cache, m, hd, nhq, nhk, ns[2], F32(1e6),
             F32(1.0), F32(1.0))
    mi.device_sync()
    assert np.array_equal(qo1.download(F32), qo2.download(F32))
    assert np.array_equal(kc1.download(np.uint16), kc2.download(np.uint16))
    assert np.array_equal(vc1.download(np.uint16), vc2.download(np.uint16))
