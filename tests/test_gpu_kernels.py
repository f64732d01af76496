"""GPU parity of the gfx950 kernels against the CPU oracle, called through the C ABI.

Bars: int32 block dots and Q8_0 activation bytes bit-exact; GEMV fp32 outputs
within 1e-3 relative (rel_err: per-element relative error with an rms floor);
attention within 2e-3 max-abs of the ggml-CPU restatement, widened to the
restatement's own distance from the exact fp64 answer when that is larger (its
V accumulator is fp16), and within 5e-5 of the exact answer.
"""
import numpy as np
import pytest

from synth import f16_bits, q4_0_weights, q8_0_split, q8_0_weights, rel_err, xq_to_blocks

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3


def _xq_parts(mi, dev_xq, m, k):
    qs = dev_xq.download(np.int8, m * k)
    d = dev_xq.download(np.uint16, m * (k // 32), offset=mi.xq_d_offset(m, k))
    return qs.reshape(m, k), d.reshape(m, k // 32)


def _packed_q8(mi, w, n, k):
    src = mi.to_device(w)
    dst = mi.DeviceBuffer(mi.q8_0_packed_size(n, k)).zero()  # plane padding is not written by the prepack
    mi.prepack_q8_0(src.ptr, dst.ptr, n, k)
    mi.device_sync()
    src.free()
    return dst


def _packed_q4(mi, w, n, k):
    src = mi.to_device(w)
    dst = mi.DeviceBuffer(mi.q4_0_packed_size(n, k)).zero()  # plane padding is not written by the prepack
    mi.prepack_q4_0(src.ptr, dst.ptr, n, k)
    mi.device_sync()
    src.free()
    return dst


# ---------------------------------------------------------------- prepack

@pytest.mark.parametrize("n,k", [(3, 64), (8960, 1536)])
def test_device_prepack_matches_host(gpu, n, k):
    mi = gpu
    rng = np.random.default_rng(100)
    w8 = q8_0_weights(rng, n, k)
    assert np.array_equal(_packed_q8(mi, w8, n, k).download(np.uint8), mi.prepack_q8_0_host(w8, n, k))
    w4 = q4_0_weights(rng, n, k)
    assert np.array_equal(_packed_q4(mi, w4, n, k).download(np.uint8), mi.prepack_q4_0_host(w4, n, k))


# ---------------------------------------------------------------- activation quantization

@pytest.mark.parametrize("rounding", [0, 1])
@pytest.mark.parametrize("k,m,smooth", [(32, 1, False), (1536, 1, False), (8960, 1, True), (1536, 3, True)])
def test_act_quant_bitexact(gpu, orc, rounding, k, m, smooth):
    mi = gpu
    rng = np.random.default_rng(k + m)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0, :32] = 0.0  # zero block
    if k >= 64:
        x[0, 32:64] = (np.arange(32) % 5 - 2) * np.float32(0.5)  # halves: ties after scaling
        x[0, 32] = 127.0  # amax 127 -> id == 1, so 0.5 / 1.5 / -0.5 are exact ties
    inv = (1.0 / rng.uniform(0.5, 2.0, k)).astype(np.float32) if smooth else None
    dx = mi.to_device(x)
    dinv = mi.to_device(inv) if smooth else None
    dq = mi.DeviceBuffer(mi.xq_size(m, k))
    mi.act_quant_q8_0(dx.ptr, dinv.ptr if smooth else None, m, k, dq.ptr, rounding)
    mi.device_sync()
    qs, d = _xq_parts(mi, dq, m, k)
    for i in range(m):
        ref = orc.quantize_row_q8_0(x[i], inv_s=inv, variant=rounding)
        assert np.array_equal(xq_to_blocks(qs[i], d[i], k), ref), f"row {i}"


# ---------------------------------------------------------------- Q8_0 GEMV

def test_q8_0_block_dots_bitexact_config0(gpu, orc):
    """Single A8W8 GEMV N=8960 x K=1536: every int32 block dot product bit-exact."""
    mi = gpu
    n, k = 8960, 1536
    rng = np.random.default_rng(0)
    w = q8_0_weights(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    wp = _packed_q8(mi, w, n, k)
    dx = mi.to_device(x)
    dq = mi.DeviceBuffer(mi.xq_size(1, k))
    mi.act_quant_q8_0(dx.ptr, None, 1, k, dq.ptr, mi.Q8_ROUND_X86)
    dots = mi.DeviceBuffer(n * (k // 32) * 4)
    mi.q8_0_block_dots(wp.ptr, dq.ptr, dots.ptr, n, k)
    mi.device_sync()
    got = dots.download(np.int32).reshape(n, k // 32)
    xq = orc.quantize_row_q8_0(x, variant=orc.Q8_ROUND_X86)
    assert np.array_equal(got, orc.q8_0_block_dots(w, xq, n, k))


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("rounding", [0, 1])
def test_q8_0_gemv_config0(gpu, orc, fused, rounding):
    mi = gpu
    n, k = 8960, 1536
    rng = np.random.default_rng(1)
    w = q8_0_weights(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    wp = _packed_q8(mi, w, n, k)
    dx = mi.to_device(x)
    dy = mi.DeviceBuffer(n * 4)
    if fused:
        assert mi.mul_mat_q8_0_workspace_size(1, k) == 0
        mi.mul_mat_q8_0_f32(wp.ptr, dx.ptr, None, dy.ptr, n, k, 1, rounding)
    else:
        dq = mi.DeviceBuffer(mi.xq_size(1, k))
        mi.act_quant_q8_0(dx.ptr, None, 1, k, dq.ptr, rounding)
        mi.gemv_q8_0(wp.ptr, dq.ptr, dy.ptr, n, k, 1)
    mi.device_sync()
    y = dy.download(np.float32)
    ref = orc.mul_mat_q8_0(w, x, n, k, variant=rounding)
    err = rel_err(y, ref)
    print(f"q8_0 gemv {n}x{k} fused={fused} rounding={rounding}: rel_err={err:.3e}")
    assert err < GEMV_TOL


@pytest.mark.parametrize("n,k,m", [(1, 32, 1), (17, 96, 2), (4095, 1536, 1), (1536, 8960, 1), (256, 1536, 3),
                                   (300, 18944, 1), (64, 32768, 1), (1536, 1536, 8), (8960, 1536, 5)])
def test_q8_0_gemv_shapes(gpu, orc, n, k, m):
    mi = gpu
    rng = np.random.default_rng(n * 7 + k + m)
    w = q8_0_weights(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    inv = (1.0 / rng.uniform(0.5, 2.0, k)).astype(np.float32)
    wp = _packed_q8(mi, w, n, k)
    dx, dinv = mi.to_device(x), mi.to_device(inv)
    dy = mi.DeviceBuffer(m * n * 4)
    dy2 = mi.DeviceBuffer(m * n * 4)
    dq = mi.DeviceBuffer(mi.xq_size(m, k))
    wsb = mi.mul_mat_q8_0_workspace_size(m, k)
    ws = mi.DeviceBuffer(max(wsb, 1))
    mi.mul_mat_q8_0_f32(wp.ptr, dx.ptr, dinv.ptr, dy.ptr, n, k, m, mi.Q8_ROUND_X86, ws.ptr, wsb)
    mi.act_quant_q8_0(dx.ptr, dinv.ptr, m, k, dq.ptr, mi.Q8_ROUND_X86)
    mi.gemv_q8_0(wp.ptr, dq.ptr, dy2.ptr, n, k, m)
    mi.device_sync()
    y = dy.download(np.float32).reshape(m, n)
    y2 = dy2.download(np.float32).reshape(m, n)
    ref = orc.mul_mat_q8_0(w, x, n, k, inv_s=inv)
    ref = ref.reshape(m, n)
    assert rel_err(y, ref) < GEMV_TOL
    assert rel_err(y2, ref) < GEMV_TOL


# ---------------------------------------------------------------- W4A16

@pytest.mark.parametrize("n,k,m", [(1536, 8960, 1), (8960, 1536, 1), (7, 32, 1), (512, 3584, 8), (100, 18944, 1),
                                   (4608, 3584, 1), (2049, 256, 1), (300, 18944, 8), (3584, 4096, 5),
                                   (1030, 3584, 16), (77, 160, 2), (5, 16384, 1), (33, 8192, 1),
                                   (9, 32000, 1), (9, 32768, 1), (50, 33792, 1), (3, 64, 1), (64, 128, 4),
                                   (4100, 128, 3)])
def test_w4a16_gemv(gpu, orc, n, k, m):
    """one activation row: the register-resident kernel for k <= 32768 (every blocks-per-
    lane / waves-per-row shape; odd n leaves the last row pair half empty), beyond that the
    fp16-from-global kernel through a workspace; several rows: the matrix-core kernel"""
    mi = gpu
    rng = np.random.default_rng(n + k + m)
    w = q4_0_weights(rng, n, k)
    x16 = f16_bits(rng.standard_normal((m, k)))
    wp = _packed_q4(mi, w, n, k)
    dx = mi.to_device(x16)
    dy = mi.DeviceBuffer(m * n * 4)
    mi.gemv_q4_0_f16(wp.ptr, dx.ptr, dy.ptr, n, k, m)
    # fp32 activation variant (cast fused in the prologue)
    x32 = x16.view(np.float16).astype(np.float32)
    dx32 = mi.to_device(x32)
    dy32 = mi.DeviceBuffer(m * n * 4)
    wsb = mi.mul_mat_q4_0_workspace_size(m, k)
    ws = mi.DeviceBuffer(max(wsb, 16))
    mi.mul_mat_q4_0_f32(wp.ptr, dx32.ptr, dy32.ptr, n, k, m, ws=ws.ptr, ws_bytes=wsb)
    mi.device_sync()
    y = dy.download(np.float32).reshape(m, n)
    for i in range(m):
        ref = orc.mul_mat_q4_0_f16(w, x16[i], n, k)
        ref64 = orc.mul_mat_q4_0_f16_f64(w, x16[i], n, k)
        err = rel_err(y[i], ref)
        print(f"w4a16 {n}x{k} row {i}: rel_err vs ggml-cpu {err:.3e}, vs fp64 {rel_err(y[i], ref64):.3e}")
        assert err < GEMV_TOL
        assert rel_err(y[i], ref64) < 1e-5
    assert rel_err(dy32.download(np.float32).reshape(m, n), y) < 1e-5


# ---------------------------------------------------------------- F16

# m = 2..8 with k a multiple of 32 take the matrix-core kernel (ragged last 16-row tile,
# padded rows, the 7B head's k); k = 72 and m = 1 the dot2 kernels
@pytest.mark.parametrize("n,k,m,pad", [(151936, 1536, 1, 0), (1000, 1536, 2, 8), (33, 8960, 1, 0), (64, 72, 8, 0),
                                       (20000, 3584, 8, 0), (4100, 256, 3, 0), (1031, 1536, 5, 8), (17, 4064, 2, 0),
                                       (300, 2048, 8, 16)])
def test_f16_gemv(gpu, orc, n, k, m, pad):
    mi = gpu
    rng = np.random.default_rng(n + k)
    ldw = k + pad
    w = f16_bits(rng.standard_normal((n, ldw)) * 0.02)
    x = rng.standard_normal((m, k)).astype(np.float32)
    dw, dx = mi.to_device(w), mi.to_device(x)
    dy = mi.DeviceBuffer(m * n * 4)
    mi.gemv_f16(dw.ptr, ldw, dx.ptr, dy.ptr, n, k, m)
    mi.device_sync()
    y = dy.download(np.float32).reshape(m, n)
    wk = np.ascontiguousarray(w[:, :k])
    for i in range(m):
        ref = orc.mul_mat_f16(wk, x[i], n, k)
        err = rel_err(y[i], ref)
        print(f"f16 gemv {n}x{k}: rel_err {err:.3e}")
        assert err < GEMV_TOL


# ---------------------------------------------------------------- flash-decoding

def _fa_run(mi, q, kc, vc, n_kv_heads, scale, mask=None, kv_len=None, cap=None):
    nq, d = q.shape
    n_kv = kc.shape[0]
    dq, dk, dv = mi.to_device(q), mi.to_device(kc), mi.to_device(vc)
    dm = mi.to_device(mask) if mask is not None else None
    dl = mi.to_device(np.array([kv_len], np.int32)) if kv_len is not None else None
    out = mi.DeviceBuffer(nq * d * 4)
    ws_bytes = mi.fa_decode_workspace_size(n_kv, nq, n_kv_heads, d)
    ws = mi.DeviceBuffer(ws_bytes).zero()
    nb1 = n_kv_heads * d * 2
    mi.fa_decode(dq.ptr, dk.ptr, dv.ptr, dm.ptr if dm else None, dl.ptr if dl else None, n_kv, nq, n_kv_heads, d,
                 nb1, d * 2, nb1, d * 2, scale, out.ptr, ws.ptr, ws_bytes)
    mi.device_sync()
    return out.download(np.float32).reshape(nq, d)


def _check_fa(orc, o, q, kc, vc, nkv, scale, mask=None, kv_len=None, label=""):
    exact = orc.flash_attn_ext_1tok(q, kc, vc, nkv, scale, mask=mask, kv_len=kv_len, mode=1)
    ggml = orc.flash_attn_ext_1tok(q, kc, vc, nkv, scale, mask=mask, kv_len=kv_len, mode=0)
    e_exact = float(np.abs(o - exact).max())
    e_ggml = float(np.abs(o - ggml).max())
    dev_ggml = float(np.abs(ggml - exact).max())
    print(f"fa {label}: max|gpu-exact|={e_exact:.2e} max|gpu-ggml|={e_ggml:.2e} (ggml own {dev_ggml:.2e})")
    # The gate is the exact fp64 attention (pinned by closed forms and brute force).  The
    # ggml-CPU restatement keeps V.softmax in an fp16 accumulator (pinned by its own KATs);
    # its distance from the exact answer grows with L and passes 2e-3 at some lengths, so
    # an exact kernel cannot meet a 2e-3 bar against it there.  That distance is printed,
    # not gated: it follows from the exact gate by the triangle inequality.
    assert e_exact < 5e-5
    assert e_ggml <= dev_ggml + 5e-5


@pytest.mark.parametrize("L", [512, 4096, 32768])
def test_fa_decode_config2(gpu, orc, L):
    """Single-token GQA decode attention, 12 q / 2 kv heads, D=128, fp16 KV of length L."""
    mi = gpu
    rng = np.random.default_rng(L)
    q = rng.standard_normal((12, 128)).astype(np.float32)
    kc = f16_bits(rng.standard_normal((L, 2, 128)))
    vc = f16_bits(rng.standard_normal((L, 2, 128)))
    o = _fa_run(mi, q, kc, vc, 2, 1 / np.sqrt(128))
    _check_fa(orc, o, q, kc, vc, 2, 1 / np.sqrt(128), label=f"L={L}")


@pytest.mark.parametrize("L", [1, 2, 15, 127, 128, 129, 239, 240, 241, 255, 256, 257, 511, 513, 1024, 5000, 8192,
                               12345])
def test_fa_decode_boundaries(gpu, orc, L):
    """Split and block edges; 5000 (79 splits) and 12345 (193) end the combine's 128-split
    chunks part way, past 64 splits where each thread loads 16 splits at once."""
    mi = gpu
    rng = np.random.default_rng(1000 + L)
    q = rng.standard_normal((12, 128)).astype(np.float32)
    kc = f16_bits(rng.standard_normal((L, 2, 128)))
    vc = f16_bits(rng.standard_normal((L, 2, 128)))
    o = _fa_run(mi, q, kc, vc, 2, 1 / np.sqrt(128))
    if L == 1:
        vf = vc.view(np.float16).astype(np.float32)
        assert np.array_equal(o[:6], np.broadcast_to(vf[0, 0], (6, 128)))
    _check_fa(orc, o, q, kc, vc, 2, 1 / np.sqrt(128), label=f"L={L}")


@pytest.mark.parametrize("nq,nkv,d", [(8, 2, 128), (16, 4, 128), (32, 8, 128), (14, 2, 64), (28, 4, 128),
                                      (4, 4, 64), (8, 1, 128)])
def test_fa_decode_gqa(gpu, orc, nq, nkv, d):
    mi = gpu
    L = 777
    rng = np.random.default_rng(nq * 100 + nkv * 10 + d)
    q = rng.standard_normal((nq, d)).astype(np.float32)
    kc = f16_bits(rng.standard_normal((L, nkv, d)))
    vc = f16_bits(rng.standard_normal((L, nkv, d)))
    o = _fa_run(mi, q, kc, vc, nkv, 1 / np.sqrt(d))
    _check_fa(orc, o, q, kc, vc, nkv, 1 / np.sqrt(d), label=f"{nq}/{nkv} d={d}")


def test_fa_decode_mask_and_kv_len(gpu, orc):
    mi = gpu
    L, used = 4096, 1500
    rng = np.random.default_rng(7)
    q = rng.standard_normal((12, 128)).astype(np.float32)
    kc = f16_bits(rng.standard_normal((L, 2, 128)))
    vc = f16_bits(rng.standard_normal((L, 2, 128)))
    mask = np.zeros(L, np.float32)
    mask[used:] = -np.inf
    mask[100:110] = -np.inf  # interior holes
    mask[200] = -3.0         # finite bias
    m16 = f16_bits(mask)
    o1 = _fa_run(mi, q, kc, vc, 2, 0.088, mask=m16)
    _check_fa(orc, o1, q, kc, vc, 2, 0.088, mask=m16, label="mask")
    o2 = _fa_run(mi, q, kc, vc, 2, 0.088, mask=m16, kv_len=used)
    _check_fa(orc, o2, q, kc, vc, 2, 0.088, mask=m16, kv_len=used, label="mask+kv_len")
    o3 = _fa_run(mi, q, kc, vc, 2, 0.088, kv_len=used)
    _check_fa(orc, o3, q, kc, vc, 2, 0.088, kv_len=used, label="kv_len")
    allm = f16_bits(np.full(L, -np.inf, np.float32))
    assert not _fa_run(mi, q, kc, vc, 2, 0.088, mask=allm).any()


def test_kv_lengths_device(gpu, orc):
    mi = gpu
    rng = np.random.default_rng(3)
    rows, n_kv = 9, 1000
    mask = np.zeros((rows, n_kv), np.float32)
    for r in range(rows):
        cut = int(rng.integers(0, n_kv + 1))
        mask[r, cut:] = -np.inf
    mask[3, 500] = np.nan
    for is_f16 in (True, False):
        mk = f16_bits(mask) if is_f16 else mask
        dm = mi.to_device(mk)
        out = mi.DeviceBuffer(rows * 4)
        mi.kv_lengths(dm.ptr, is_f16, n_kv, rows, out.ptr)
        mi.device_sync()
        assert np.array_equal(out.download(np.int32), orc.kv_lengths(mk, is_f16=is_f16))


def test_fa_decode_batch_eight_sequences(gpu, orc):
    """Eight sequences in one launch (the plan spreads ~512 workgroups over all of them:
    8 blocks of 16 positions per wave), ragged kv lengths, the last split partly past the
    view."""
    mi = gpu
    n_seq, L, nq, nkv, d = 8, 12000, 28, 4, 128
    lens = [L, 37, 1234, L, L - 1, 2048, 2049, 5000]
    rng = np.random.default_rng(L)
    q = rng.standard_normal((n_seq, nq, d)).astype(np.float32)
    kc = f16_bits(rng.standard_normal((n_seq, L, nkv, d)))
    vc = f16_bits(rng.standard_normal((n_seq, L, nkv, d)))
    dq, dk, dv = mi.to_device(q), mi.to_device(kc), mi.to_device(vc)
    dl = mi.to_device(np.array(lens, np.int32))
    out = mi.DeviceBuffer(n_seq * nq * d * 4)
    wsb = mi.fa_decode_batch_workspace_size(L, nq, nkv, d, n_seq)
    ws = mi.DeviceBuffer(wsb).zero()
    nb1 = nkv * d * 2
    seq_bytes = L * nb1
    mi.fa_decode_batch(dq.ptr, dk.ptr, dv.ptr, None, dl.ptr, L, nq, nkv, d, nb1, d * 2, nb1, d * 2, 1 / np.sqrt(d),
                       out.ptr, n_seq, nq * d, seq_bytes, seq_bytes, 0, nq * d, ws.ptr, wsb)
    mi.device_sync()
    o = out.download(np.float32).reshape(n_seq, nq, d)
    for s in range(n_seq):
        _check_fa(orc, o[s], q[s], kc[s], vc[s], nkv, 1 / np.sqrt(d), kv_len=lens[s], label=f"seq {s}")


@pytest.mark.parametrize("T,L,p0,use_kvl", [(8, 4096, 1000, True), (3, 256, 100, False), (8, 512, 0, True),
                                             (5, 32768, 30000, True), (2, 768, 700, False)])
def test_fa_decode_rows_prompt_ubatch(gpu, orc, T, L, p0, use_kvl):
    """A prompt ubatch of one sequence: T query rows per head (q [d, T, n_head] as llama.cpp
    permutes it), one K/V view and kv length for all rows, llama.cpp's causal mask (row t
    keeps positions <= p0 + t) with a hole and a finite bias; every row against the oracle
    run with its own mask row."""
    mi = gpu
    nq, nkv, d = 12, 2, 128
    rng = np.random.default_rng(T * 7 + L)
    q = rng.standard_normal((T, nq, d)).astype(np.float32)
    kc = f16_bits(rng.standard_normal((L, nkv, d)))
    vc = f16_bits(rng.standard_normal((L, nkv, d)))
    mask = np.zeros((T, L), np.float32)
    for t in range(T):
        mask[t, p0 + t + 1:] = -np.inf
    mask[:, p0 // 2: p0 // 2 + 3] = -np.inf
    mask[:, p0 // 3] = -2.5
    m16 = f16_bits(mask)
    kvl = p0 + T if use_kvl else None
    dq, dk, dv, dm = mi.to_device(q), mi.to_device(kc), mi.to_device(vc), mi.to_device(m16)
    dl = mi.to_device(np.array([kvl], np.int32)) if use_kvl else None
    out = mi.DeviceBuffer(T * nq * d * 4)
    wsb = mi.fa_decode_batch_workspace_size(L, nq, nkv, d, T)
    ws = mi.DeviceBuffer(wsb).zero()
    nb1 = nkv * d * 2
    mi.fa_decode_rows(dq.ptr, dk.ptr, dv.ptr, dm.ptr, dl.ptr if dl else None, L, nq, nkv, d, nb1, d * 2, nb1, d * 2,
                      1 / np.sqrt(d), out.ptr, T, nq * d, L, nq * d, ws.ptr, wsb)
    mi.device_sync()
    o = out.download(np.float32).reshape(T, nq, d)
    for t in range(T):
        _check_fa(orc, o[t], q[t], kc, vc, nkv, 1 / np.sqrt(d), mask=m16[t], kv_len=kvl, label=f"row {t}")


@pytest.mark.parametrize("L", [600_000, 1_100_000])
def test_fa_decode_longest_views(gpu, orc, L):
    """Views past 512K positions, where the split count cap lengthens each wave's run to
    16 (L=600000) or 32 (L=1100000) blocks; the last split partly past the view."""
    mi = gpu
    nq, nkv, d = 2, 1, 64
    rng = np.random.default_rng(L)
    q = rng.standard_normal((nq, d)).astype(np.float32)
    kc = f16_bits(rng.standard_normal((L, nkv, d)) * 0.5)
    vc = f16_bits(rng.standard_normal((L, nkv, d)))
    o = _fa_run(mi, q, kc, vc, nkv, 1 / np.sqrt(d))
    _check_fa(orc, o, q, kc, vc, nkv, 1 / np.sqrt(d), label=f"L={L}")


@pytest.mark.parametrize("use_mask", [False, True])
def test_fa_decode_batch_sequences(gpu, orc, use_mask):
    """Independent sequences in one launch (grid z), each with its own cache region, length
    and mask row; against the oracle run per sequence."""
    mi = gpu
    n_seq, L, nq, nkv, d = 3, 1100, 28, 4, 128
    stride_rows = 1200                 # cache positions per sequence (> the view length L)
    lens = [1100, 37, 700]
    rng = np.random.default_rng(55 + use_mask)
    q = rng.standard_normal((n_seq, nq, d)).astype(np.float32)
    kc = f16_bits(rng.standard_normal((n_seq, stride_rows, nkv, d)))
    vc = f16_bits(rng.standard_normal((n_seq, stride_rows, nkv, d)))
    mask = np.zeros((n_seq, L), np.float32)
    for s in range(n_seq):
        mask[s, lens[s]:] = -np.inf
    mask[0, 5] = -np.inf
    m16 = f16_bits(mask)
    dq, dk, dv = mi.to_device(q), mi.to_device(kc), mi.to_device(vc)
    dm = mi.to_device(m16) if use_mask else None
    dl = mi.to_device(np.array(lens, np.int32))
    out = mi.DeviceBuffer(n_seq * nq * d * 4)
    wsb = mi.fa_decode_batch_workspace_size(L, nq, nkv, d, n_seq)
    ws = mi.DeviceBuffer(wsb).zero()
    nb1 = nkv * d * 2
    seq_bytes = stride_rows * nb1
    mi.fa_decode_batch(dq.ptr, dk.ptr, dv.ptr, dm.ptr if dm else None, dl.ptr, L, nq, nkv, d, nb1, d * 2, nb1, d * 2,
                       1 / np.sqrt(d), out.ptr, n_seq, nq * d, seq_bytes, seq_bytes, L, nq * d, ws.ptr, wsb)
    mi.device_sync()
    o = out.download(np.float32).reshape(n_seq, nq, d)
    for s in range(n_seq):
        _check_fa(orc, o[s], q[s], np.ascontiguousarray(kc[s, :L]), np.ascontiguousarray(vc[s, :L]), nkv,
                  1 / np.sqrt(d), mask=m16[s] if use_mask else None, kv_len=lens[s], label=f"seq {s}")
