"""The drop-in boundary driven directly through the ggml backend vtables, the way
llama.cpp's loader and scheduler call them (cf. patch:1700-1847 set_tensor /
get_alloc_size, patch:1957-1983 supports_op):
  - get_alloc_size picks the weights that get a side copy (and the A8W8 env selection);
  - set_tensor in chunks, out of order and from two threads gives the side copy a
    whole-tensor upload gives;
  - F16 weights on the A8W8 path are quantized on the device bit for bit as the
    oracle's quantize_row_q8_0_ref of W*diag(s) (s applied before or after the upload);
  - supports_op rejects what the kernels do not take (the scheduler then runs it on CPU);
  - a tensor flagged as a graph output is written even where a fusion would skip it."""
import ctypes
import threading

import numpy as np
import pytest

import ggml_api as ga
from synth import f16_bits, q8_0_weights, rel_err

pytestmark = pytest.mark.gpu


def _pad256(n):
    return (n + 255) // 256 * 256


@pytest.fixture(scope="module")
def api(gpu):
    L = ga.bind(gpu.lib())
    be = L.ggml_backend_mi355x_init(0)
    assert be
    yield gpu, L, be, L.ggml_backend_mi355x_buffer_type(0)
    L.ggml_backend_free(be)


def _side_copy(mi, L, t, nbytes_packed):
    """bytes of the side copy at tensor->data + pad256(nbytes)"""
    src = t.contents.data + _pad256(L.ggml_nbytes(t))
    out = np.empty(nbytes_packed, np.uint8)
    mi._call("mi_memcpy_d2h", mi._P(out.ctypes.data), mi._P(src), nbytes_packed, None)
    return out


def test_alloc_size_selects_side_copies(api, monkeypatch):
    mi, L, be, buft = api
    k, n = 256, 64
    names = ["blk.0.ffn_up.weight", "blk.1.ffn_up.weight", "blk.4.attn_q.weight", "blk.6.attn_output.weight",
             "blk.7.ffn_down.weight", "token_embd.weight", "blk.0.attn_norm.weight"]
    q8 = mi.q8_0_packed_size(n, k)
    for a8w8, disabled in ((None, None), ("1", "1,3-5"), ("1", "")):
        for var, val in (("GGML_MI355X_A8W8", a8w8), ("GGML_MI355X_A8W8_DISABLE_LAYERS", disabled)):
            if val is None:
                monkeypatch.delenv(var, raising=False)
            else:
                monkeypatch.setenv(var, val)
        ctx = ga.Context(mi.lib())
        got = {}
        for nm in names:
            t = ctx.tensor(ga.GGML_TYPE_F32 if "norm" in nm else ga.GGML_TYPE_F16, k, n, name=nm)
            got[nm] = L.ggml_backend_buft_get_alloc_size(buft, t) - L.ggml_nbytes(t)
        qw = ctx.tensor(ga.GGML_TYPE_Q8_0, k, n, name="blk.2.ffn_gate.weight")
        assert L.ggml_backend_buft_get_alloc_size(buft, qw) == _pad256(L.ggml_nbytes(qw)) + q8
        side = _pad256(k * n * 2) - k * n * 2 + q8
        if a8w8 is None:
            assert all(v == 0 for v in got.values()), got
        else:
            off = {"1,3-5": {"blk.1.ffn_up.weight", "blk.4.attn_q.weight"}, "": set()}[disabled]
            for nm, v in got.items():
                expect = side if (nm.startswith("blk.") and "norm" not in nm and nm not in off) else 0
                assert v == expect, (disabled, nm, v)
        ctx.free()


def _upload_chunks(ctx, t, blob, cuts, order):
    pieces = [(cuts[i], cuts[i + 1]) for i in range(len(cuts) - 1)]
    for i in order:
        a, b = pieces[i]
        ctx.set(t, blob[a:b], offset=a)


def test_set_tensor_chunked_out_of_order_and_concurrent(api):
    mi, L, be, buft = api
    rng = np.random.default_rng(77)
    n, k = 512, 1536
    blobs = [q8_0_weights(rng, n, k).reshape(-1) for _ in range(4)]
    ctx = ga.Context(mi.lib())
    ts = [ctx.tensor(ga.GGML_TYPE_Q8_0, k, n, name=f"blk.{i}.ffn_gate.weight") for i in range(4)]
    ctx.alloc(buft)
    size = blobs[0].size
    want = [np.empty(mi.q8_0_packed_size(n, k), np.uint8) for _ in range(4)]
    for b, w in zip(blobs, want):
        mi._call("mi_prepack_q8_0_host", mi._P(b.ctypes.data), mi._P(w.ctypes.data), n, k)
    # 0: one write; 1: three chunks (not block-aligned) in reverse order
    ctx.set(ts[0], blobs[0])
    _upload_chunks(ctx, ts[1], blobs[1], [0, 1001, size - 3333, size], [2, 1, 0])
    # 2 and 3: two threads, each uploading its own tensor in 7 interleaved chunks
    cuts = [0] + sorted(np.random.default_rng(5).choice(np.arange(1, size), 6, replace=False).tolist()) + [size]
    th = [threading.Thread(target=_upload_chunks, args=(ctx, ts[i], blobs[i], cuts, [6, 0, 5, 1, 4, 2, 3]))
          for i in (2, 3)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    for i in range(4):
        got = _side_copy(mi, L, ts[i], want[i].size)
        assert np.array_equal(got, want[i]), f"tensor {i}"
        assert np.array_equal(ctx.get(ts[i], np.uint8), blobs[i]), f"ggml bytes of tensor {i}"
    ctx.free()


def test_a8w8_f16_weights_quantized_at_upload(api, orc, monkeypatch):
    mi, L, be, buft = api
    monkeypatch.setenv("GGML_MI355X_A8W8", "1")
    monkeypatch.setenv("GGML_MI355X_A8W8_DISABLE_LAYERS", "1")
    rng = np.random.default_rng(78)
    n, k = 384, 1536
    w16 = f16_bits(rng.standard_normal((n, k)) * 0.02)
    wf = w16.view(np.float16).astype(np.float32)
    s1 = rng.uniform(0.5, 2.0, k).astype(np.float32)
    s2 = rng.uniform(0.5, 2.0, k).astype(np.float32)
    psz = mi.q8_0_packed_size(n, k)

    def expect(s):
        blocks = orc.quantize_weight_q8_0(wf, s)
        out = np.empty(psz, np.uint8)
        mi._call("mi_prepack_q8_0_host", mi._P(blocks.ctypes.data), mi._P(out.ctypes.data), n, k)
        return out

    ctx = ga.Context(mi.lib())
    a = ctx.tensor(ga.GGML_TYPE_F16, k, n, name="blk.0.ffn_up.weight")     # s after the upload
    b = ctx.tensor(ga.GGML_TYPE_F16, k, n, name="blk.0.ffn_gate.weight")   # s before the last chunk
    c = ctx.tensor(ga.GGML_TYPE_F16, k, n, name="blk.0.attn_q.weight")     # no s
    d = ctx.tensor(ga.GGML_TYPE_F16, k, n, name="blk.1.ffn_up.weight")     # layer kept F16
    ctx.alloc(buft)
    assert L.ggml_backend_buft_get_alloc_size(buft, d) == L.ggml_nbytes(d)
    # smoothing an unquantized weight is the identity: accepted, nothing to store
    assert L.ggml_backend_mi355x_set_smooth_factors(d, s1.ctypes.data, k)
    blob = w16.reshape(-1).view(np.uint8)
    ctx.set(a, blob)
    assert np.array_equal(_side_copy(mi, L, a, psz), expect(None))
    assert L.ggml_backend_mi355x_set_smooth_factors(a, s1.ctypes.data, k)
    assert np.array_equal(_side_copy(mi, L, a, psz), expect(s1))
    assert L.ggml_backend_mi355x_set_smooth_factors(a, s2.ctypes.data, k)   # re-quantized from the F16 bytes
    assert np.array_equal(_side_copy(mi, L, a, psz), expect(s2))
    _upload_chunks(ctx, b, blob, [0, 5000, blob.size], [1])
    assert L.ggml_backend_mi355x_set_smooth_factors(b, s1.ctypes.data, k)
    _upload_chunks(ctx, b, blob, [0, 5000, blob.size], [0])
    assert np.array_equal(_side_copy(mi, L, b, psz), expect(s1))
    _upload_chunks(ctx, c, blob, [0, 777, 100000, blob.size], [2, 0, 1])
    assert np.array_equal(_side_copy(mi, L, c, psz), expect(None))
    assert np.array_equal(ctx.get(a, np.uint16), w16.reshape(-1))   # ggml bytes untouched
    bad = s1.copy()
    bad[3] = -1.0
    assert not L.ggml_backend_mi355x_set_smooth_factors(c, bad.ctypes.data, k)
    assert not L.ggml_backend_mi355x_set_smooth_factors(c, s1.ctypes.data, k - 32)
    ctx.free()


def test_supports_op_rejections(api):
    mi, L, be, buft = api
    wctx = ga.Context(mi.lib())
    W = wctx.tensor(ga.GGML_TYPE_Q8_0, 1536, 256, name="blk.0.attn_q.weight")
    wctx.alloc(buft)
    fctx = ga.Context(mi.lib())
    Wf = fctx.tensor(ga.GGML_TYPE_Q8_0, 1536, 256, name="blk.0.attn_k.weight")
    fctx.alloc(L.ggml_backend_cpu_buffer_type())
    foreign = ctypes.create_string_buffer(64)
    Wf.contents.extra = ctypes.addressof(foreign)   # a CPU repack buffer type's own data
    g = ga.Context(mi.lib())
    ok = lambda t: bool(L.ggml_backend_supports_op(be, t))
    mm = lambda w, m: L.ggml_mul_mat(g.ctx, w, g.tensor(ga.GGML_TYPE_F32, 1536, m))
    assert ok(mm(W, 1)) and ok(mm(W, 8))
    assert not ok(mm(W, 9))                       # M = 9: beyond the decode GEMVs
    assert not ok(mm(Wf, 1))                      # weight in another backend's buffer

    def fa(d=128, nq=1, kv_type=ga.GGML_TYPE_F16, mask_type=None, n_kv=512):
        q = g.tensor(ga.GGML_TYPE_F32, d, nq, 12, 1)
        kk = g.tensor(kv_type, d, n_kv, 2, 1)
        vv = g.tensor(kv_type, d, n_kv, 2, 1)
        m = g.tensor(mask_type, n_kv, nq) if mask_type is not None else None
        return L.ggml_flash_attn_ext(g.ctx, q, kk, vv, m, 0.0884, 0.0, 0.0)

    assert ok(fa()) and ok(fa(mask_type=ga.GGML_TYPE_F16)) and ok(fa(d=64))
    assert not ok(fa(d=96))                       # head dim 96
    assert not ok(fa(kv_type=ga.GGML_TYPE_F32))   # F32 K/V
    assert not ok(fa(mask_type=ga.GGML_TYPE_F32))  # F32 mask
    assert not ok(fa(nq=2))                       # two query rows per head (a prompt ubatch)
    for c in (g, fctx, wctx):
        c.free()


def _rms_ref(x, w, eps):
    xs = x.astype(np.float64)
    scale = np.float32(1.0 / np.sqrt(np.float32(np.mean(xs * xs)) + np.float32(eps)))
    return ((x * scale).astype(np.float32) * w).astype(np.float32)


@pytest.mark.parametrize("flag", [False, True])
def test_output_flag_is_written_through_fusion(api, orc, flag):
    """RMS_NORM -> MUL(w) -> gate/up MUL_MATs is one fused launch that never writes the MUL
    output; flagged as a graph output (llama.cpp's result_norm, the embeddings it reads
    back), the MUL output must be written.  The unflagged run shows the fusion happens:
    a sentinel in the MUL tensor survives it."""
    mi, L, be, buft = api
    rng = np.random.default_rng(79)
    k, n = 1536, 512
    w1, w2 = q8_0_weights(rng, n, k), q8_0_weights(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    nw = rng.uniform(0.8, 1.2, k).astype(np.float32)
    wctx = ga.Context(mi.lib())
    tw1 = wctx.tensor(ga.GGML_TYPE_Q8_0, k, n, name="blk.0.ffn_gate.weight")
    tw2 = wctx.tensor(ga.GGML_TYPE_Q8_0, k, n, name="blk.0.ffn_up.weight")
    tx = wctx.tensor(ga.GGML_TYPE_F32, k, name="x")
    tnw = wctx.tensor(ga.GGML_TYPE_F32, k, name="blk.0.ffn_norm.weight")
    wctx.alloc(buft)
    for t, a in ((tw1, w1), (tw2, w2), (tx, x), (tnw, nw)):
        wctx.set(t, a)
    g = ga.Context(mi.lib())
    mul = L.ggml_mul(g.ctx, L.ggml_rms_norm(g.ctx, tx, 1e-6), tnw)
    if flag:
        L.ggml_set_output(mul)
    gt, ut = L.ggml_mul_mat(g.ctx, tw1, mul), L.ggml_mul_mat(g.ctx, tw2, mul)
    gf = L.ggml_new_graph(g.ctx)
    L.ggml_build_forward_expand(gf, gt)
    L.ggml_build_forward_expand(gf, ut)
    ga_ = L.ggml_gallocr_new(buft)
    assert L.ggml_gallocr_alloc_graph(ga_, gf)
    sentinel = np.full(k, 12345.0, np.float32)
    g.set(mul, sentinel)
    assert L.ggml_backend_graph_compute(be, gf) == 0
    xn = _rms_ref(x, nw, 1e-6)
    got_mul = g.get(mul, np.float32)
    if flag:
        assert rel_err(got_mul, xn) < 1e-6
    else:
        assert np.array_equal(got_mul, sentinel)
    for wt, t in ((w1, gt), (w2, ut)):
        assert rel_err(g.get(t, np.float32), orc.mul_mat_q8_0(wt, xn, n, k)) < 1e-3
    L.ggml_gallocr_free(ga_)
    g.free()
    wctx.free()
