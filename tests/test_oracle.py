"""Pins the CPU oracle (oracle/ggml_oracle.c) before it is trusted as the checker.

Every check here is independent of the formula it tests: numpy's IEEE fp16
conversion, integer brute force, fp64 closed forms, special cases that reduce
to a textbook answer, and the known answers the reference's own probes use
(experiments/a8w8/quant_matmul_v3_probe.cpp:30-32,76-77;
experiments/a8w8/custom_a8w8_chain_probe.cpp:104-115,189).
"""
import numpy as np
import pytest

from synth import f16_bits, q4_0_weights, q8_0_split, q8_0_weights, rel_err

RNG = np.random.default_rng


# ---------------------------------------------------------------- fp16

def test_fp16_to_fp32_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint16)
    got = orc.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def test_fp32_to_fp16_matches_numpy_rne(orc):
    rng = RNG(1)
    bits = rng.integers(0, 2**32, size=1_000_000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[np.isfinite(f)]
    # add exact ties and subnormal edges
    ties = (np.arange(0, 2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24)
    edge = np.array([65504.0, 65519.99, 65520.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 6.1e-5, -0.0],
                    dtype=np.float32)
    f = np.concatenate([f, ties, edge])
    with np.errstate(over="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(orc.f32_to_f16(f), want)


# ---------------------------------------------------------------- Q8_0 quantization

def _split_xq(blocks, k):
    qs, d = q8_0_split(blocks.reshape(1, -1), 1, k)
    return qs.reshape(-1), d.reshape(-1)


@pytest.mark.parametrize("variant", [0, 1])
def test_q8_0_quant_invariants(orc, variant):
    rng = RNG(2)
    k = 4096
    x = rng.standard_normal(k).astype(np.float32)
    x[32:64] = 0.0  # an all-zero block
    qs, d = _split_xq(orc.quantize_row_q8_0(x, variant=variant), k)
    xb = x.reshape(-1, 32)
    qb = qs.reshape(-1, 32).astype(np.int32)
    assert np.all(np.abs(qb) <= 127)
    # the element of largest magnitude maps to +-127, except the zero block
    for b in range(xb.shape[0]):
        if b == 1:
            assert d[b] == 0.0 and not qb[b].any()
            continue
        i = np.argmax(np.abs(xb[b]))
        assert abs(qb[b, i]) == 127 and np.sign(qb[b, i]) == np.sign(xb[b, i])
    # d is amax/127 rounded to fp16
    amax = np.abs(xb).max(axis=1)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float32).astype(np.float16).astype(np.float32))
    # reconstruction error bounded by half a step (plus the fp16 rounding of d)
    err = np.abs(qb * d[:, None] - xb)
    assert np.all(err <= 0.5 * d[:, None] * 1.01 + amax[:, None] * 2.0 ** -10)


@pytest.mark.parametrize("variant", [0, 1])
def test_q8_0_quant_symmetry_and_pow2_scaling(orc, variant):
    rng = RNG(3)
    k = 2048
    x = rng.standard_normal(k).astype(np.float32)
    q1, d1 = _split_xq(orc.quantize_row_q8_0(x, variant=variant), k)
    q2, d2 = _split_xq(orc.quantize_row_q8_0(-x, variant=variant), k)
    q3, d3 = _split_xq(orc.quantize_row_q8_0(x * np.float32(4.0), variant=variant), k)
    assert np.array_equal(q2, -q1) and np.array_equal(d1, d2)
    assert np.array_equal(q3, q1) and np.array_equal(d3, 4 * d1)


def test_q8_0_rounding_variants_differ_only_on_ties(orc):
    # block: amax = 127 so that id == 1 in both variants; 2.5 -> ref 3 (away), x86 2 (even)
    x = np.zeros(32, dtype=np.float32)
    x[0] = 127.0
    x[1] = 2.5
    x[2] = -3.5
    x[3] = 1.25
    qr, _ = _split_xq(orc.quantize_row_q8_0(x, variant=orc.Q8_ROUND_REF), 32)
    qx, _ = _split_xq(orc.quantize_row_q8_0(x, variant=orc.Q8_ROUND_X86), 32)
    assert list(qr[:4]) == [127, 3, -4, 1]
    assert list(qx[:4]) == [127, 2, -4, 1]


def test_q8_0_constant_input_kat(orc):
    # custom_a8w8_chain_probe.cpp:100,189: x = 1.0 quantizes to 127
    for variant in (0, 1):
        qs, d = _split_xq(orc.quantize_row_q8_0(np.ones(1536, np.float32), variant=variant), 1536)
        assert np.all(qs == 127)
        assert np.all(d == np.float32(np.float16(1.0 / 127.0)))


def test_q8_0_smoothquant_divisor_folded(orc):
    rng = RNG(4)
    k = 1536
    x = rng.standard_normal(k).astype(np.float32)
    s = rng.uniform(0.5, 2.0, k).astype(np.float32)
    inv = (np.float32(1.0) / s).astype(np.float32)
    a = orc.quantize_row_q8_0(x, inv_s=inv)
    b = orc.quantize_row_q8_0((x * inv).astype(np.float32))
    assert np.array_equal(a, b)


# ---------------------------------------------------------------- Q8_0 dot products

def test_block_dots_brute_force(orc):
    rng = RNG(5)
    n, k = 64, 1536
    w = q8_0_weights(rng, n, k)
    xq = orc.quantize_row_q8_0(rng.standard_normal(k).astype(np.float32))
    got = orc.q8_0_block_dots(w, xq, n, k)
    wq, _ = q8_0_split(w, n, k)
    xqs, _ = _split_xq(xq, k)
    want = (wq.astype(np.int64).reshape(n, -1, 32) * xqs.astype(np.int64).reshape(1, -1, 32)).sum(axis=2)
    assert np.array_equal(got, want)


def test_all_ones_kat(orc):
    # quant_matmul_v3_probe.cpp:30-32,76-77: x = w = 1 gives out[n] = K (here int32 block dots,
    # 32 per block; the fp32 output is K * 127 * fp16(1/127) with d_w = 1)
    n, k = 16, 1536
    blk = np.zeros((n, k // 32, 34), dtype=np.uint8)
    blk[:, :, 0:2] = f16_bits(np.ones((n, k // 32))).view(np.uint8).reshape(n, k // 32, 2)
    blk[:, :, 2:] = 1
    w = blk.reshape(n, -1)
    xq = np.zeros((k // 32, 34), dtype=np.uint8)
    xq[:, 0:2] = f16_bits(np.ones(k // 32)).view(np.uint8).reshape(-1, 2)
    xq[:, 2:] = 1
    dots = orc.q8_0_block_dots(w, xq.reshape(-1), n, k)
    assert np.all(dots == 32)
    assert np.all(dots.sum(axis=1) == k)
    y = orc.mul_mat_q8_0(w, np.ones(k, np.float32), n, k)
    assert np.allclose(y, k * 127 * np.float32(np.float16(1 / 127)), rtol=1e-6)


def test_chain_probe_pattern_kat(orc):
    # custom_a8w8_chain_probe.cpp:104-115,189: w[row][col] = (row%7)-3+(col%3), x = 1,
    # PASS when |out[0] - sum_row w[row][0]| <= 8.  ggml weights are [N rows][K]; row index
    # of the probe is the K index here.
    k, n = 1536, 64
    kk = np.arange(k)[None, :]
    nn = np.arange(n)[:, None]
    wv = ((kk % 7) - 3 + (nn % 3)).astype(np.int8)
    blk = np.zeros((n, k // 32, 34), dtype=np.uint8)
    blk[:, :, 0:2] = f16_bits(np.ones((n, k // 32))).view(np.uint8).reshape(n, k // 32, 2)
    blk[:, :, 2:] = wv.reshape(n, k // 32, 32).view(np.uint8)
    y = orc.mul_mat_q8_0(blk.reshape(n, -1), np.ones(k, np.float32), n, k)
    expected = wv.astype(np.int64).sum(axis=1)
    assert abs(y[0] - expected[0]) <= 8
    assert np.allclose(y, expected * 127 * np.float64(np.float16(1 / 127)), rtol=1e-5, atol=1e-3)


def test_mul_mat_q8_0_vs_fp64(orc):
    rng = RNG(6)
    n, k = 512, 1536
    w = q8_0_weights(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    for variant in (0, 1):
        xq = orc.quantize_row_q8_0(x, variant=variant)
        y = orc.mul_mat_q8_0(w, x, n, k, variant=variant)
        wq, wd = q8_0_split(w, n, k)
        xqs, xd = _split_xq(xq, k)
        ref = ((wq.astype(np.float64).reshape(n, -1, 32) * xqs.astype(np.float64).reshape(1, -1, 32)).sum(axis=2)
               * (wd.astype(np.float64) * xd.astype(np.float64)[None, :])).sum(axis=1)
        assert rel_err(y, ref) < 1e-5
    ymt = orc.mul_mat_q8_0_mt(w, x, n, k, n_threads=4)
    assert rel_err(ymt, orc.mul_mat_q8_0(w, x, n, k)) < 1e-5


def test_weight_quantizer_smoothquant(orc):
    rng = RNG(7)
    n, k = 32, 256
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    s = rng.uniform(0.5, 2.0, k).astype(np.float32)
    q = orc.quantize_weight_q8_0(w, s)
    deq = orc.dequantize_q8_0(q, k)
    ws = w * s[None, :]
    amax = np.abs(ws.reshape(n, -1, 32)).max(axis=2)
    assert np.all(np.abs(deq - ws).reshape(n, -1, 32) <= (amax / 127 * 0.51 + amax * 2.0 ** -10)[:, :, None])


def test_weight_quantizer_is_ref_rounding_of_w_times_s(orc):
    """Exact pin: with power-of-two factors w*s is exact in fp32, so each weight row must
    quantize to the bytes quantize_row_q8_0_ref gives for w*s (the row quantizer is pinned
    by its own known answers); a divide by s, or the SIMD rounding, fails this."""
    rng = RNG(8)
    n, k = 16, 128
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    s = (2.0 ** rng.integers(-3, 4, k)).astype(np.float32)
    q = orc.quantize_weight_q8_0(w, s)
    ws = w * s
    for r in range(n):
        assert np.array_equal(q[r], orc.quantize_row_q8_0(ws[r], variant=orc.Q8_ROUND_REF).reshape(-1)), r
    assert not np.array_equal(q, orc.quantize_weight_q8_0(w / s))
    assert np.array_equal(orc.quantize_weight_q8_0(w), orc.quantize_weight_q8_0(w, np.ones(k, np.float32)))


# ---------------------------------------------------------------- Q4_0

def test_q4_0_dequant_closed_form(orc):
    # one block: nibbles j (low) and 15-j (high) with d = 0.5
    qs = np.array([(j & 15) | ((15 - j) << 4) for j in range(16)], dtype=np.uint8)
    blk = np.concatenate([f16_bits([0.5]).view(np.uint8), qs])
    y = orc.dequantize_q4_0(blk, 32).reshape(-1)
    want = np.array([(j - 8) * 0.5 for j in range(16)] + [(15 - j - 8) * 0.5 for j in range(16)], np.float32)
    assert np.array_equal(y, want)


def test_q4_0_gemv_vs_fp64(orc):
    rng = RNG(8)
    n, k = 256, 8960
    w = q4_0_weights(rng, n, k)
    x16 = f16_bits(rng.standard_normal(k))
    y = orc.mul_mat_q4_0_f16(w, x16, n, k)
    deq = orc.dequantize_q4_0(w, k).astype(np.float64)
    ref = deq @ x16.view(np.float16).astype(np.float64)
    assert rel_err(y, ref) < 1e-5
    assert rel_err(orc.mul_mat_q4_0_f16_f64(w, x16, n, k), ref) < 1e-12
    assert rel_err(orc.mul_mat_q4_0_f16_mt(w, x16, n, k, n_threads=4), ref) < 1e-5


# ---------------------------------------------------------------- F16

def test_f16_gemv_vs_fp64(orc):
    rng = RNG(9)
    n, k = 300, 1536
    w16 = f16_bits(rng.standard_normal((n, k)) * 0.02)
    x = rng.standard_normal(k).astype(np.float32)
    xr = x.astype(np.float16).astype(np.float64)  # ggml rounds src1 to its vec_dot type
    ref = w16.view(np.float16).astype(np.float64) @ xr
    assert rel_err(orc.mul_mat_f16(w16, x, n, k), ref) < 1e-5
    assert rel_err(orc.mul_mat_f16_f64(w16, x, n, k), ref) < 1e-12
    assert rel_err(orc.mul_mat_f16_mt(w16, x, n, k, n_threads=4), ref) < 1e-5


# ---------------------------------------------------------------- attention

def _attn_inputs(rng, L, nq, nkv, d):
    q = rng.standard_normal((nq, d)).astype(np.float32)
    k = f16_bits(rng.standard_normal((L, nkv, d)))
    v = f16_bits(rng.standard_normal((L, nkv, d)))
    return q, k, v


def _numpy_attention(q, k, v, nkv, scale, mask=None):
    nq, d = q.shape
    qh = q.astype(np.float16).astype(np.float64)
    kf = k.view(np.float16).astype(np.float64)
    vf = v.view(np.float16).astype(np.float64)
    out = np.zeros((nq, d))
    g = nq // nkv
    for h in range(nq):
        s = kf[:, h // g, :] @ qh[h] * scale
        if mask is not None:
            s = s + mask.view(np.float16).astype(np.float64)[: len(s)]
        if np.all(np.isneginf(s)):
            continue
        p = np.exp(s - s.max())
        out[h] = p @ vf[:, h // g, :] / p.sum()
    return out


@pytest.mark.parametrize("L", [1, 7, 240, 241, 513])
def test_attention_f64_mode_matches_numpy(orc, L):
    rng = RNG(10 + L)
    q, k, v = _attn_inputs(rng, L, 12, 2, 128)
    o = orc.flash_attn_ext_1tok(q, k, v, 2, 1 / np.sqrt(128), mode=1)
    assert np.abs(o - _numpy_attention(q, k, v, 2, 1 / np.sqrt(128))).max() < 1e-6


def test_attention_special_cases(orc):
    rng = RNG(11)
    q, k, v = _attn_inputs(rng, 1, 12, 2, 128)
    for mode in (0, 1):
        o = orc.flash_attn_ext_1tok(q, k, v, 2, 0.088, mode=mode)
        vf = v.view(np.float16).astype(np.float32)
        # L = 1: the output is V[0] of the head's kv group exactly
        assert np.array_equal(o[:6], np.broadcast_to(vf[0, 0], (6, 128)))
        assert np.array_equal(o[6:], np.broadcast_to(vf[0, 1], (6, 128)))
    q0 = np.zeros((12, 128), np.float32)
    _, k, v = _attn_inputs(rng, 300, 12, 2, 128)
    o = orc.flash_attn_ext_1tok(q0, k, v, 2, 0.088, mode=1)
    # q = 0: uniform softmax -> mean of V
    mean = v.view(np.float16).astype(np.float64).mean(axis=0)
    assert np.abs(o[0] - mean[0]).max() < 1e-6 and np.abs(o[11] - mean[1]).max() < 1e-6


def test_attention_gqa_equals_repeated_mha(orc):
    rng = RNG(12)
    q, k, v = _attn_inputs(rng, 200, 8, 2, 128)
    o = orc.flash_attn_ext_1tok(q, k, v, 2, 0.1, mode=0)
    krep = np.repeat(k, 4, axis=1)
    vrep = np.repeat(v, 4, axis=1)
    o2 = orc.flash_attn_ext_1tok(q, krep, vrep, 8, 0.1, mode=0)
    assert np.array_equal(o, o2)


def test_attention_mask_and_kv_len(orc):
    rng = RNG(13)
    L = 500
    q, k, v = _attn_inputs(rng, L, 12, 2, 128)
    mask = np.zeros(L, np.float32)
    mask[300:] = -np.inf
    m16 = f16_bits(mask)
    for mode in (0, 1):
        a = orc.flash_attn_ext_1tok(q, k, v, 2, 0.1, mask=m16, mode=mode)
        b = orc.flash_attn_ext_1tok(q, k[:300].copy(), v[:300].copy(), 2, 0.1, mode=mode)
        c = orc.flash_attn_ext_1tok(q, k, v, 2, 0.1, kv_len=300, mode=mode)
        assert np.array_equal(a, b) and np.array_equal(a, c)
    # fully masked row: ggml writes zeros (S == 0 -> S_inv = 0)
    allm = f16_bits(np.full(L, -np.inf, np.float32))
    assert not orc.flash_attn_ext_1tok(q, k, v, 2, 0.1, mask=allm, mode=0).any()


@pytest.mark.parametrize("L,expect", [(1, 1.0), (2047, 1.0), (2048, 1.0), (2049, 2048 / 2049), (4096, 0.5),
                                      (6144, 1 / 3)])
def test_attention_ggml_mode_fp16_accumulator_kat(orc, L, expect):
    """Closed form of ggml-CPU's fp16 V accumulator.  q = 0 scores every position 0, so every
    softmax weight is exactly 1 and the fp32 sum S counts the positions; with V = 1 the fp16
    accumulator counts too, but fp16 spacing is 2 above 2048, so 2048 + 1 rounds (to even)
    back to 2048 and the count stops there: output = min(L, 2048) / L.  An fp32 or fp64
    accumulator would give 1.0 for every L; the exact mode must."""
    d = 128
    q = np.zeros((2, d), np.float32)
    k = f16_bits(RNG(L).standard_normal((L, 1, d)))
    v = f16_bits(np.ones((L, 1, d)))
    o = orc.flash_attn_ext_1tok(q, k, v, 1, 1 / np.sqrt(d), mode=0)
    assert np.all(o == np.float32(expect)), (o[0, 0], expect)
    assert np.all(orc.flash_attn_ext_1tok(q, k, v, 1, 1 / np.sqrt(d), mode=1) == 1.0)


def test_attention_ggml_mode_mask_rescale_kat(orc):
    """Three positions worked by hand, scale 1, one query head, D = 2.
    q = (1, 0); K rows (0, 0), (2, 0), (5, 0); mask (0, -1, -inf); V rows (1, 0), (0, 1), (7, 7).
      p0: s = 0           -> M = 0, acc = V0 = (1, 0), S = 1
      p1: s = 2 - 1 = 1   -> new max: ms = e^-1, acc = fp16(acc * ms) + V1, S = ms + 1
      p2: masked (-inf)   -> skipped, V2 never read into the sum
    so out = (fp16(e^-1), 1) / (1 + e^-1): the first component carries the rescaled fp16
    accumulator (0.367919921875 = 1507 * 2^-12), the second a clean 1.  The exact answer has
    e^-1 there instead."""
    import math
    q = np.array([[1.0, 0.0]], np.float32)
    k = f16_bits([[[0.0, 0.0]], [[2.0, 0.0]], [[5.0, 0.0]]])
    v = f16_bits([[[1.0, 0.0]], [[0.0, 1.0]], [[7.0, 7.0]]])
    mask = f16_bits([0.0, -1.0, -np.inf])
    ms = np.float32(math.exp(-1.0))
    S = np.float32(ms + np.float32(1.0))
    acc0 = np.float32(np.float16(ms))
    assert acc0 == np.float32(1507 * 2.0 ** -12)
    o = orc.flash_attn_ext_1tok(q, k, v, 1, 1.0, mask=mask, mode=0)
    inv = np.float32(1.0) / S
    assert o[0, 0] == acc0 * inv and o[0, 1] == np.float32(1.0) * inv, o
    ex = orc.flash_attn_ext_1tok(q, k, v, 1, 1.0, mask=mask, mode=1)
    e1 = math.exp(-1.0)
    assert abs(ex[0, 0] - e1 / (1 + e1)) < 1e-7 and abs(ex[0, 1] - 1 / (1 + e1)) < 1e-7


def test_attention_ggml_mode_error_and_simd(orc):
    """The ggml-CPU restatement keeps the V accumulator in fp16 (ggml_vec_mad_f16); its distance
    to the exact answer is what bounds the achievable GPU-vs-ggml agreement."""
    rng = RNG(14)
    for L in (64, 4096):
        q, k, v = _attn_inputs(rng, L, 12, 2, 128)
        o0 = orc.flash_attn_ext_1tok(q, k, v, 2, 1 / np.sqrt(128), mode=0)
        o1 = orc.flash_attn_ext_1tok(q, k, v, 2, 1 / np.sqrt(128), mode=1)
        assert np.abs(o0 - o1).max() < 4e-3
        assert np.array_equal(orc.flash_attn_ext_1tok(q, k, v, 2, 1 / np.sqrt(128), n_threads=4), o0)


# ---------------------------------------------------------------- kv_lengths (patch:2900-2929)

def test_kv_lengths_kat(orc):
    mask = np.zeros((4, 10), np.float32)
    mask[0, 6:] = -np.inf          # trailing -inf -> 6
    mask[1, :] = -np.inf           # all masked -> minimum 1
    mask[2, 3] = -np.inf           # interior -inf does not shorten -> 10
    mask[3, 9] = np.nan            # NaN counts as non-finite -> 9
    assert list(orc.kv_lengths(mask, is_f16=False)) == [6, 1, 10, 9]
    assert list(orc.kv_lengths(f16_bits(mask), is_f16=True)) == [6, 1, 10, 9]


# ---------------------------------------------------------------- reference-side A8W8 scheme

def test_reference_per_channel_quant_and_nz_layout(orc):
    rng = RNG(15)
    k, n = 64, 64
    w = f16_bits(rng.standard_normal((n, k)) * 0.05)  # [column n][row k], ne0 = k
    q_nz, s = orc.quantize_a8w8_per_channel(w, k, n)
    wf = w.view(np.float16).astype(np.float32)
    scale = np.maximum(np.abs(wf).max(axis=1) / 127, 1e-8).astype(np.float32)
    assert np.array_equal(s, f16_bits(scale))
    # gather back through the FRACTAL_NZ 16x32 index of patch:1690-1691
    col = np.arange(n)[:, None]
    row = np.arange(k)[None, :]
    nz = (((col // 32) * (k // 16) + row // 16) * 16 + row % 16) * 32 + col % 32
    q = q_nz[nz]
    assert np.all(np.abs(q.astype(np.int32)) <= 127)
    assert np.all(np.abs(q * scale[:, None] - wf) <= 0.5 * scale[:, None] * 1.0001)


def test_reference_per_token_quant_kat(orc):
    xq, s = orc.quantize_per_token_i8(f16_bits(np.ones(1536)))
    assert np.all(xq == 127) and s == f16_bits([1 / 127])[0]
    # zero input: the 1.27e-6 floor keeps 127/maxAbs finite, so xq is 0 (not NaN garbage); the
    # stored fp16 scale 1e-8 underflows to 0 exactly as the kernel's static_cast<half> does
    xq, s = orc.quantize_per_token_i8(np.zeros(64, np.uint16))
    assert not xq.any() and s == 0
