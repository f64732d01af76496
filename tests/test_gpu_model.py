"""Whole-model decode through the ggml backend (ggml_backend_mi355x + the Qwen2 driver)
against the CPU restatement of the same llama.cpp Qwen2 graph (oracle/qwen2_oracle.c).

Bar: greedy tokens identical to the ggml-CPU restatement step by step (both fed the same
tokens), with the logit max-abs error stated; logits within a relative 2e-3 of the CPU
model whose attention is exact (fp64), which isolates the backend from ggml-CPU's fp16
attention accumulator -- or, for Q8_0 models, within 3x the spread between two ggml-CPU
builds when that is larger.  Q8_0 activation quantization is discontinuous: an fp32
rounding difference upstream can move an activation across a rounding boundary, so the
logits depend on the summation order of every earlier dot.  ggml's own SIMD (AVX2/VNNI)
and generic builds differ by up to ~1e-2 relative on a 1536-wide model; the spread is
measured in the test by running the CPU model both ways.
"""
import numpy as np
import pytest

import lldump
from synth import rel_err
import qwen2_synth as qs

pytestmark = pytest.mark.gpu


def a8w8_reference(orc, hp, tensors, smooth):
    """The CPU model of an F16 model run on the A8W8 path: every projection W (F16) with
    its SmoothQuant factors s becomes the Q8_0 blocks of W*diag(s) by the oracle's weight
    quantizer (quantize_row_q8_0_ref, what the backend does on the device at upload)."""
    q = dict(tensors)
    for il in range(hp["n_layer"]):
        for name, n, k, _ in qs.projections(hp):
            key = f"blk.{il}.{name}.weight"
            w = tensors[key].view(np.float16).astype(np.float32).reshape(n, k)
            q[key] = orc.quantize_weight_q8_0(w, smooth.get(key))
    return dict(hp, wtype=qs.GGML_TYPE_Q8_0), q


def _run(gpu, orc, hp, n_prompt, n_gen, seed, threads=8):
    mi = gpu
    tensors, smooth = qs.synth(hp, seed=seed, qk_gain=6.0)   # peaked attention
    model = mi.Qwen2Model(hp)
    model.load(tensors, smooth)
    chp, ct = (hp, tensors) if hp["wtype"] != qs.GGML_TYPE_F16 else a8w8_reference(orc, hp, tensors, smooth)
    cpu = orc.Qwen2(chp, ct, smooth, fa_mode=0, n_threads=threads)
    cpu_exact = orc.Qwen2(chp, ct, smooth, fa_mode=1, n_threads=threads)
    q8 = chp["wtype"] == qs.GGML_TYPE_Q8_0
    cpu_generic = orc.Qwen2(chp, ct, smooth, fa_mode=1, n_threads=threads, q8_generic=True) if q8 else None
    rng = np.random.default_rng(seed + 1)
    tokens = list(rng.integers(0, hp["n_vocab"], n_prompt))
    max_err_ggml = max_rel_exact = spread = 0.0
    mismatches = 0
    nxt = None
    for pos in range(n_prompt + n_gen):
        tok = tokens[pos] if pos < n_prompt else nxt
        g_tok, g_log = model.decode(tok, pos, want_logits=True)
        c_tok, c_log = cpu.decode(tok, pos)
        e_tok, e_log = cpu_exact.decode(tok, pos)
        max_err_ggml = max(max_err_ggml, float(np.abs(g_log - c_log).max()))
        scale = float(np.abs(e_log).max())
        max_rel_exact = max(max_rel_exact, float(np.abs(g_log - e_log).max()) / scale)
        if cpu_generic is not None:
            spread = max(spread, float(np.abs(cpu_generic.decode(tok, pos)[1] - e_log).max()) / scale)
        if pos >= n_prompt - 1:
            mismatches += int(g_tok != c_tok)
        nxt = g_tok
    model.free()
    print(f"{hp['n_layer']}L x {hp['n_embd']}: logit max-abs vs ggml-CPU {max_err_ggml:.3e}, "
          f"rel vs exact-attention CPU {max_rel_exact:.3e} (ggml SIMD/generic spread {spread:.3e}), "
          f"greedy mismatches {mismatches}/{n_gen + 1}")
    return max_err_ggml, max_rel_exact, spread, mismatches


def _bar(spread):
    return max(2e-3, 3.0 * spread)


def test_qwen2_small_q8_0(gpu, orc):
    hp = qs.qwen2_1p5b(n_layer=2, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_ff=512, n_vocab=1000,
                       n_ctx=300)
    err, rel, spread, mism = _run(gpu, orc, hp, n_prompt=260, n_gen=24, seed=3)
    assert rel < _bar(spread)
    assert mism == 0


def test_qwen2_small_q4_0(gpu, orc):
    hp = qs.qwen2_1p5b(n_layer=2, n_embd=256, n_head=4, n_head_kv=1, head_dim=64, n_ff=512, n_vocab=1000,
                       n_ctx=64, wtype=qs.GGML_TYPE_Q4_0)
    err, rel, spread, mism = _run(gpu, orc, hp, n_prompt=8, n_gen=24, seed=4)
    assert rel < 2e-3
    assert mism == 0


def test_qwen2_1p5b_width_two_layers(gpu, orc):
    """Full Qwen2.5-1.5B width (hidden 1536, 12/2 heads of 128, FFN 8960, vocab 151936), two layers."""
    hp = qs.qwen2_1p5b(n_layer=2, n_ctx=64)
    err, rel, spread, mism = _run(gpu, orc, hp, n_prompt=16, n_gen=16, seed=5)
    assert rel < _bar(spread)
    assert mism == 0


def test_qwen2_7b_width_two_layers_q4_0(gpu, orc):
    """Qwen2.5-7B width with W4A16 projections (hidden 3584, 28/4 heads of 128, FFN 18944,
    vocab 152064), two layers: the fused W4A16 chains at their real shapes."""
    hp = qs.qwen2_7b(n_layer=2, n_ctx=64)
    err, rel, spread, mism = _run(gpu, orc, hp, n_prompt=8, n_gen=8, seed=6)
    assert rel < 2e-3
    assert mism == 0


def test_qwen2_a8w8_from_f16_weights(gpu, orc, monkeypatch):
    """An F16 model on the A8W8 path (GGML_MI355X_A8W8=1, the reference's GGML_CANN_A8W8) at
    the full Qwen2.5-1.5B width: every projection is quantized at upload to Q8_0 of
    W*diag(s).  Its logits must be bit-identical to the same backend running the Q8_0 model
    the oracle's weight quantizer makes of the same F16 weights (so the upload path adds
    nothing), and its greedy tokens identical to the CPU model of that Q8_0 model."""
    mi = gpu
    monkeypatch.setenv("GGML_MI355X_A8W8", "1")
    monkeypatch.delenv("GGML_MI355X_A8W8_DISABLE_LAYERS", raising=False)
    hp = qs.qwen2_1p5b(n_layer=2, n_ctx=64, wtype=qs.GGML_TYPE_F16)
    tensors, smooth = qs.synth(hp, seed=15)
    f16 = mi.Qwen2Model(hp)
    f16.load(tensors, smooth)
    qhp, qt = a8w8_reference(orc, hp, tensors, smooth)
    q8 = mi.Qwen2Model(qhp)
    q8.load(qt, smooth)
    cpu = orc.Qwen2(qhp, qt, smooth, fa_mode=0, n_threads=8)
    rng = np.random.default_rng(16)
    tok, worst, mism = None, 0.0, 0
    for pos in range(32):
        t = int(rng.integers(0, hp["n_vocab"])) if pos < 16 else tok
        ta, la = f16.decode(t, pos, want_logits=True)
        tb, lb = q8.decode(t, pos, want_logits=True)
        tc, lc = cpu.decode(t, pos)
        assert ta == tb and np.array_equal(la, lb), f"position {pos}"
        worst = max(worst, float(np.abs(la - lc).max() / np.abs(lc).max()))
        mism += int(pos >= 15 and ta != tc)
        tok = ta
    print(f"A8W8 from F16, 2L x 1536: logits bit-identical to the oracle-quantized Q8_0 model; rel vs ggml-CPU "
          f"{worst:.3e}, greedy mismatches {mism}/17")
    assert mism == 0
    f16.free()
    q8.free()


@pytest.mark.parametrize("wtype", [qs.GGML_TYPE_Q8_0, qs.GGML_TYPE_Q4_0])
def test_fused_graph_matches_unfused(gpu, monkeypatch, wtype):
    """The backend's fused launches against its node-by-node path on the same graph."""
    mi = gpu
    hp = qs.qwen2_1p5b(n_layer=2, n_ctx=64, wtype=wtype)
    tensors, smooth = qs.synth(hp, seed=9, qk_gain=6.0)
    fused = mi.Qwen2Model(hp)
    fused.load(tensors, smooth)
    monkeypatch.setenv("GGML_MI355X_FUSION", "0")
    plain = mi.Qwen2Model(hp)
    plain.load(tensors, smooth)
    rng = np.random.default_rng(10)
    tok_f = tok_p = None
    worst = 0.0
    identical = True
    for pos in range(24):
        t = int(rng.integers(0, hp["n_vocab"])) if pos < 8 else tok_f
        tok_f, lf = fused.decode(t, pos, want_logits=True)
        tok_p, lp = plain.decode(t, pos, want_logits=True)
        identical = identical and np.array_equal(lf, lp)
        worst = max(worst, float(np.abs(lf - lp).max() / np.abs(lp).max()))
        assert tok_f == tok_p, f"position {pos}"
    print(f"fused vs node-by-node: logits bit-identical {identical}, max rel {worst:.3e}")
    assert worst < 1e-4
    fused.free()
    plain.free()


@pytest.mark.parametrize("wtype", [qs.GGML_TYPE_Q8_0, qs.GGML_TYPE_Q4_0])
def test_fused_graph_matches_unfused_long_context(gpu, monkeypatch, wtype):
    """As above from a 600-position cache (KV view of 768 rows: 12 attention splits)."""
    mi = gpu
    hp = qs.qwen2_1p5b(n_layer=2, n_ctx=1024, wtype=wtype)
    tensors, smooth = qs.synth(hp, seed=19, qk_gain=6.0)
    fused = mi.Qwen2Model(hp)
    fused.load(tensors, smooth)
    monkeypatch.setenv("GGML_MI355X_FUSION", "0")
    plain = mi.Qwen2Model(hp)
    plain.load(tensors, smooth)
    start = 600
    fused.fill_cache(start, seed=3, scale=1.0)
    plain.fill_cache(start, seed=3, scale=1.0)
    tok = 17
    worst = 0.0
    for pos in range(start, start + 8):
        tok_f, lf = fused.decode(tok, pos, want_logits=True)
        tok_p, lp = plain.decode(tok, pos, want_logits=True)
        worst = max(worst, float(np.abs(lf - lp).max() / np.abs(lp).max()))
        assert tok_f == tok_p, f"position {pos}"
        tok = tok_f
    print(f"fused vs node-by-node at context {start}: max rel {worst:.3e}")
    assert worst < 1e-4
    fused.free()
    plain.free()


@pytest.mark.parametrize("wtype", [qs.GGML_TYPE_Q4_0, qs.GGML_TYPE_Q8_0])
def test_fused_graph_matches_unfused_batch(gpu, monkeypatch, wtype):
    """A ubatch of 4 sequences (one token each): the backend's fused launches (grouped
    q/k/v + bias, gate/up, GLU + down + residual on the Q4_0 path) against its node-by-node
    path, logits bit-identical."""
    mi = gpu
    n_seq = 4
    hp = qs.qwen2_1p5b(n_layer=2, n_ctx=64, wtype=wtype, n_seq=n_seq)
    tensors, smooth = qs.synth(hp, seed=29, qk_gain=6.0)
    fused = mi.Qwen2Model(hp)
    fused.load(tensors, smooth)
    monkeypatch.setenv("GGML_MI355X_FUSION", "0")
    plain = mi.Qwen2Model(hp)
    plain.load(tensors, smooth)
    rng = np.random.default_rng(30)
    toks = rng.integers(0, hp["n_vocab"], n_seq)
    for pos in range(12):
        tf, lf = fused.decode_batch(toks, [pos] * n_seq, want_logits=True)
        tp, lp = plain.decode_batch(toks, [pos] * n_seq, want_logits=True)
        assert np.array_equal(lf, lp), f"position {pos}: max rel {np.abs(lf - lp).max() / np.abs(lp).max():.3e}"
        assert np.array_equal(tf, tp)
        toks = tf
    fused.free()
    plain.free()


def test_fused_graph_matches_unfused_batch_7b_width(gpu, monkeypatch):
    """A ubatch of 4 sequences at the Qwen2.5-7B width (W4A16, 28/4 heads of 128, FFN
    18944, two layers): the fused launches at their real shapes (q/k/v with RoPE pairs and
    the cache writes, the combine writing the o projection's activation, gate/up GLU
    pairs, the matrix-core head) against the node-by-node path, logits bit-identical."""
    mi = gpu
    n_seq = 4
    hp = qs.qwen2_7b(n_layer=2, n_ctx=48, n_seq=n_seq)
    tensors, smooth = qs.synth(hp, seed=31)
    fused = mi.Qwen2Model(hp)
    fused.load(tensors, smooth)
    monkeypatch.setenv("GGML_MI355X_FUSION", "0")
    plain = mi.Qwen2Model(hp)
    plain.load(tensors, smooth)
    rng = np.random.default_rng(32)
    toks = rng.integers(0, hp["n_vocab"], n_seq)
    for pos in range(6):
        tf, lf = fused.decode_batch(toks, [pos] * n_seq, want_logits=True)
        tp, lp = plain.decode_batch(toks, [pos] * n_seq, want_logits=True)
        assert np.array_equal(lf, lp), f"position {pos}: max rel {np.abs(lf - lp).max() / np.abs(lp).max():.3e}"
        assert np.array_equal(tf, tp)
        toks = tf
    fused.free()
    plain.free()


@pytest.mark.parametrize("wtype", [qs.GGML_TYPE_Q4_0, qs.GGML_TYPE_Q8_0])
def test_qwen2_batch_of_sequences(gpu, orc, wtype):
    """Three sequences decoded together (one ubatch of 3 tokens per step, per-sequence KV
    streams) against three independent CPU runs: greedy tokens identical per sequence."""
    mi = gpu
    n_seq, n_prompt, n_gen = 3, 12, 12
    hp = qs.qwen2_1p5b(n_layer=2, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_ff=512, n_vocab=1000,
                       n_ctx=40, wtype=wtype, n_seq=n_seq)
    tensors, smooth = qs.synth(hp, seed=21, qk_gain=6.0)
    model = mi.Qwen2Model(hp)
    model.load(tensors, smooth)
    assert model.n_seq == n_seq
    cpus = [orc.Qwen2(hp, tensors, smooth, fa_mode=1, n_threads=4) for _ in range(n_seq)]
    gens = [orc.Qwen2(hp, tensors, smooth, fa_mode=1, n_threads=4, q8_generic=True) for _ in range(n_seq)] \
        if wtype == qs.GGML_TYPE_Q8_0 else None
    rng = np.random.default_rng(22)
    prompts = rng.integers(0, hp["n_vocab"], (n_seq, n_prompt))
    nxt = [0] * n_seq
    worst = spread = 0.0
    mism = 0
    for pos in range(n_prompt + n_gen):
        toks = [int(prompts[s, pos]) if pos < n_prompt else int(nxt[s]) for s in range(n_seq)]
        g_tok, g_log = model.decode_batch(toks, [pos] * n_seq, want_logits=True)
        for s in range(n_seq):
            c_tok, c_log = cpus[s].decode(toks[s], pos)
            scale = float(np.abs(c_log).max())
            worst = max(worst, float(np.abs(g_log[s] - c_log).max()) / scale)
            if gens is not None:
                spread = max(spread, float(np.abs(gens[s].decode(toks[s], pos)[1] - c_log).max()) / scale)
            if pos >= n_prompt - 1:
                mism += int(g_tok[s] != c_tok)
        nxt = g_tok
    model.free()
    print(f"batch of {n_seq} ({'Q8_0' if wtype == qs.GGML_TYPE_Q8_0 else 'Q4_0'}): rel vs exact-attention CPU "
          f"{worst:.3e} (ggml SIMD/generic spread {spread:.3e}), greedy mismatches {mism}/{n_seq * (n_gen + 1)}")
    assert worst < _bar(spread)
    assert mism == 0


@pytest.mark.parametrize("wtype,n_ubatch", [(qs.GGML_TYPE_Q8_0, 8), (qs.GGML_TYPE_Q4_0, 8), (qs.GGML_TYPE_Q8_0, 3)])
def test_qwen2_prompt_ubatches(gpu, orc, wtype, n_ubatch):
    """The prompt fed in ubatches of n_ubatch tokens (mi_qwen2_prefill: MUL_MATs of several
    rows, FLASH_ATTN_EXT with several query rows under llama.cpp's causal mask, the last
    token's logits) against the same model fed one token per step on the GPU and against
    the CPU models fed one token per step.

    Bar: with Q8_0 weights the ubatch path is bit-identical to the one-token path (logits,
    every K/V cache row, and the greedy steps decoded afterwards: the several-row GEMV keeps
    each row's block order); with Q4_0 weights (matrix-core several-row GEMVs) within a
    relative 2e-3.  Against the CPU at the prompt's end: logits within the whole-model bar
    of this file and the same greedy token."""
    mi = gpu
    n_prompt, n_gen = 261, 8   # a ragged last ubatch; KV views of 256 and 320 positions
    hp = qs.qwen2_1p5b(n_layer=2, n_ctx=320, n_vocab=32000, wtype=wtype)
    tensors, smooth = qs.synth(hp, seed=27, qk_gain=6.0)
    model, ref = mi.Qwen2Model(hp), mi.Qwen2Model(hp)
    model.load(tensors, smooth)
    ref.load(tensors, smooth)
    cpu = orc.Qwen2(hp, tensors, smooth, fa_mode=0, n_threads=8)
    exact = orc.Qwen2(hp, tensors, smooth, fa_mode=1, n_threads=8)
    q8 = wtype == qs.GGML_TYPE_Q8_0
    gen = orc.Qwen2(hp, tensors, smooth, fa_mode=1, n_threads=8, q8_generic=True) if q8 else None
    rng = np.random.default_rng(28)
    prompt = [int(t) for t in rng.integers(0, hp["n_vocab"], n_prompt)]
    g_tok, g_log, _ = model.prefill(prompt, 0, n_ubatch, want_logits=True)
    spread = 0.0
    for pos, tok in enumerate(prompt):
        r_tok, r_log = ref.decode(tok, pos, want_logits=True)
        c_tok, c_log = cpu.decode(tok, pos)
        e_tok, e_log = exact.decode(tok, pos)
        if gen is not None:
            spread = max(spread, float(np.abs(gen.decode(tok, pos)[1] - e_log).max()) / float(np.abs(e_log).max()))
    scale = float(np.abs(e_log).max())
    rel_tbt = float(np.abs(g_log - r_log).max()) / scale
    cache_diff = 0.0
    for il in range(hp["n_layer"]):
        for is_v in (0, 1):
            a = model.get_cache(il, is_v, n_prompt).view(np.float16).astype(np.float32)
            b = ref.get_cache(il, is_v, n_prompt).view(np.float16).astype(np.float32)
            cache_diff = max(cache_diff, float(np.abs(a - b).max()))
    err_ggml = float(np.abs(g_log - c_log).max())
    rel = float(np.abs(g_log - e_log).max()) / scale
    print(f"prompt in ubatches of {n_ubatch} ({'Q8_0' if q8 else 'Q4_0'}): vs one token per step on the GPU: "
          f"logits rel {rel_tbt:.3e}, cache max-abs {cache_diff:.3e}; vs CPU: logit max-abs {err_ggml:.3e}, "
          f"rel vs exact-attention {rel:.3e} (ggml SIMD/generic spread {spread:.3e}); greedy {g_tok} / {r_tok} / {c_tok}")
    if q8:
        assert rel_tbt == 0.0 and cache_diff == 0.0
    else:
        assert rel_tbt < 2e-3
    assert g_tok == r_tok == c_tok
    assert rel < _bar(spread)
    tok = g_tok
    for pos in range(n_prompt, n_prompt + n_gen):
        g_tok, g_log = model.decode(tok, pos, want_logits=True)
        r_tok, r_log = ref.decode(tok, pos, want_logits=True)
        if q8:
            assert np.array_equal(g_log, r_log), f"position {pos}"
        else:
            assert float(np.abs(g_log - r_log).max()) / float(np.abs(r_log).max()) < 2e-3, f"position {pos}"
        tok = g_tok
    model.free()
    ref.free()


def test_smooth_scale_file_and_layer_dump(gpu, tmp_path):
    """A SmoothQuant scale file (fp32 [layers, hidden], the scale tool's format) gives the
    same logits as the per-weight factors; the LLDUMP1 dump holds every layer's output per
    step, and the last layer's output through the output norm and the tied head gives the
    logits the step returned."""
    mi = gpu
    hp = qs.qwen2_1p5b(n_layer=2, n_ctx=64, wtype=qs.GGML_TYPE_Q8_0)
    tensors, smooth = qs.synth(hp, seed=41)
    L, E = hp["n_layer"], hp["n_embd"]
    sq = np.stack([smooth[f"blk.{i}.ffn_gate.weight"] for i in range(L)]).astype("<f4")
    assert all(np.array_equal(smooth[f"blk.{i}.ffn_up.weight"], sq[i]) for i in range(L))
    sq_path = tmp_path / "sq-scales-a05.bin"
    sq.tofile(sq_path)
    a = mi.Qwen2Model(hp)
    a.load(tensors, smooth)
    b = mi.Qwen2Model(hp)
    b.load(tensors, {k: v for k, v in smooth.items() if ".ffn_gate." not in k and ".ffn_up." not in k})
    with pytest.raises(mi.MiError, match=r"must already hold W\*diag\(s\)"):
        b.load_smooth_file(sq_path)            # Q8_0 weights: only when asserted pre-smoothed
    b.load_smooth_file(sq_path, weights_presmoothed=True)
    with pytest.raises(mi.MiError, match="no decode step"):
        a.dump_layers(tmp_path / "early.bin")
    dump = tmp_path / "layers.bin"
    rng = np.random.default_rng(42)
    for pos in range(6):
        t = int(rng.integers(0, hp["n_vocab"]))
        ta, la = a.decode(t, pos, want_logits=True)
        tb, lb = b.decode(t, pos, want_logits=True)
        assert ta == tb and np.array_equal(la, lb), f"position {pos}"
        b.dump_layers(dump, append=pos > 0)
    d = lldump.read_dump(dump)
    assert sorted(d) == [f"l_out-{i}" for i in range(L)]
    assert all(len(v) == 6 and all(r.size == E and np.isfinite(r).all() for r in v) for v in d.values())
    x = d[f"l_out-{L - 1}"][-1].astype(np.float64)
    xn = x / np.sqrt(np.mean(x * x) + hp["rms_eps"]) * tensors["output_norm.weight"]
    head = tensors["token_embd.weight"].view(np.float16).astype(np.float64).reshape(hp["n_vocab"], E)
    ref = head @ xn
    err = float(np.abs(lb - ref).max() / np.abs(ref).max())
    print(f"logits from the dumped l_out-{L - 1}: max rel {err:.2e}")
    assert err < 2e-3
    a.dump_layers(tmp_path / "a.bin")
    rows = lldump.compare(lldump.read_dump(tmp_path / "a.bin"), {k: v[-1:] for k, v in d.items()})
    assert [r[1] for r in rows] == [f"l_out-{i}" for i in range(L)]
    assert all(r[3] == pytest.approx(1.0) and r[4] == 0.0 for r in rows)
    a.free()
    b.free()


def test_layer_dump_ffn_records(gpu, orc, tmp_path):
    """With the layer dump on, each step writes ffn_norm-N, ffn_out-N, l_out-N per layer (the
    records the reference's SmoothQuant collector and layer comparison read); the fusions that
    would skip writing ffn_norm / ffn_out give way, and the logits stay bit-identical to the
    fused model's.  Closed forms tie the records together: ffn_norm = RMSNorm(l_out - ffn_out)
    * w, and ffn_out is the FFN (oracle matmuls) of ffn_norm."""
    mi = gpu
    hp = qs.qwen2_1p5b(n_layer=2, n_ctx=64, wtype=qs.GGML_TYPE_Q8_0)
    tensors, smooth = qs.synth(hp, seed=43)
    L, E, F = hp["n_layer"], hp["n_embd"], hp["n_ff"]
    a = mi.Qwen2Model(hp)
    a.load(tensors, smooth)
    b = mi.Qwen2Model(hp)
    b.load(tensors, smooth)
    b.set_layer_dump(True)
    dump = tmp_path / "d.bin"
    rng = np.random.default_rng(44)
    for pos in range(4):
        t = int(rng.integers(0, hp["n_vocab"]))
        ta, la = a.decode(t, pos, want_logits=True)
        tb, lb = b.decode(t, pos, want_logits=True)
        assert ta == tb and np.array_equal(la, lb), f"position {pos}"
        b.dump_layers(dump, append=pos > 0)
    d = lldump.LayerDump(dump)
    assert d.names == [f"{kind}-{i}" for i in range(L) for kind in ("ffn_norm", "ffn_out", "l_out")]
    for i in range(L):
        fn, fo, lo = d.matrix(f"ffn_norm-{i}"), d.matrix(f"ffn_out-{i}"), d.matrix(f"l_out-{i}")
        assert fn.shape == fo.shape == lo.shape == (4, E)
        inp = (lo - fo)[-1]
        w = tensors[f"blk.{i}.ffn_norm.weight"].astype(np.float64)
        ref_norm = inp / np.sqrt(np.mean(inp * inp) + hp["rms_eps"]) * w
        assert rel_err(fn[-1], ref_norm) < 1e-4, i
        x = fn[-1].astype(np.float32)
        p = f"blk.{i}."
        g = orc.mul_mat_q8_0(tensors[p + "ffn_gate.weight"], x, F, E, inv_s=1 / smooth[p + "ffn_gate.weight"])
        u = orc.mul_mat_q8_0(tensors[p + "ffn_up.weight"], x, F, E, inv_s=1 / smooth[p + "ffn_up.weight"])
        h = (g / (1 + np.exp(-g)) * u).astype(np.float32)
        down = orc.mul_mat_q8_0(tensors[p + "ffn_down.weight"], h, E, F, inv_s=1 / smooth[p + "ffn_down.weight"])
        assert rel_err(fo[-1], down) < 2e-2, i
    # what smoothquant-collect.py takes from such a dump: per layer the max |ffn_norm| channel
    amax = np.stack([np.abs(d.matrix(f"ffn_norm-{i}")).max(axis=0) for i in range(L)])
    assert amax.shape == (L, E) and np.all(amax > 0)
    b.set_layer_dump(False)
    tb2, lb2 = b.decode(5, 4, want_logits=True)
    ta2, la2 = a.decode(5, 4, want_logits=True)
    assert tb2 == ta2 and np.array_equal(lb2, la2)
    a.free()
    b.free()
