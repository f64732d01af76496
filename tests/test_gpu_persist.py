"""The persistent layer-stack decode (GGML_MI355X_PERSIST=1: one launch runs every
decoder layer of an A8W8 token) against the backend's per-node launches on the same
model and inputs, and against the CPU restatement of the graph.

Bar: logits bit-identical to the per-node path at every step (the persistent phases
compute what the per-node kernels compute, in the same order), greedy tokens identical
to the ggml-CPU restatement.  The error path is forced from the host: a hop whose waits
expect one arrival too many (GGML_MI355X_PERSIST_STALL_HOP) with a short spin limit
ends every workgroup through the kernel's error word, the decode reports the failure,
and the next decode of the same token is correct again.
"""
import numpy as np
import pytest

import qwen2_synth as qs

pytestmark = pytest.mark.gpu


def _pair(mi, monkeypatch, hp, seed, mask=None):
    # mask: MI_QWEN2_KQ_MASK for both models ("1" causal, "swa:N" a sliding window)
    if mask is not None:
        monkeypatch.setenv("MI_QWEN2_KQ_MASK", mask)
    tensors, smooth = qs.synth(hp, seed=seed, qk_gain=6.0)
    monkeypatch.setenv("GGML_MI355X_PERSIST", "0")
    node = mi.Qwen2Model(hp)
    node.load(tensors, smooth)
    monkeypatch.setenv("GGML_MI355X_PERSIST", "1")
    pers = mi.Qwen2Model(hp)
    pers.load(tensors, smooth)
    monkeypatch.delenv("GGML_MI355X_PERSIST")
    monkeypatch.delenv("MI_QWEN2_KQ_MASK", raising=False)
    return node, pers


def _assert_persistent_runs(mi, monkeypatch, hp, seed, mask):
    # a fresh model of this configuration whose first launch stalls a hop: the decode
    # fails only when the persistent launch runs (a silent per-node fallback would pass)
    monkeypatch.setenv("MI_QWEN2_KQ_MASK", mask)
    monkeypatch.setenv("GGML_MI355X_PERSIST", "1")
    m = mi.Qwen2Model(hp)
    m.load(*qs.synth(hp, seed=seed, qk_gain=6.0))
    monkeypatch.setenv("GGML_MI355X_PERSIST_SPIN", "20000")
    monkeypatch.setenv("GGML_MI355X_PERSIST_STALL_HOP", "1")
    with pytest.raises(mi.MiError, match="gave up waiting"):
        m.decode(3, 0)
    for k in ("MI_QWEN2_KQ_MASK", "GGML_MI355X_PERSIST", "GGML_MI355X_PERSIST_SPIN", "GGML_MI355X_PERSIST_STALL_HOP"):
        monkeypatch.delenv(k)
    m.free()


def _same_steps(node, pers, start, n, tok, label):
    for pos in range(start, start + n):
        tn, ln = node.decode(tok, pos, want_logits=True)
        tp, lp = pers.decode(tok, pos, want_logits=True)
        assert np.array_equal(ln, lp), f"{label}: position {pos}: max |diff| {np.abs(ln - lp).max():.3e}"
        assert tn == tp
        tok = tn
    return tok


@pytest.mark.parametrize("start", [0, 300, 600, 1000])
def test_persistent_matches_per_node(gpu, monkeypatch, start):
    # attention views of 256, 512, 768 and 1024 positions: 4, 8, 12 and 16 splits
    hp = qs.qwen2_1p5b(n_layer=3, n_ctx=1024, wtype=qs.GGML_TYPE_Q8_0)
    node, pers = _pair(gpu, monkeypatch, hp, seed=31 + start)
    if start:
        node.fill_cache(start, seed=4, scale=1.0)
        pers.fill_cache(start, seed=4, scale=1.0)
    n = 24 if start + 24 <= 1024 else 1024 - start
    _same_steps(node, pers, start, n, 23, f"context {start}")
    print(f"persistent == per-node, {hp['n_layer']} layers, {n} steps from position {start}")
    node.free()
    pers.free()


def test_persistent_full_depth(gpu, monkeypatch):
    # the Qwen2.5-1.5B decode stack (28 layers) from a 512-position cache
    hp = qs.qwen2_1p5b(n_layer=28, n_ctx=576, wtype=qs.GGML_TYPE_Q8_0)
    node, pers = _pair(gpu, monkeypatch, hp, seed=41)
    node.fill_cache(512, seed=6, scale=1.0)
    pers.fill_cache(512, seed=6, scale=1.0)
    _same_steps(node, pers, 512, 16, 5, "28 layers")
    node.free()
    pers.free()


def test_persistent_beyond_its_views_falls_back(gpu, monkeypatch):
    # a 1280-position view needs 20 splits: the per-node launches run it, same results
    hp = qs.qwen2_1p5b(n_layer=2, n_ctx=1536, wtype=qs.GGML_TYPE_Q8_0)
    node, pers = _pair(gpu, monkeypatch, hp, seed=51)
    node.fill_cache(1100, seed=7, scale=1.0)
    pers.fill_cache(1100, seed=7, scale=1.0)
    _same_steps(node, pers, 1100, 4, 9, "context 1100")
    node.free()
    pers.free()


@pytest.mark.parametrize("start", [0, 600])
def test_persistent_with_kq_mask(gpu, monkeypatch, start):
    # the graph with llama.cpp's KQ mask beside the kv lengths: the persistent launch
    # adds the mask row like the per-node attention, and a causal mask (0 up to the
    # position, -inf after it, all beyond the kv length) changes no bit
    hp = qs.qwen2_1p5b(n_layer=3, n_ctx=1024, wtype=qs.GGML_TYPE_Q8_0)
    _assert_persistent_runs(gpu, monkeypatch, hp, 81, "1")
    node, pers = _pair(gpu, monkeypatch, hp, seed=81, mask="1")
    plain, spare = _pair(gpu, monkeypatch, hp, seed=81)
    spare.free()
    for m in (node, pers, plain):
        if start:
            m.fill_cache(start, seed=8, scale=1.0)
    tok = 17
    for pos in range(start, start + 12):
        tn, ln = node.decode(tok, pos, want_logits=True)
        tp, lp = pers.decode(tok, pos, want_logits=True)
        tu, lu = plain.decode(tok, pos, want_logits=True)
        assert np.array_equal(ln, lp), f"position {pos}: persistent {np.abs(ln - lp).max():.3e} from per-node"
        assert np.array_equal(ln, lu), f"position {pos}: masked {np.abs(ln - lu).max():.3e} from unmasked"
        assert tn == tp == tu
        tok = tn
    for m in (node, pers, plain):
        m.free()


def test_persistent_with_sliding_window_mask(gpu, monkeypatch):
    # a mask that drops positions inside the kv length (the last 200 kept): persistent ==
    # per-node bit for bit, and the logits move away from the causal-only ones
    hp = qs.qwen2_1p5b(n_layer=3, n_ctx=1024, wtype=qs.GGML_TYPE_Q8_0)
    _assert_persistent_runs(gpu, monkeypatch, hp, 91, "swa:200")
    node, pers = _pair(gpu, monkeypatch, hp, seed=91, mask="swa:200")
    causal, spare = _pair(gpu, monkeypatch, hp, seed=91, mask="1")
    spare.free()
    for m in (node, pers, causal):
        m.fill_cache(700, seed=9, scale=1.0)
    tok, moved = 29, 0
    for pos in range(700, 710):
        tn, ln = node.decode(tok, pos, want_logits=True)
        tp, lp = pers.decode(tok, pos, want_logits=True)
        _, lc = causal.decode(tok, pos, want_logits=True)
        assert np.array_equal(ln, lp), f"position {pos}: persistent {np.abs(ln - lp).max():.3e} from per-node"
        assert tn == tp
        moved += not np.array_equal(ln, lc)
        tok = tn
    assert moved == 10
    for m in (node, pers, causal):
        m.free()


def test_persistent_greedy_matches_oracle(gpu, orc, monkeypatch):
    # the per-node oracle check at full 1.5B width (test_gpu_model) with the persistent
    # launch serving every token: a 64-position view, one attention split
    from test_gpu_model import _bar, _run
    monkeypatch.setenv("GGML_MI355X_PERSIST", "1")
    hp = qs.qwen2_1p5b(n_layer=2, n_ctx=64)
    err, rel, spread, mism = _run(gpu, orc, hp, n_prompt=16, n_gen=16, seed=5)
    assert rel < _bar(spread)
    assert mism == 0


@pytest.mark.parametrize("hop", [0, 2, 4])
def test_persistent_stalled_hop_reports_and_recovers(gpu, monkeypatch, hop):
    hp = qs.qwen2_1p5b(n_layer=2, n_ctx=64, wtype=qs.GGML_TYPE_Q8_0)
    node, pers = _pair(gpu, monkeypatch, hp, seed=71)
    tok = 11
    for pos in range(3):  # a few good steps first (the graph is replayed from the second)
        tok = _same_steps(node, pers, pos, 1, tok, "before the stall")
    # a fresh model: its first graph runs eagerly, launching with the hooks set below
    monkeypatch.setenv("GGML_MI355X_PERSIST", "1")
    stalled = gpu.Qwen2Model(hp)
    stalled.load(*qs.synth(hp, seed=71, qk_gain=6.0))
    monkeypatch.setenv("GGML_MI355X_PERSIST_SPIN", "20000")
    monkeypatch.setenv("GGML_MI355X_PERSIST_STALL_HOP", str(hop))
    with pytest.raises(gpu.MiError, match="gave up waiting"):
        stalled.decode(11, 0)
    monkeypatch.delenv("GGML_MI355X_PERSIST_SPIN")
    monkeypatch.delenv("GGML_MI355X_PERSIST_STALL_HOP")
    # the same token again (its cache rows are rewritten), then more steps: all correct
    monkeypatch.setenv("GGML_MI355X_PERSIST", "0")
    ref = gpu.Qwen2Model(hp)
    ref.load(*qs.synth(hp, seed=71, qk_gain=6.0))
    _same_steps(ref, stalled, 0, 6, 11, f"after a stall on hop {hop}")
    for m in (node, pers, stalled, ref):
        m.free()


def test_persistent_launch_timing(gpu, monkeypatch):
    # GGML_MI355X_PERSIST_TIMING: every eager persistent launch is timed with events on the
    # backend's stream and counted; graph replays are not; results are unchanged
    hp = qs.qwen2_1p5b(n_layer=3, n_ctx=64, wtype=qs.GGML_TYPE_Q8_0)
    tensors, smooth = qs.synth(hp, seed=61, qk_gain=6.0)
    monkeypatch.setenv("GGML_MI355X_PERSIST", "0")
    ref = gpu.Qwen2Model(hp)
    ref.load(tensors, smooth)
    monkeypatch.setenv("GGML_MI355X_PERSIST", "1")
    with pytest.raises(gpu.MiError, match="timing is off"):
        ref.persist_timing()
    monkeypatch.setenv("GGML_MI355X_PERSIST_TIMING", "1")
    monkeypatch.setenv("GGML_MI355X_GRAPHS", "0")
    eager = gpu.Qwen2Model(hp)
    eager.load(tensors, smooth)
    monkeypatch.delenv("GGML_MI355X_GRAPHS")
    replay = gpu.Qwen2Model(hp)
    replay.load(tensors, smooth)
    for k in ("GGML_MI355X_PERSIST", "GGML_MI355X_PERSIST_TIMING"):
        monkeypatch.delenv(k)
    assert eager.persist_timing() == (0, 0.0)
    want, _ = ref.decode_steps(7, 0, 8)
    got, _ = eager.decode_steps(7, 0, 8)
    assert np.array_equal(want, got)
    n, ms = eager.persist_timing()
    assert n == 8 and 0.0 < ms < 8 * 50.0, (n, ms)
    got, _ = replay.decode_steps(7, 0, 8)
    assert np.array_equal(want, got)
    n, _ = replay.persist_timing()
    assert 1 <= n < 8, n  # the first graph runs eagerly; the captured replays are not timed
    for m in (ref, eager, replay):
        m.free()
