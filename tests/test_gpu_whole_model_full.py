"""Whole-model parity at the workload sizes, GPU through the ggml backend against the CPU
restatement of the same llama.cpp Qwen2 graph (oracle/qwen2_oracle.c), both fed the same
tokens from empty or identically filled caches (no KV hand-off from one side to the
other).

  - Qwen2.5-1.5B shape, 28 layers, A8W8 Q8_0 + SmoothQuant: a 512-token random prompt,
    one token per step on both sides, then 64 greedy tokens.
  - Qwen2.5-7B shape, 28 layers, W4A16 Q4_0: every sequence's KV cache filled to 32764
    positions by one seeded fill (on the device, copied to the CPU models), then 4 greedy
    steps, for 1 sequence and for 8 independent sequences.

Bar: the greedy token of every generated step identical to the ggml-CPU restatement's.
The logit max-abs errors against that restatement and against the CPU model with exact
(fp64) attention are printed (the numbers the design notes quote)."""
import os
import time

import numpy as np
import pytest

import qwen2_synth as qs

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)


def _margin(logits):
    top = np.partition(logits, -2)[-2:]
    return float(top[1] - top[0])


@pytest.mark.timeout(900)
def test_qwen2_1p5b_a8w8_prompt512_then_64_greedy(gpu, orc):
    mi = gpu
    n_prompt, n_gen = 512, 64
    hp = qs.qwen2_1p5b(n_ctx=n_prompt + n_gen + 8)
    tensors, smooth = qs.synth(hp, seed=1234)
    model = mi.Qwen2Model(hp)
    model.load(tensors, smooth)
    cpu = orc.Qwen2(hp, tensors, smooth, fa_mode=0, n_threads=THREADS)
    exact = orc.Qwen2(hp, tensors, smooth, fa_mode=1, n_threads=THREADS)
    prompt = np.random.default_rng(1235).integers(0, hp["n_vocab"], n_prompt)
    err_ggml = err_exact_rel = 0.0
    mism, gen = [], []
    t0 = time.time()
    nxt = None
    for pos in range(n_prompt + n_gen):
        tok = int(prompt[pos]) if pos < n_prompt else nxt
        g_tok, g_log = model.decode(tok, pos, want_logits=True)
        c_tok, c_log = cpu.decode(tok, pos)
        _, e_log = exact.decode(tok, pos)
        err_ggml = max(err_ggml, float(np.abs(g_log - c_log).max()))
        err_exact_rel = max(err_exact_rel, float(np.abs(g_log - e_log).max() / np.abs(e_log).max()))
        if pos >= n_prompt - 1:
            gen.append(g_tok)
            if g_tok != c_tok:
                mism.append((pos, g_tok, c_tok, _margin(c_log)))
        nxt = g_tok
        if pos % 64 == 63:
            print(f"  position {pos + 1}: {time.time() - t0:.0f} s", flush=True)
    model.free()
    print(f"1.5B A8W8 28L, prompt {n_prompt} + {n_gen} greedy: logit max-abs vs ggml-CPU restatement "
          f"{err_ggml:.3e}, max rel vs exact-attention CPU {err_exact_rel:.3e}, greedy mismatches "
          f"{len(mism)}/{n_gen + 1} {mism}, {time.time() - t0:.0f} s; tokens {gen[:8]}...")
    assert not mism


@pytest.mark.timeout(1200)
@pytest.mark.parametrize("n_seq", [1, 8])
def test_qwen2_7b_w4a16_context_32k(gpu, orc, n_seq):
    mi = gpu
    n_steps = 4
    n_fill = 32768 - n_steps
    hp = qs.qwen2_7b(n_ctx=32768, n_seq=n_seq)
    t0 = time.time()
    tensors, _ = qs.synth(hp, seed=2024)
    print(f"  7B weights synthesized: {time.time() - t0:.0f} s", flush=True)
    model = mi.Qwen2Model(hp)
    model.load(tensors)
    model.fill_cache(n_fill, seed=2025, scale=1.0)
    print(f"  loaded, caches filled: {time.time() - t0:.0f} s", flush=True)
    chp = dict(hp, n_seq=1)
    cpus = [orc.Qwen2(chp, tensors, None, fa_mode=0, n_threads=THREADS) for _ in range(n_seq)]
    exact = orc.Qwen2(chp, tensors, None, fa_mode=1, n_threads=THREADS) if n_seq == 1 else None
    for s, cpu in enumerate(cpus):
        for il in range(hp["n_layer"]):
            for is_v, cache in ((0, cpu.k_cache), (1, cpu.v_cache)):
                cache[il, :n_fill] = model.get_cache_seq(il, is_v, s, n_fill)
                if exact is not None:
                    (exact.v_cache if is_v else exact.k_cache)[il, :n_fill] = cache[il, :n_fill]
    print(f"  caches copied to the CPU models: {time.time() - t0:.0f} s", flush=True)
    toks = np.random.default_rng(2026).integers(0, hp["n_vocab"], n_seq).astype(np.int32)
    err_ggml = err_exact_rel = 0.0
    mism = []
    for step in range(n_steps):
        pos = np.full(n_seq, n_fill + step, np.int32)
        g_tok, g_log = model.decode_batch(toks, pos, want_logits=True)
        for s, cpu in enumerate(cpus):
            c_tok, c_log = cpu.decode(int(toks[s]), int(pos[s]))
            err_ggml = max(err_ggml, float(np.abs(g_log[s] - c_log).max()))
            if g_tok[s] != c_tok:
                mism.append((step, s, int(g_tok[s]), c_tok, _margin(c_log)))
            if exact is not None:
                _, e_log = exact.decode(int(toks[s]), int(pos[s]))
                err_exact_rel = max(err_exact_rel, float(np.abs(g_log[s] - e_log).max() / np.abs(e_log).max()))
        toks = g_tok.astype(np.int32)
        print(f"  step {step + 1}/{n_steps}: {time.time() - t0:.0f} s", flush=True)
    model.free()
    print(f"7B W4A16 28L, {n_seq} sequence(s) at context {n_fill}, {n_steps} greedy steps: logit max-abs vs "
          f"ggml-CPU restatement {err_ggml:.3e}" + (f", max rel vs exact-attention CPU {err_exact_rel:.3e}"
                                                   if exact is not None else "") +
          f", greedy mismatches {len(mism)}/{n_seq * n_steps} {mism}, {time.time() - t0:.0f} s")
    assert not mism
