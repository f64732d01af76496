#!/usr/bin/env python3
"""Decode throughput on one MI355X: Qwen2.5-1.5B-shaped A8W8 model, bs=1, through the
ggml backend (ggml_backend_mi355x) driven by the Qwen2 decode driver (mi_qwen2.h).

Prints ONE JSON line.  Phases:
  1. decode: a 512-token random-id context (fed in ubatches of 8 tokens; its rate is
     reported as config.prompt_tok_s), W untimed
     greedy decode steps, then K timed greedy decode steps; every step is the whole
     llama.cpp Qwen2 graph (RMSNorm, q/k/v/o/gate/up/down A8W8 Q8_0 projections with
     SmoothQuant, RoPE, fp16 KV cache write, GQA flash-decoding, SwiGLU, residuals,
     tied fp16 head, argmax) run by ggml_backend_graph_compute, replayed as a HIP graph;
     the argmax is read back to the host each step, as llama.cpp's sampler does.
     tokens/s = K / elapsed, bracketed by device synchronisation.  Both decode paths of
     the backend are timed: the persistent one (all 28 layers in one launch,
     GGML_MI355X_PERSIST=1; the headline) and the per-node one (one launch per fused node
     group, the backend's default, reported beside it); their greedy tokens are compared.
  2. roofline: the dominant kernel of the headline path, the persistent layer-stack
     launch, timed live with HIP events the backend records on its stream around each
     launch (GGML_MI355X_PERSIST_TIMING=1, launches run eagerly) over K decode steps of a
     second model at the same positions; its 1.39 GB of weights are over 5x the 256 MB
     MALL, so every launch streams them from HBM; achieved = algorithmic bytes (weights,
     vectors, K/V rows read and written) / average launch time.  Beside it, the per-node
     path's dominant kernel, the grouped gate+up Q8_0 GEMV of one layer (two 8960 x 1536
     matrices on one activation row, one launch), timed with HIP events over back-to-back
     launches on the stream they are issued to, rotating through enough weight copies
     (> 2x the MALL) to be HBM-cold.
  3. cpu_baseline: the ggml-CPU restatement in oracle/ (AVX2/AVX-512 VNNI, OpenMP) on a
     bounded sample of the same decode: it takes the GPU's KV cache after the warm-up
     steps and decodes K steps from the same token and position (at most ~15 s), then
     the same K steps again until at least 10 s are timed; its greedy tokens are compared
     with the GPU's timed tokens.

  4. configs: every other workload measured in the same run, each HBM-cold (rotating
     through copies of its weights or KV cache, more than 2x the 256 MB MALL) with live
     HIP-event timing, next to the same operation of the ggml-CPU restatement on the
     host's cores (median of 20 runs after warm-up):
       C1 the A8W8 Q8_0 GEMV 8960 x 1536 (activation quantization fused),
       C2 the W4A16 Q4_0 GEMV 1536 x 8960 on an fp16 row,
       C3 the GQA flash-decoding 12q/2kv D=128 at L = 512, 4096, 32768 (split + combine),
       C5 the Qwen2.5-7B-shaped W4A16 decode at a 32768-position context, 128 timed
          tokens at batch 1 and at batch 8, with the attention's KV-read rate.
     --quick skips this leg.

Synthetic data: random weights of the Qwen2.5-1.5B shape (28 layers, hidden 1536,
12 q / 2 kv heads of dim 128, FFN 8960, vocab 151936, fp16 tied head), SmoothQuant
factors uniform in [0.5, 2] (no checkpoints exist offline).
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "llama-cpp-ascend310b4-addon_amd"))

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20
PREFILL = 512
PROMPT_UBATCH = 8
SEED = 1234


T_START = time.perf_counter()


def log(msg):
    """progress on stderr (stdout carries only the JSON line)"""
    print(f"[bench {time.perf_counter() - T_START:6.1f} s] {msg}", file=sys.stderr, flush=True)


def cpu_threads():
    return min(16, os.cpu_count() or 1)


def host_info(orc, threads):
    model = "?"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"threads": threads, "nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
            "cpu_model": model, "isa": orc.simd_isa(),
            "pinning": "none: OpenMP default placement (OMP_NUM_THREADS=%s)" % os.environ.get("OMP_NUM_THREADS", "unset")}


def cold_launch_us(mi, st, launch, n_launches, plug):
    """average us per launch of launch(i), i = 0..n_launches-1, issued back to back behind a
    4 GiB device copy (the GPU is busy while they queue up, so they run back to back
    whatever the host's launch rate); HIP events on the launch stream; median of 3"""
    e0, e1 = mi.Event(), mi.Event()
    samples = []
    for _ in range(3):
        for _ in range(2):
            mi._call("mi_memcpy_d2d", mi._P(plug[1].ptr), mi._P(plug[0].ptr), 2 << 30, mi._P(st.ptr))
        e0.record(st.ptr)
        for i in range(n_launches):
            launch(i)
        e1.record(st.ptr)
        st.sync()
        samples.append(e0.elapsed_ms(e1) * 1e3 / n_launches)
    return float(np.median(samples))


def cpu_median_us(fn, reps=20, warm=3):
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)) * 1e6


def _rate(algo, us):
    return {"us": round(us, 3), "algorithmic_bytes": algo, "GBps": round(algo / us / 1e3, 1),
            "frac": round(algo / us / 1e3 / HBM_PEAK_GBS, 4)}


def measure_c1(mi, qs, orc, rng, st, plug, threads):
    """A8W8 Q8_0 GEMV N=8960 x K=1536, one fp32 row quantized in the kernel's prologue"""
    n, k = 8960, 1536
    blocks = qs.q8_0_rows(rng, n, k)
    psz = mi.q8_0_packed_size(n, k)
    copies = int(np.ceil(2 * MALL_BYTES / psz)) + 1
    src = mi.to_device(blocks)
    big = mi.DeviceBuffer(copies * psz)
    for c in range(copies):
        mi.prepack_q8_0(src.ptr, big.ptr + c * psz, n, k, stream=st.ptr)
    x = rng.standard_normal(k).astype(np.float32)
    dx, dy = mi.to_device(x), mi.DeviceBuffer(n * 4)
    fn = mi.lib().mi_mul_mat_q8_0_f32
    args = [(mi._P(st.ptr), mi._P(big.ptr + c * psz), mi._P(dx.ptr), None, mi._P(dy.ptr), n, k, 1, mi.Q8_ROUND_X86,
             None, 0) for c in range(copies)]
    us = cold_launch_us(mi, st, lambda i: fn(*args[i % copies]), 4 * copies, plug)
    cpu_us = cpu_median_us(lambda: orc.mul_mat_q8_0_mt(blocks, x, n, k, n_threads=threads))
    for b in (src, big, dx, dy):
        b.free()
    return dict(_rate(n * k // 32 * 34 + k * 4 + n * 4, us), kernel="k_gemv_q8_0_fused1 (act-quant fused, 1 launch)",
                shape=f"Q8_0 {n}x{k}, fp32 row", cpu_us=round(cpu_us, 1), weight_copies=copies)


def measure_c2(mi, qs, orc, rng, st, plug, threads):
    """W4A16 Q4_0 GEMV N=1536 x K=8960 on an fp16 activation row"""
    n, k = 1536, 8960
    blocks = qs.q4_0_rows(rng, n, k)
    psz = mi.q4_0_packed_size(n, k)
    copies = int(np.ceil(2 * MALL_BYTES / psz)) + 1
    src = mi.to_device(blocks)
    big = mi.DeviceBuffer(copies * psz)
    for c in range(copies):
        mi.prepack_q4_0(src.ptr, big.ptr + c * psz, n, k, stream=st.ptr)
    x16 = rng.standard_normal(k).astype(np.float32).astype(np.float16).view(np.uint16)
    dx, dy = mi.to_device(x16), mi.DeviceBuffer(n * 4)
    fn = mi.lib().mi_gemv_q4_0_f16
    args = [(mi._P(st.ptr), mi._P(big.ptr + c * psz), mi._P(dx.ptr), mi._P(dy.ptr), n, k, 1) for c in range(copies)]
    us = cold_launch_us(mi, st, lambda i: fn(*args[i % copies]), 4 * copies, plug)
    cpu_us = cpu_median_us(lambda: orc.mul_mat_q4_0_f16_mt(blocks, x16, n, k, n_threads=threads))
    for b in (src, big, dx, dy):
        b.free()
    return dict(_rate(n * k // 32 * 18 + k * 2 + n * 4, us), kernel="k_gemv_q4_0_kb", shape=f"Q4_0 {n}x{k}, fp16 row",
                cpu_us=round(cpu_us, 1), weight_copies=copies)


def measure_c3(mi, orc, rng, st, plug, threads, L):
    """GQA decode attention 12q/2kv D=128 over an fp16 KV cache of L positions (split + combine)"""
    nq, nkv, d = 12, 2, 128
    row = nkv * d * 2
    kvb = L * row
    copies = max(2, int(np.ceil(2 * MALL_BYTES / (2 * kvb))) + 1)
    kbig, vbig = mi.DeviceBuffer(copies * kvb), mi.DeviceBuffer(copies * kvb)
    for b, sd in ((kbig, 11), (vbig, 12)):
        mi._call("mi_fill_f16_uniform", mi._P(st.ptr), mi._P(b.ptr), copies * L, nkv * d, row, ctypes.c_uint64(sd),
                 ctypes.c_float(1.0))
    q = rng.standard_normal((nq, d)).astype(np.float32)
    dq, out = mi.to_device(q), mi.DeviceBuffer(nq * d * 4)
    wsb = mi.fa_decode_workspace_size(L, nq, nkv, d)
    ws = mi.DeviceBuffer(wsb).zero(stream=st.ptr)
    fn = mi.lib().mi_fa_decode
    scale = ctypes.c_float(1.0 / np.sqrt(d))
    args = [(mi._P(st.ptr), mi._P(dq.ptr), mi._P(kbig.ptr + c * kvb), mi._P(vbig.ptr + c * kvb), None, None, L, nq, nkv,
             d, row, d * 2, row, d * 2, scale, mi._P(out.ptr), mi._P(ws.ptr), wsb) for c in range(copies)]
    us = cold_launch_us(mi, st, lambda i: fn(*args[i % copies]), 4 * copies, plug)
    kc = rng.standard_normal((L, nkv, d)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((L, nkv, d)).astype(np.float16).view(np.uint16)
    cpu_us = cpu_median_us(lambda: orc.flash_attn_ext_1tok(q, kc, vc, nkv, 1.0 / np.sqrt(d), n_threads=threads))
    for b in (kbig, vbig, dq, out, ws):
        b.free()
    return dict(_rate(2 * kvb + 2 * nq * d * 4, us), kernel="k_fa_mfma + k_fa_combine",
                shape=f"12q/2kv D=128, L={L}", cpu_us=round(cpu_us, 1), kv_copies=copies)


def measure_configs(mi, qs, orc, threads):
    rng = np.random.default_rng(SEED + 7)
    st = mi.Stream()
    plug = (mi.DeviceBuffer(2 << 30), mi.DeviceBuffer(2 << 30))
    out = {"C1": measure_c1(mi, qs, orc, rng, st, plug, threads)}
    log("C1 done")
    out["C2"] = measure_c2(mi, qs, orc, rng, st, plug, threads)
    log("C2 done")
    for L in (512, 4096, 32768):
        out[f"C3_L{L}"] = measure_c3(mi, orc, rng, st, plug, threads, L)
        log(f"C3 L={L} done")
    for b in plug:
        b.free()
    st.destroy()
    return out


def measure_roofline(mi, qs, hp, rng):
    """the model's gate+up launch (RMSNorm * w, SmoothQuant, Q8_0 quantization fused, two
    8960 x 1536 matrices), HBM-cold, live HIP-event timing on the launch stream"""
    n, k = hp["n_ff"], hp["n_embd"]
    psz = mi.q8_0_packed_size(n, k)
    st = mi.Stream()
    src = mi.to_device(qs.q8_0_rows(rng, n, k))
    pair_bytes = 2 * psz
    copies = int(np.ceil(2 * MALL_BYTES / pair_bytes)) + 1
    bufs = []
    for _ in range(2 * copies):
        b = mi.DeviceBuffer(psz)
        mi.prepack_q8_0(src.ptr, b.ptr, n, k, stream=st.ptr)
        bufs.append(b)
    x = mi.to_device(rng.standard_normal(k).astype(np.float32))
    nw = mi.to_device(rng.uniform(0.8, 1.2, k).astype(np.float32))
    inv_s = mi.to_device((1.0 / rng.uniform(0.5, 2.0, k)).astype(np.float32))
    y0, y1 = mi.DeviceBuffer(n * 4), mi.DeviceBuffer(n * 4)
    plug_a, plug_b = mi.DeviceBuffer(2 << 30), mi.DeviceBuffer(2 << 30)
    st.sync()
    # weights + x + norm weight + 1/s + outputs
    algo = 2 * n * (k // 32) * 34 + 3 * k * 4 + 2 * n * 4
    launches = copies * 8
    # argument tuples built once: the launch loop is then one C call per launch
    fn = mi.lib().mi_mul_mat_q8_0_f32_fused
    ns = (ctypes.c_int64 * 2)(n, n)
    ys = (ctypes.c_void_p * 2)(y0.ptr, y1.ptr)
    adds = (ctypes.c_void_p * 2)(None, None)
    ws = [(ctypes.c_void_p * 2)(bufs[2 * c].ptr, bufs[2 * c + 1].ptr) for c in range(copies)]
    args = [(mi._P(st.ptr), 2, ctypes.cast(w, ctypes.c_void_p), ctypes.cast(ns, ctypes.c_void_p),
             ctypes.cast(ys, ctypes.c_void_p), ctypes.cast(adds, ctypes.c_void_p), k, mi._P(x.ptr), mi._P(nw.ptr),
             ctypes.c_float(hp["rms_eps"]), mi._P(inv_s.ptr), mi.Q8_ROUND_X86) for w in ws]
    e0, e1 = mi.Event(), mi.Event()
    samples = []
    for _ in range(3):
        # a 4 GiB device copy first keeps the GPU busy while the launches queue up, so
        # they run back to back whatever the host-side launch rate
        for _ in range(2):
            mi._call("mi_memcpy_d2d", mi._P(plug_b.ptr), mi._P(plug_a.ptr), 2 << 30, mi._P(st.ptr))
        e0.record(st.ptr)
        for i in range(launches):
            if fn(*args[i % copies]) != 0:
                raise mi.MiError("mi_mul_mat_q8_0_f32_fused", -1, mi.last_error())
        e1.record(st.ptr)
        samples.append(e0.elapsed_ms(e1) * 1e3 / launches)
    avg_us = float(np.median(samples))
    for b in bufs + [src, x, nw, inv_s, y0, y1, plug_a, plug_b]:
        b.free()
    st.destroy()
    achieved = algo / avg_us / 1e3
    # HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes over
    # `bench.py --roofline-only` (counters cannot be read from inside this process); used
    # only while the counted kernel is the one timed here
    kernel = "k_gemv_q8_0_fused1<16,3,2,true>"
    traffic, source = None, None
    tpath = os.path.join(ROOT, "profiles", "traffic_gate_up_q8_0.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            t = json.load(f)
        if t.get("kernel", "").replace(" ", "") == kernel:
            traffic = t.get("hbm_bytes_per_launch")
            source = "profiles/traffic_gate_up_q8_0.md (rocprofv3 --pmc of this kernel, " + t.get("measured", "?") + ")"
    return {"kernel": kernel + ": the gate+up launch of every layer (RMSNorm*w, SmoothQuant "
                      "and Q8_0 act-quant fused; 2 x Q8_0 8960x1536), HBM-cold", "bound": "hbm",
            "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": source,
            "avg_us": round(avg_us, 3), "algorithmic_bytes": algo, "launches": launches, "weight_copies": copies}


def persist_launch_bytes(qs, hp, kv_len):
    """algorithmic HBM bytes of one persistent launch (every layer of one decode token) when
    the attention reads kv_len positions: Q8_0 weights, q/k/v biases, the two RMSNorm
    weights, the four SmoothQuant 1/s rows, the K and V rows read and the new position's
    written, and the residual row in and out"""
    E, F, nkv = hp["n_embd"], hp["n_ff"], hp["n_head_kv"] * hp["head_dim"]
    per = sum(n * k // 32 * 34 for _, n, k, _ in qs.projections(hp))
    per += (E + 2 * nkv) * 4 + 2 * E * 4 + (3 * E + F) * 4
    per += kv_len * nkv * 2 * 2 + nkv * 2 * 2
    return hp["n_layer"] * per + 2 * E * 4


PERSIST_KERNEL = "k_persist_q8_0"


def measure_persist_roofline(mi, qs, hp, tensors, smooth, steps, warm):
    """the persistent layer-stack launch (all 28 layers of one decode token in one launch),
    timed live with HIP events that the backend records on its stream around each launch
    (GGML_MI355X_PERSIST_TIMING=1; launches run eagerly so every one is timed); the weights
    (1.39 GB) are over 5x the 256 MB MALL, so every launch streams them from HBM"""
    env = {"GGML_MI355X_PERSIST": "1", "GGML_MI355X_PERSIST_TIMING": "1", "GGML_MI355X_GRAPHS": "0"}
    saved = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        model = mi.Qwen2Model(hp)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    model.load(tensors, smooth)
    model.fill_cache(PREFILL, seed=SEED + 3, scale=1.0)
    nxt = 0
    if warm:
        wt, _ = model.decode_steps(0, PREFILL, warm)
        nxt = int(wt[-1])
    pos0 = PREFILL + warm
    n0, ms0 = model.persist_timing()
    model.decode_steps(nxt, pos0, steps)
    n1, ms1 = model.persist_timing()
    model.free()
    launches = n1 - n0
    if launches != steps:
        raise RuntimeError(f"persistent roofline: {launches} launches timed for {steps} decode steps "
                           "(the persistent path did not take every step)")
    avg_us = (ms1 - ms0) * 1e3 / launches
    algo = sum(persist_launch_bytes(qs, hp, pos0 + j + 1) for j in range(steps)) // steps
    achieved = algo / avg_us / 1e3
    traffic, source = None, None
    tpath = os.path.join(ROOT, "profiles", "traffic_persist_q8_0.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            t = json.load(f)
        if t.get("kernel") == PERSIST_KERNEL and t.get("first_position") == pos0 and t.get("steps") == steps:
            traffic = t.get("hbm_bytes_per_launch")
            source = "profiles/traffic_persist_q8_0.md (rocprofv3 --pmc of this kernel, " + t.get("measured", "?") + ")"
    return {"kernel": PERSIST_KERNEL + ": the persistent layer stack, all 28 layers of a decode token in one "
                      "launch of 256 workgroups (norms, A8W8 q/k/v + RoPE + KV write, flash-decoding, o, "
                      "gate/up + SwiGLU, down, residuals), weights HBM-cold", "bound": "hbm",
            "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": source,
            "avg_us": round(avg_us, 3), "algorithmic_bytes": algo, "launches": launches,
            "positions": [pos0 + 1, pos0 + steps]}


def cpu_baseline(qs, hp, tensors, smooth, model, token, pos, gpu_tokens, budget_s=15.0, min_s=10.0):
    """the ggml-CPU restatement decoding from the GPU's KV cache at `pos`, timed; the same
    steps are decoded again (same input tokens, rewriting the same cache rows) until at
    least min_s of CPU decode is timed; then the GPU re-decodes the CPU's steps (same input
    tokens, same positions) for the logit error"""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    threads = cpu_threads()
    cpu = orc.Qwen2(hp, tensors, smooth, fa_mode=0, n_threads=threads)
    for il in range(hp["n_layer"]):
        cpu.k_cache[il, :pos] = model.get_cache(il, 0, pos)
        cpu.v_cache[il, :pos] = model.get_cache(il, 1, pos)
    toks, inputs, logits = [], [], []
    t0 = time.perf_counter()
    nxt = token
    for i in range(len(gpu_tokens)):
        inputs.append(nxt)
        nxt, lg = cpu.decode(nxt, pos + i)
        toks.append(nxt)
        logits.append(lg)
        if time.perf_counter() - t0 >= budget_s:
            break
    n_steps, passes = len(toks), 1
    while time.perf_counter() - t0 < min_s:
        for i, t in enumerate(inputs):
            cpu.decode(t, pos + i)
        n_steps += len(inputs)
        passes += 1
    el = time.perf_counter() - t0
    err = rel = 0.0
    for i, (t, lc) in enumerate(zip(inputs, logits)):
        _, lg = model.decode(t, pos + i, want_logits=True)
        err = max(err, float(np.abs(lg - lc).max()))
        rel = max(rel, float(np.abs(lg - lc).max() / np.abs(lc).max()))
    agree = int(np.sum(np.asarray(toks) == np.asarray(gpu_tokens[:len(toks)])))
    first_diff = next((i for i, (a, b) in enumerate(zip(toks, gpu_tokens)) if a != b), None)
    return {"value": round(n_steps / el, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{len(toks)} greedy decode steps of the same model from the GPU's KV cache at position {pos}, "
                      f"{passes} pass(es), {n_steps} steps (ggml-CPU restatement in oracle/, {orc.simd_isa()}, "
                      f"{threads} threads, {el:.1f} s)",
            "greedy_agreement": f"{agree}/{len(toks)}", "first_divergence": first_diff,
            "logit_max_abs": round(err, 6), "logit_max_rel": round(rel, 6), "host": host_info(orc, threads)}


def measure_fa(mi, hp, n_seq, n_kv, rng):
    """flash-decoding at the model's attention shape over n_seq synthetic caches of n_kv
    positions (fresh buffers rotated, HBM-cold): KV-read GB/s of split + combine"""
    nq, nkv, d = hp["n_head"], hp["n_head_kv"], hp["head_dim"]
    st = mi.Stream()
    kv_bytes = n_seq * n_kv * nkv * d * 2
    copies = max(2, int(np.ceil(2 * MALL_BYTES / (2 * kv_bytes))) + 1)
    caches = []
    for c in range(copies):
        kb, vb = mi.DeviceBuffer(kv_bytes), mi.DeviceBuffer(kv_bytes)
        for b, sd in ((kb, 2 * c), (vb, 2 * c + 1)):
            mi._call("mi_fill_f16_uniform", mi._P(st.ptr), mi._P(b.ptr), n_seq * n_kv, nkv * d, nkv * d * 2,
                     ctypes.c_uint64(sd), ctypes.c_float(1.0))
        caches.append((kb, vb))
    q = mi.to_device(rng.standard_normal((n_seq, nq, d)).astype(np.float32))
    out = mi.DeviceBuffer(n_seq * nq * d * 4)
    wsb = mi.fa_decode_batch_workspace_size(n_kv, nq, nkv, d, n_seq)
    ws = mi.DeviceBuffer(wsb).zero(stream=st.ptr)
    nb1 = nkv * d * 2
    seq_b = n_kv * nb1
    run = lambda kb, vb: mi.fa_decode_batch(q.ptr, kb.ptr, vb.ptr, None, None, n_kv, nq, nkv, d, nb1, d * 2, nb1,
                                            d * 2, 1.0 / np.sqrt(d), out.ptr, n_seq, nq * d, seq_b, seq_b, 0, nq * d,
                                            ws.ptr, wsb, stream=st.ptr)
    for kb, vb in caches:
        run(kb, vb)
    st.sync()
    e0, e1 = mi.Event(), mi.Event()
    launches = 4 * copies
    e0.record(st.ptr)
    for i in range(launches):
        run(*caches[i % copies])
    e1.record(st.ptr)
    st.sync()
    us = e0.elapsed_ms(e1) * 1e3 / launches
    algo = 2 * kv_bytes + 2 * n_seq * nq * d * 4
    for kb, vb in caches:
        kb.free()
        vb.free()
    st.destroy()
    return {"kernel": "k_fa_mfma + k_fa_combine (flash-decoding, MFMA)", "n_seq": n_seq, "n_kv": n_kv,
            "heads": f"{nq}q/{nkv}kv", "avg_us": round(us, 2), "algorithmic_bytes": algo,
            "achieved": round(algo / us / 1e3, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(algo / us / 1e3 / HBM_PEAK_GBS, 4), "bound": "hbm"}


def decode_7b(mi, qs, hp, tensors, steps, warm):
    """one Qwen2.5-7B-shaped W4A16 model of hp["n_seq"] sequences: every sequence's KV cache
    filled on the device to n_ctx - steps - warm positions, warm untimed then `steps`
    timed greedy steps -> (seconds, first position, model)"""
    S = hp["n_seq"]
    model = mi.Qwen2Model(hp)
    model.load(tensors)
    n_fill = hp["n_ctx"] - steps - warm
    model.fill_cache(n_fill, seed=SEED, scale=1.0)
    rng = np.random.default_rng(SEED + 2)
    toks = rng.integers(0, hp["n_vocab"], S).astype(np.int32)
    pos = np.full(S, n_fill, np.int32)
    wt, _ = model.decode_steps_batch(toks, pos, warm)
    toks, pos = wt[-1], pos + warm
    mi.device_sync()
    t0 = time.perf_counter()
    model.decode_steps_batch(toks, pos, steps)
    mi.device_sync()
    return time.perf_counter() - t0, int(pos[0]), model


def c5_line(mi, qs, hp, el, pos0, steps, warm, weight_bytes, fa):
    S = hp["n_seq"]
    kv_step = qs.kv_bytes_per_position(hp) * S * (pos0 + steps // 2)
    step_bytes = weight_bytes + kv_step
    return {"tok_s": round(S * steps / el, 2), "ms_per_step": round(el * 1e3 / steps, 4), "batch": S,
            "steps": steps, "warmup": warm, "context": hp["n_ctx"], "bytes_per_step": step_bytes,
            "kv_bytes_per_step": kv_step, "step_GBps": round(step_bytes * steps / el / 1e9, 1),
            "kv_GBps_in_step": round(kv_step * steps / el / 1e9, 1),
            "step_roofline_frac": round(step_bytes * steps / el / 1e9 / HBM_PEAK_GBS, 4), "attention": fa}


def measure_c5(mi, qs, orc, threads, batches=(1, 8), steps=128, warm=8, cpu_steps=2):
    """Qwen2.5-7B-shaped W4A16 decode at context 32768 for each batch size, one weight
    synthesis shared by the models; a bounded CPU sample (cpu_steps tokens of sequence 0
    from the same filled cache) beside batch 1"""
    n_ctx = 32768
    hp1 = qs.qwen2_7b(n_ctx=n_ctx, n_seq=1)
    tensors, _ = qs.synth(hp1, seed=SEED)
    log("7B weights synthesized")
    wbytes = qs.weight_bytes(hp1)
    out = {}
    for S in batches:
        hp = qs.qwen2_7b(n_ctx=n_ctx, n_seq=S)
        el, pos0, model = decode_7b(mi, qs, hp, tensors, steps, warm)
        fa = measure_fa(mi, hp, S, n_ctx, np.random.default_rng(SEED + 3))
        line = c5_line(mi, qs, hp, el, pos0, steps, warm, wbytes, fa)
        if S == 1 and cpu_steps > 0:
            cpu = orc.Qwen2(hp1, tensors, None, fa_mode=0, n_threads=threads)
            n_pos = pos0 + steps - cpu_steps   # the positions the last timed GPU steps decoded
            for il in range(hp["n_layer"]):
                cpu.k_cache[il, :n_pos] = model.get_cache_seq(il, 0, 0, n_pos)
                cpu.v_cache[il, :n_pos] = model.get_cache_seq(il, 1, 0, n_pos)
            t0 = time.perf_counter()
            tok = 0
            for i in range(cpu_steps):
                tok, _ = cpu.decode(tok, n_pos + i)
            el_cpu = time.perf_counter() - t0
            line["cpu_baseline"] = {"value": round(cpu_steps / el_cpu, 3), "unit": "tok/s", "cores": threads,
                                    "kind": "port", "sample": f"{cpu_steps} decode steps of sequence 0 at position "
                                    f"{n_pos} (ggml-CPU restatement, {orc.simd_isa()}, {threads} threads)"}
            del cpu
        model.free()
        out[f"C5_bs{S}"] = line
        log(f"C5 bs={S}: {line['tok_s']} tok/s")
    return out


def run_7b(args, mi, qs):
    """--workload qwen2-7b-w4a16: the C5 decode as the headline line, bs = --batch sequences"""
    S = args.batch
    warm = max(args.warmup, 1)
    hp = qs.qwen2_7b(n_ctx=32768, n_seq=S)
    tensors, _ = qs.synth(dict(hp, n_seq=1), seed=SEED)
    el, pos0, model = decode_7b(mi, qs, hp, tensors, args.steps, warm)
    model.free()
    fa = None if args.no_roofline else measure_fa(mi, hp, S, hp["n_ctx"], np.random.default_rng(SEED + 3))
    line = c5_line(mi, qs, hp, el, pos0, args.steps, warm, qs.weight_bytes(hp), fa)
    return {
        "metric": f"decode tok/s, Qwen2.5-7B-shape W4A16 bs={S} at context 32768",
        "value": line["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": warm,
        "ms_per_step": line["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "W4A16 (int4 g32 weights x fp16 activations, fp32 accumulate), fp16 KV and head",
        "data": "synthetic (random weights of the named shape, random KV-cache contents of the named length)",
        "config": {"workload": f"Qwen2.5-7B-shaped Q4_0 W4A16 whole-model greedy decode, {S} independent sequence(s), "
                               "28 layers, hidden 3584, 28q/4kv heads x 128, FFN 18944, vocab 152064 tied fp16 head; "
                               f"KV cache of {pos0} positions per sequence, then the timed tokens", **line},
        "roofline": fa, "cpu_baseline": None,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of replaying HIP graphs")
    ap.add_argument("--no-roofline", action="store_true", help="skip the standalone roofline leg")
    ap.add_argument("--roofline-only", nargs="?", const="persistent", choices=["persistent", "gate-up"],
                    help="run only one roofline leg (a short program for rocprofv3 counter passes)")
    ap.add_argument("--workload", default="qwen2-1.5b-a8w8", choices=["qwen2-1.5b-a8w8", "qwen2-7b-w4a16"],
                    help="qwen2-7b-w4a16: the 7B-shaped W4A16 decode at a 32K context (see --batch)")
    ap.add_argument("--batch", type=int, default=1, help="independent sequences for qwen2-7b-w4a16 (1..8)")
    ap.add_argument("--quick", action="store_true", help="skip the configs leg (C1, C2, C3, C5)")
    ap.add_argument("--decode-path", default="persistent", choices=["per-node", "persistent"],
                    help="the C4 headline's decode path (the other one is timed too and reported beside it); "
                         "the roofline is that path's dominant launch, the other path's is reported beside it")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); how the decode path "
              "would shard across GPUs is described in the design notes, not implemented", file=sys.stderr)
        sys.exit(2)
    if args.no_graph:
        os.environ["GGML_MI355X_GRAPHS"] = "0"

    import ggml_mi355x as mi
    import qwen2_synth as qs
    if mi.device_count() < 1:
        print("bench.py: no HIP device: " + mi.last_error(), file=sys.stderr)
        sys.exit(1)

    if args.workload == "qwen2-7b-w4a16":
        print(json.dumps(run_7b(args, mi, qs)))
        return

    warm = max(args.warmup, 0)
    hp = qs.qwen2_1p5b(n_ctx=PREFILL + warm + args.steps)
    if args.roofline_only == "gate-up":
        print(json.dumps({"roofline": measure_roofline(mi, qs, hp, np.random.default_rng(SEED + 1))}))
        return
    tensors, smooth = qs.synth(hp, seed=SEED)
    if args.roofline_only == "persistent":
        print(json.dumps({"roofline": measure_persist_roofline(mi, qs, hp, tensors, smooth, args.steps, warm)}))
        return

    def c4_run(persistent):
        """the C4 decode through one of the backend's two decode paths; returns the model
        (still loaded), the last token, the first timed position, the timed tokens and
        the elapsed seconds"""
        os.environ["GGML_MI355X_PERSIST"] = "1" if persistent else "0"
        model = mi.Qwen2Model(hp)
        model.load(tensors, smooth)
        rng = np.random.default_rng(SEED + 1)
        prompt = rng.integers(0, hp["n_vocab"], PREFILL)
        log(f"1.5B model loaded ({'persistent' if persistent else 'per-node'} decode)")
        # context: the 512-token prompt in ubatches of 8 (bit-identical to one token per
        # step for Q8_0 weights); fed twice, the second time timed (the first builds and
        # captures the ubatch graphs), then the warm-up decode steps
        model.prefill(prompt, 0, PROMPT_UBATCH)
        nxt, _, prompt_s = model.prefill(prompt, 0, PROMPT_UBATCH)
        prompt_rate[persistent] = PREFILL / prompt_s
        if warm:
            wt, _ = model.decode_steps(nxt, PREFILL, warm)
            nxt = int(wt[-1])
        pos0 = PREFILL + warm
        mi.device_sync()
        t0 = time.perf_counter()
        toks, _ = model.decode_steps(nxt, pos0, args.steps)
        mi.device_sync()
        return model, nxt, pos0, toks, time.perf_counter() - t0

    persistent = args.decode_path == "persistent"
    prompt_rate = {}
    # the other path first (its model freed), then the headline path
    other, _, _, other_toks, other_el = c4_run(not persistent)
    other.free()
    other_tok_s = args.steps / other_el
    log(f"C4 decode, {'per-node' if persistent else 'persistent'} path: {other_tok_s:.1f} tok/s")
    model, nxt, pos0, toks, el = c4_run(persistent)
    tok_s = args.steps / el
    step_bytes = qs.weight_bytes(hp) + qs.kv_bytes_per_position(hp) * (pos0 + args.steps // 2)
    rng = np.random.default_rng(SEED + 2)

    log(f"C4 decode: {tok_s:.1f} tok/s")
    roof = roof_other = None
    if not args.no_roofline:
        roof_p = measure_persist_roofline(mi, qs, hp, tensors, smooth, args.steps, warm)
        log("persistent roofline leg done")
        roof_g = measure_roofline(mi, qs, hp, rng)
        log("gate+up roofline leg done")
        roof, roof_other = (roof_p, roof_g) if persistent else (roof_g, roof_p)
    cpu = None if args.no_cpu else cpu_baseline(qs, hp, tensors, smooth, model, nxt, pos0, list(toks))
    model.free()
    del tensors, smooth
    configs = None
    if not args.quick:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as orc
        configs = measure_configs(mi, qs, orc, cpu_threads())
        configs.update(measure_c5(mi, qs, orc, cpu_threads()))

    out = {
        "metric": "decode tok/s, Qwen2.5-1.5B-shape bs=1; GEMV HBM GB/s as % of peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": warm,
        "ms_per_step": round(el * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 A8W8 (Q8_0 dots, int32 accumulate), fp16 KV cache and head, fp32 elsewhere",
        "data": "synthetic (random weights of the named shape, random token ids)",
        "config": {
            "workload": "Qwen2.5-1.5B-shaped A8W8 Q8_0 + SmoothQuant whole-model greedy decode, bs=1: 28 layers, "
                        "hidden 1536, 12q/2kv heads x 128, FFN 8960, vocab 151936 tied fp16 head; 512-token "
                        "context then the timed decode tokens, through ggml_backend_graph_compute",
            "context": PREFILL, "graph": not args.no_graph,
            "decode_path": args.decode_path + (" (one persistent launch for the 28 layers, GGML_MI355X_PERSIST=1)"
                                               if persistent else " (one launch per fused node group)"),
            "other_path_tok_s": round(other_tok_s, 2),
            "other_path_same_tokens": [int(t) for t in other_toks] == [int(t) for t in toks],
            "prompt_tok_s": round(prompt_rate[persistent], 1),
            "prompt": f"the {PREFILL}-token context fed in ubatches of {PROMPT_UBATCH} (mi_qwen2_prefill, one graph "
                      "per ubatch: several-row GEMVs and flash-decoding over the ubatch's query rows under the causal "
                      "mask), the second of two passes timed",
            "bytes_per_step": step_bytes,
            "step_GBps": round(step_bytes * args.steps / el / 1e9, 1),
            "step_roofline_frac": round(step_bytes * args.steps / el / 1e9 / HBM_PEAK_GBS, 4),
        },
        "roofline": roof,
        ("roofline_gate_up" if persistent else "roofline_persistent"): roof_other,
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
