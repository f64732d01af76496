#!/usr/bin/env python3
"""Decode throughput on one MI355X: Qwen2.5-1.5B-shaped A8W8 model, bs=1, through the
ggml backend (ggml_backend_mi355x) driven by the Qwen2 decode driver (mi_qwen2.h).

Prints ONE JSON line.  Phases:
  1. decode: a 512-token random-id context (one token per step, untimed), W untimed
     greedy decode steps, then K timed greedy decode steps; every step is the whole
     llama.cpp Qwen2 graph (RMSNorm, q/k/v/o/gate/up/down A8W8 Q8_0 projections with
     SmoothQuant, RoPE, fp16 KV cache write, GQA flash-decoding, SwiGLU, residuals,
     tied fp16 head, argmax) run by ggml_backend_graph_compute, replayed as a HIP graph;
     the argmax is read back to the host each step, as llama.cpp's sampler does.
     tokens/s = K / elapsed, bracketed by device synchronisation.
  2. roofline: the dominant kernel, the grouped gate+up Q8_0 GEMV of one layer (two
     8960 x 1536 matrices on one activation row, one launch), timed live with HIP events
     over back-to-back launches on the stream they are issued to, rotating through enough
     weight copies (> 2x the 256 MB MALL) to be HBM-cold; achieved = algorithmic bytes /
     average launch time.
  3. cpu_baseline: the ggml-CPU restatement in oracle/ (AVX2/AVX-512 VNNI, OpenMP) on a
     bounded sample of the same decode: it takes the GPU's KV cache after the warm-up
     steps and decodes from the same token and position, timed for ~15 s or K steps;
     its greedy tokens are compared with the GPU's timed tokens.

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
SEED = 1234


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
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic_gate_up_q8_0.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    return {"kernel": "k_gemv_q8_0_fused1<16,3,2,true>: the gate+up launch of every layer (RMSNorm*w, SmoothQuant "
                      "and Q8_0 act-quant fused; 2 x Q8_0 8960x1536), HBM-cold", "bound": "hbm",
            "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "avg_us": round(avg_us, 3),
            "algorithmic_bytes": algo, "launches": launches, "weight_copies": copies}


def cpu_baseline(qs, hp, tensors, smooth, model, token, pos, gpu_tokens, budget_s=15.0):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    threads = min(16, os.cpu_count() or 1)
    cpu = orc.Qwen2(hp, tensors, smooth, fa_mode=0, n_threads=threads)
    for il in range(hp["n_layer"]):
        cpu.k_cache[il, :pos] = model.get_cache(il, 0, pos)
        cpu.v_cache[il, :pos] = model.get_cache(il, 1, pos)
    toks = []
    t0 = time.perf_counter()
    nxt = token
    for i in range(len(gpu_tokens)):
        nxt, _ = cpu.decode(nxt, pos + i)
        toks.append(nxt)
        if time.perf_counter() - t0 >= budget_s:
            break
    el = time.perf_counter() - t0
    agree = int(np.sum(np.asarray(toks) == np.asarray(gpu_tokens[:len(toks)])))
    first_diff = next((i for i, (a, b) in enumerate(zip(toks, gpu_tokens)) if a != b), None)
    return {"value": round(len(toks) / el, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{len(toks)} greedy decode steps of the same model from the GPU's KV cache at position {pos} "
                      f"(ggml-CPU restatement in oracle/, {orc.simd_isa()}, {threads} threads, {el:.1f} s)",
            "greedy_agreement": f"{agree}/{len(toks)}", "first_divergence": first_diff}


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


def run_7b(args, mi, qs):
    """Qwen2.5-7B-shaped W4A16 decode at a 32768-position context, bs = --batch sequences"""
    S = args.batch
    n_ctx = 32768
    warm = max(args.warmup, 1)
    hp = qs.qwen2_7b(n_ctx=n_ctx, n_seq=S)
    tensors, _ = qs.synth(hp, seed=SEED)
    model = mi.Qwen2Model(hp)
    model.load(tensors)
    weight_bytes = qs.weight_bytes(hp)
    del tensors
    n_fill = n_ctx - args.steps - warm
    model.fill_cache(n_fill, seed=SEED, scale=1.0)
    rng = np.random.default_rng(SEED + 2)
    toks = rng.integers(0, hp["n_vocab"], S).astype(np.int32)
    pos = np.full(S, n_fill, np.int32)
    wt, _ = model.decode_steps_batch(toks, pos, warm)
    toks, pos = wt[-1], pos + warm
    mi.device_sync()
    t0 = time.perf_counter()
    out, _ = model.decode_steps_batch(toks, pos, args.steps)
    mi.device_sync()
    el = time.perf_counter() - t0
    model.free()
    kv_step = qs.kv_bytes_per_position(hp) * S * (int(pos[0]) + args.steps // 2)
    step_bytes = weight_bytes + kv_step
    fa = None if args.no_roofline else measure_fa(mi, hp, S, n_ctx, rng)
    return {
        "metric": f"decode tok/s, Qwen2.5-7B-shape W4A16 bs={S} at context 32768",
        "value": round(S * args.steps / el, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": warm,
        "ms_per_step": round(el * 1e3 / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "W4A16 (int4 g32 weights x fp16 activations, fp32 accumulate), fp16 KV and head",
        "data": "synthetic (random weights of the named shape, random KV-cache contents of the named length)",
        "config": {"workload": f"Qwen2.5-7B-shaped Q4_0 W4A16 whole-model greedy decode, {S} independent sequence(s), "
                               "28 layers, hidden 3584, 28q/4kv heads x 128, FFN 18944, vocab 152064 tied fp16 head; "
                               f"KV cache of {int(pos[0])} positions per sequence, then the timed tokens",
                   "batch": S, "context": n_ctx, "bytes_per_step": step_bytes, "kv_bytes_per_step": kv_step,
                   "step_GBps": round(step_bytes * args.steps / el / 1e9, 1),
                   "kv_GBps_in_step": round(kv_step * args.steps / el / 1e9, 1),
                   "step_roofline_frac": round(step_bytes * args.steps / el / 1e9 / HBM_PEAK_GBS, 4)},
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
    ap.add_argument("--roofline-only", action="store_true",
                    help="run only the roofline leg (short program for rocprofv3 counter passes)")
    ap.add_argument("--workload", default="qwen2-1.5b-a8w8", choices=["qwen2-1.5b-a8w8", "qwen2-7b-w4a16"],
                    help="qwen2-7b-w4a16: the 7B-shaped W4A16 decode at a 32K context (see --batch)")
    ap.add_argument("--batch", type=int, default=1, help="independent sequences for qwen2-7b-w4a16 (1..8)")
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
    if args.roofline_only:
        print(json.dumps({"roofline": measure_roofline(mi, qs, hp, np.random.default_rng(SEED + 1))}))
        return
    tensors, smooth = qs.synth(hp, seed=SEED)
    model = mi.Qwen2Model(hp)
    model.load(tensors, smooth)
    rng = np.random.default_rng(SEED + 1)
    prompt = rng.integers(0, hp["n_vocab"], PREFILL)

    # context: 512 tokens, one per step (untimed), then the warm-up decode steps
    nxt = 0
    for i, t in enumerate(prompt):
        nxt = model.decode(int(t), i)
    if warm:
        wt, _ = model.decode_steps(nxt, PREFILL, warm)
        nxt = int(wt[-1])
    pos0 = PREFILL + warm
    mi.device_sync()
    t0 = time.perf_counter()
    toks, _ = model.decode_steps(nxt, pos0, args.steps)
    mi.device_sync()
    el = time.perf_counter() - t0
    tok_s = args.steps / el
    step_bytes = qs.weight_bytes(hp) + qs.kv_bytes_per_position(hp) * (pos0 + args.steps // 2)

    roof = None if args.no_roofline else measure_roofline(mi, qs, hp, rng)
    cpu = None if args.no_cpu else cpu_baseline(qs, hp, tensors, smooth, model, nxt, pos0, list(toks))
    model.free()

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
            "bytes_per_step": step_bytes,
            "step_GBps": round(step_bytes * args.steps / el / 1e9, 1),
            "step_roofline_frac": round(step_bytes * args.steps / el / 1e9 / HBM_PEAK_GBS, 4),
        },
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
