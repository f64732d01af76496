#!/usr/bin/env python3
"""Decode throughput on one MI355X for the Qwen2.5-1.5B-shaped A8W8 model, bs=1.

Prints ONE JSON line (driver contract).  Phases:
  1. decode: W untimed + K timed token steps, each step replayed as one HIP graph;
     tokens/s = K / elapsed (inputs resident in HBM).
  2. roofline: the dominant kernel (Q8_0 GEMV, 8960 x 1536, ggml Q8_0 weights) timed
     live with HIP events over back-to-back launches that rotate through enough weight
     copies (> 2x the 256 MB MALL) to be HBM-cold; achieved = algorithmic bytes / avg.
  3. cpu_baseline (rank 0, N=1): the CPU restatement of ggml-CPU (oracle/) on a bounded
     sample of the same token step, multithreaded, scaled to tokens/s.

Synthetic data: random weights of the Qwen2.5-1.5B shape (28 layers, hidden 1536,
12 q / 2 kv heads of dim 128, FFN 8960, vocab 151936, fp16 tied head), SmoothQuant
factors uniform in [0.5, 2], KV context 512 + generated tokens.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "llama-cpp-ascend310b4-addon_amd"))

import ggml_mi355x as mi  # noqa: E402

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20

# Qwen2.5-1.5B shape
N_LAYER, N_EMBD, N_HEAD, N_HEAD_KV, HEAD_DIM, N_FF, N_VOCAB = 28, 1536, 12, 2, 128, 8960, 151936
PREFILL = 512


def f16_bits(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def q8_0_weights(rng, n, k):
    nb = k // 32
    blk = np.empty((n, nb, 34), dtype=np.uint8)
    blk[:, :, 2:] = rng.integers(-127, 128, size=(n, nb, 32), dtype=np.int8).view(np.uint8)
    d = f16_bits(np.abs(rng.standard_normal((n, nb), dtype=np.float32)) * np.float32(0.02 / 127.0))
    blk[:, :, 0:2] = d.view(np.uint8).reshape(n, nb, 2)
    return blk.reshape(n, nb * 34)


class HotPathModel:
    """Device-resident weights of the decode hot path and one token step as launches."""

    PROJ = (("q", N_EMBD, N_EMBD), ("k", N_HEAD_KV * HEAD_DIM, N_EMBD), ("v", N_HEAD_KV * HEAD_DIM, N_EMBD),
            ("o", N_EMBD, N_EMBD), ("gate", N_FF, N_EMBD), ("up", N_FF, N_EMBD), ("down", N_EMBD, N_FF))

    def __init__(self, rng, n_ctx, keep_host=False):
        self.n_ctx = n_ctx
        self.host = {} if keep_host else None
        self.layers = []
        self.weight_bytes = 0
        for il in range(N_LAYER):
            lw = {}
            for name, n, k in self.PROJ:
                blocks = q8_0_weights(rng, n, k)
                src = mi.to_device(blocks)
                dst = mi.DeviceBuffer(mi.q8_0_packed_size(n, k))
                mi.prepack_q8_0(src.ptr, dst.ptr, n, k)
                mi.device_sync()
                src.free()
                inv_s = (1.0 / rng.uniform(0.5, 2.0, k)).astype(np.float32)
                lw[name] = (dst, mi.to_device(inv_s), n, k)
                self.weight_bytes += blocks.nbytes
                if keep_host:
                    self.host[(il, name)] = (blocks, inv_s)
            kc = f16_bits(rng.standard_normal((n_ctx, N_HEAD_KV, HEAD_DIM), dtype=np.float32))
            vc = f16_bits(rng.standard_normal((n_ctx, N_HEAD_KV, HEAD_DIM), dtype=np.float32))
            lw["kc"], lw["vc"] = mi.to_device(kc), mi.to_device(vc)
            if keep_host:
                self.host[(il, "kv")] = (kc, vc)
            self.layers.append(lw)
        head = f16_bits(rng.standard_normal((N_VOCAB, N_EMBD), dtype=np.float32) * np.float32(0.02))
        self.head = mi.to_device(head)
        self.weight_bytes += head.nbytes
        if keep_host:
            self.host["head"] = head
        x = rng.standard_normal(N_EMBD).astype(np.float32)
        if keep_host:
            self.host["x"] = x
        self.x = mi.to_device(x)
        self.xq = mi.DeviceBuffer(mi.xq_size(1, N_FF))
        self.q = mi.DeviceBuffer(N_EMBD * 4)
        self.kv = mi.DeviceBuffer(N_HEAD_KV * HEAD_DIM * 4)
        self.att = mi.DeviceBuffer(N_EMBD * 4)
        self.ff = mi.DeviceBuffer(N_FF * 4)
        self.ff2 = mi.DeviceBuffer(N_FF * 4)
        self.logits = mi.DeviceBuffer(N_VOCAB * 4)
        self.kv_len = mi.to_device(np.array([n_ctx], np.int32))
        self.ws_bytes = mi.fa_decode_workspace_size(n_ctx, N_HEAD, N_HEAD_KV, HEAD_DIM)
        self.ws = mi.DeviceBuffer(self.ws_bytes).zero()
        mi.device_sync()

    def step(self, st):
        """One token: per layer q/k/v, attention, o, gate/up, down; then the tied fp16 head."""
        R = mi.Q8_ROUND_X86
        nb1 = N_HEAD_KV * HEAD_DIM * 2
        for lw in self.layers:
            for name, out in (("q", self.q), ("k", self.kv), ("v", self.kv)):
                w, inv, n, k = lw[name]
                mi.mul_mat_q8_0_f32(w.ptr, self.x.ptr, inv.ptr, out.ptr, n, k, 1, R, stream=st.ptr)
            mi.fa_decode(self.q.ptr, lw["kc"].ptr, lw["vc"].ptr, None, self.kv_len.ptr, self.n_ctx, N_HEAD,
                         N_HEAD_KV, HEAD_DIM, nb1, HEAD_DIM * 2, nb1, HEAD_DIM * 2, 1.0 / np.sqrt(HEAD_DIM),
                         self.att.ptr, self.ws.ptr, self.ws_bytes, stream=st.ptr)
            w, inv, n, k = lw["o"]
            mi.mul_mat_q8_0_f32(w.ptr, self.att.ptr, inv.ptr, self.q.ptr, n, k, 1, R, stream=st.ptr)
            for name, out in (("gate", self.ff), ("up", self.ff2)):
                w, inv, n, k = lw[name]
                mi.mul_mat_q8_0_f32(w.ptr, self.x.ptr, inv.ptr, out.ptr, n, k, 1, R, stream=st.ptr)
            w, inv, n, k = lw["down"]
            mi.act_quant_q8_0(self.ff.ptr, inv.ptr, 1, k, self.xq.ptr, R, stream=st.ptr)
            mi.gemv_q8_0(w.ptr, self.xq.ptr, self.q.ptr, n, k, 1, stream=st.ptr)
        mi.gemv_f16(self.head.ptr, N_EMBD, self.x.ptr, self.logits.ptr, N_VOCAB, N_EMBD, 1, stream=st.ptr)


def kv_bytes(n_ctx):
    return N_LAYER * 2 * n_ctx * N_HEAD_KV * HEAD_DIM * 2


def measure_roofline(rng, st):
    """Q8_0 GEMV 8960 x 1536 (the FFN gate/up shape), HBM-cold, live event timing."""
    n, k = N_FF, N_EMBD
    blocks = q8_0_weights(rng, n, k)
    src = mi.to_device(blocks)
    psz = mi.q8_0_packed_size(n, k)
    copies = int(np.ceil(2 * MALL_BYTES / psz)) + 1
    bufs = []
    for _ in range(copies):
        b = mi.DeviceBuffer(psz)
        mi.prepack_q8_0(src.ptr, b.ptr, n, k, stream=st.ptr)
        bufs.append(b)
    x = mi.to_device(rng.standard_normal(k).astype(np.float32))
    y = mi.DeviceBuffer(n * 4)
    plug_a, plug_b = mi.DeviceBuffer(2 << 30), mi.DeviceBuffer(2 << 30)
    st.sync()
    algo = n * (k // 32) * 34 + k * 4 + n * 4
    launches = copies * 8
    e0, e1 = mi.Event(), mi.Event()
    samples = []
    for rep in range(3):
        # a 2 GiB device copy first: the queue fills while it runs, so the timed
        # launches execute back to back whatever the host-side launch rate
        for _ in range(2):
            mi._call("mi_memcpy_d2d", mi._P(plug_b.ptr), mi._P(plug_a.ptr), 2 << 30, mi._P(st.ptr))
        e0.record(st.ptr)
        for i in range(launches):
            mi.mul_mat_q8_0_f32(bufs[i % copies].ptr, x.ptr, None, y.ptr, n, k, 1, mi.Q8_ROUND_X86, stream=st.ptr)
        e1.record(st.ptr)
        samples.append(e0.elapsed_ms(e1) * 1e3 / launches)
    avg_us = float(np.median(samples))
    for b in bufs + [src, plug_a, plug_b]:
        b.free()
    achieved = algo / avg_us / 1e3
    return {"kernel": "k_gemv_q8_0_fused1 (A8W8 Q8_0 GEMV, N=8960, K=1536, HBM-cold)", "bound": "hbm",
            "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "avg_us": round(avg_us, 3),
            "algorithmic_bytes": algo, "launches": launches, "weight_copies": copies}


def cpu_baseline(model, budget_s=12.0):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    threads = min(16, os.cpu_count() or 1)
    x = model.host["x"]
    t0 = time.perf_counter()
    tokens = 0
    while True:
        for il in range(N_LAYER):
            for name, n, k in HotPathModel.PROJ:
                blocks, inv = model.host[(il, name)]
                orc.mul_mat_q8_0_mt(blocks, x if k == N_EMBD else np.resize(x, k), n, k, inv_s=inv, n_threads=threads)
            kc, vc = model.host[(il, "kv")]
            orc.flash_attn_ext_1tok(np.resize(x, (N_HEAD, HEAD_DIM)).astype(np.float32), kc, vc, N_HEAD_KV,
                                    1.0 / np.sqrt(HEAD_DIM), n_threads=threads)
        orc.mul_mat_f16_mt(model.host["head"], x, N_VOCAB, N_EMBD, n_threads=threads)
        tokens += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return {"value": round(tokens / el, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{tokens} token steps of the same hot path (196 Q8_0 GEMVs + 28 attention + fp16 head) "
                      f"on the ggml-CPU restatement in oracle/, {orc.simd_isa()}, {el:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of replaying HIP graphs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); multi-GPU sharding is "
              "described in DESIGN.md and not implemented", file=sys.stderr)
        sys.exit(2)
    if mi.device_count() < 1:
        print("bench.py: no HIP device: " + mi.last_error(), file=sys.stderr)
        sys.exit(1)

    rng = np.random.default_rng(1234)
    n_ctx = PREFILL + args.warmup + args.steps
    want_cpu = not args.no_cpu
    model = HotPathModel(rng, n_ctx, keep_host=want_cpu)
    st = mi.Stream()

    graph = None
    if not args.no_graph:
        graph = mi.Graph(st)
        with graph:
            model.step(st)
    run = graph.launch if graph else (lambda: model.step(st))
    for _ in range(args.warmup):
        run()
    st.sync()
    e0, e1 = mi.Event(), mi.Event()
    mi.device_sync()
    e0.record(st.ptr)
    for _ in range(args.steps):
        run()
    e1.record(st.ptr)
    ms = e0.elapsed_ms(e1)
    mi.device_sync()
    tok_s = args.steps / (ms / 1e3)
    step_bytes = model.weight_bytes + kv_bytes(n_ctx)

    roof = measure_roofline(rng, st)
    cpu = cpu_baseline(model) if want_cpu else None

    out = {
        "metric": "decode tok/s, Qwen2.5-1.5B-shape bs=1; GEMV HBM GB/s as % of peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 (A8W8 Q8_0 dots, int32 accumulate) / fp16 KV and head, fp32 accumulation",
        "data": "synthetic (random weights of the named shape)",
        "config": {
            "workload": "Qwen2.5-1.5B-shaped A8W8 decode hot path, bs=1: per token 28 x (q,k,v,o,gate,up,down "
                        "Q8_0 GEMVs + GQA flash-decoding over the KV cache) + tied fp16 head 151936x1536; "
                        "glue ops (RMSNorm, RoPE, SwiGLU, residual, argmax) not yet in the step",
            "n_ctx": n_ctx, "graph": graph is not None,
            "bytes_per_step": step_bytes,
            "step_GBps": round(step_bytes / (ms / args.steps) / 1e6, 1),
        },
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
