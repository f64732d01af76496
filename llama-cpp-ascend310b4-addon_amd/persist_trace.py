#!/usr/bin/env python3
"""Summarise a phase-timestamp dump of the persistent layer-stack decode.

The backend writes the dump when it is freed if GGML_MI355X_PERSIST=1 and
GGML_MI355X_PERSIST_TRACE=<file> were set when it was created: int32 n_layer, n_wg,
n_events, float64 clock ticks per microsecond, then uint64 [n_layer][n_wg][n_events]
device wall-clock stamps of the last launch (0 where a workgroup has no such event).
Events per (layer, workgroup), as k_persist_q8_0 records them:
  0 layer start, 1 q/k/v waited, 2 q/k/v done, 3 attention waited, 4 attention done,
  5 o waited, 6 o done, 7 gate/up start, 8 gate/up waited, 9 gate/up done,
  10 down start, 11 down waited, 12 down done, 13 down activation staged,
  14 o input staged, 15 gate/up input staged, 16 o records requested,
  17 o group weights, 18 o head weights, 19 attention scores formed,
  20 attention waves merged, 21 attention partials stored; in layer 0 also 22 kernel
  entry and 23 exit (after the last workgroup has reset the counters).

usage: python persist_trace.py DUMP [--layers FIRST LAST]
Prints per phase the span (first workgroup past the hop -> last one done), the median
workgroup's time, the gap from the previous phase's last producer to the first consumer
past the hop, and the per-layer period, averaged over the given layers.
"""
import argparse
import struct
import sys

import numpy as np

PHASES = [("q/k/v", 1, 2), ("attention", 3, 4), ("merge + o", 5, 6), ("gate/up", 8, 9), ("down", 11, 12)]
STAGES = [("attention: q read + first scores", 3, 19), ("attention: partials stored", 19, 21),
          ("o: merge input staged", 5, 14), ("o: dot + arrive", 14, 6), ("gate/up: input staged", 8, 15),
          ("gate/up: dots + swiglu + arrive", 15, 9), ("down: product quantized", 11, 13),
          ("down: dot + arrive", 13, 12)]


def load(path):
    raw = open(path, "rb").read()
    nl, nw, ne = struct.unpack("iii", raw[:12])
    (tpu,) = struct.unpack("d", raw[12:20])
    t = np.frombuffer(raw[20:], np.uint64).reshape(nl, nw, ne).astype(np.int64)
    first = t[0, :, [0, 22]] if ne > 22 else t[0, :, [0]]
    t0 = first[first > 0].min()  # the launch's start: the earliest entry or layer-0 stamp
    us = (t - t0) / tpu
    us[t < t0] = np.nan  # stamps left from an earlier launch (roles depend on the view length)
    us[t == 0] = np.nan
    return us


def summarise(us, first, last):
    nl = us.shape[0]
    layers = range(max(first, 1), min(last, nl - 1) + 1)
    spans = {}
    for name, a, b in PHASES:
        s = [np.nanmax(us[l, :, b]) - np.nanmin(us[l, :, a]) for l in layers]
        med = [np.nanmedian(us[l, :, b] - us[l, :, a]) for l in layers]
        spans[name] = (np.mean(s), np.mean(med))
    gaps = {}
    for i, (name, a, _) in enumerate(PHASES):
        if i == 0:
            g = [np.nanmin(us[l, :, a]) - np.nanmax(us[l - 1, :, PHASES[-1][2]]) for l in layers]
        else:
            pb = PHASES[i - 1][2]
            g = [np.nanmin(us[l, :, a]) - np.nanmax(us[l, :, pb]) for l in layers]
        gaps[name] = np.mean(g)
    period = np.mean([np.nanmin(us[l + 1, :, 0]) - np.nanmin(us[l, :, 0]) for l in layers if l + 1 < nl])
    lines = [f"{'phase':<12} {'span us':>8} {'median WG us':>13} {'gap before us':>14}"]
    for name, _, _ in PHASES:
        lines.append(f"{name:<12} {spans[name][0]:8.2f} {spans[name][1]:13.2f} {gaps[name]:14.2f}")
    lines.append(f"per-layer period {period:.2f} us over layers {layers.start}..{layers.stop - 1}")
    for name, a, b in STAGES:
        d = np.concatenate([us[l, :, b] - us[l, :, a] for l in layers])
        if np.isfinite(d).any():
            lines.append(f"{name}: median {np.nanmedian(d):.2f} us")
    return "\n".join(lines)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("dump")
    ap.add_argument("--layers", nargs=2, type=int, default=[2, 26])
    args = ap.parse_args()
    us = load(args.dump)
    print(f"{us.shape[0]} layers x {us.shape[1]} workgroups, launch span {np.nanmax(us):.1f} us")
    print(summarise(us, *args.layers))
    if us.shape[2] > 23 and np.isfinite(us[0, :, 22]).any():
        nl = us.shape[0]
        last_done = np.nanmax(us[nl - 1, :, 12])
        print(f"entry: workgroups start over {np.nanmax(us[0, :, 22]) - np.nanmin(us[0, :, 22]):.2f} us; "
              f"entry -> layer 0 start: median {np.nanmedian(us[0, :, 0] - us[0, :, 22]):.2f} us; "
              f"last layer done -> last exit: {np.nanmax(us[0, :, 23]) - last_done:.2f} us "
              f"(median workgroup exit {np.nanmedian(us[0, :, 23]) - last_done:.2f} us)")


if __name__ == "__main__":
    sys.exit(main())
