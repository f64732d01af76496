"""CPU checks of the persistent decode's phase-trace reader (persist_trace.py) on a
dump built field by field."""
import struct

import numpy as np

import persist_trace


def _dump(path, nl=4, nw=8, ne=24, tpu=100.0):
    t = np.zeros((nl, nw, ne), np.uint64)
    base = 1_000_000
    for l in range(nl):
        t0 = base + l * 3000  # 30 us per layer at 100 ticks/us
        t[l, :, 0] = t0
        # every workgroup: q/k/v waited at +100 ticks, done at +300 (a span of 2 us,
        # workgroup 7 done 1 us later); the other phases 400 ticks apart
        for w in range(nw):
            t[l, w, 1] = t0 + 100
            t[l, w, 2] = t0 + 300 + (100 if w == 7 else 0)
            for k, (a, b) in enumerate(((3, 4), (5, 6), (8, 9), (11, 12))):
                t[l, w, a] = t0 + 500 + 500 * k
                t[l, w, b] = t0 + 800 + 500 * k
    t[0, 3, 5] = base - 10  # a stamp from an earlier launch: ignored
    with open(path, "wb") as f:
        f.write(struct.pack("iii", nl, nw, ne))
        f.write(struct.pack("d", tpu))
        f.write(t.tobytes())


def test_reader_spans_gaps_and_period(tmp_path):
    p = tmp_path / "trace.bin"
    _dump(p)
    us = persist_trace.load(str(p))
    assert us.shape == (4, 8, 24)
    assert np.isnan(us[0, 3, 5]) and np.isnan(us[0, 0, 20])
    out = persist_trace.summarise(us, 1, 2)
    rows = {line.split()[0]: line.split() for line in out.splitlines()[1:6]}
    assert float(rows["q/k/v"][1]) == 3.0      # waited +1 us .. last done +4 us
    assert float(rows["q/k/v"][2]) == 2.0      # median workgroup
    assert float(rows["attention"][3]) == 1.0  # q/k/v's last done +4 us -> attention +5 us
    assert float(rows["q/k/v"][3]) == 8.0      # the previous layer's down ends 7 us before this layer starts
    assert "per-layer period 30.00 us" in out
