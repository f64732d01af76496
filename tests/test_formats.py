"""On-disk formats around the decode path, on the CPU: LLDUMP1 layer dumps and the
SmoothQuant scale file (host parsing only; no device)."""
import math
import struct

import numpy as np
import pytest

import lldump


def _by_hand(records):
    """The LLDUMP1 bytes built field by field with struct, independent of write_dump."""
    b = b"LLDUMP1\x00"
    for name, v in records:
        raw = name.encode()
        v = np.asarray(v, "<f4")
        b += struct.pack("<H", len(raw)) + raw + struct.pack("<Q", v.size) + v.tobytes()
    return b


def test_lldump_bytes_and_round_trip(tmp_path):
    recs = [("l_out-0", np.arange(5, dtype=np.float32)), ("l_out-1", np.array([-1.5, 2.25], np.float32)),
            ("l_out-0", np.full(5, 3.0, np.float32))]
    p = tmp_path / "a.bin"
    lldump.write_dump(p, recs[:2])
    lldump.write_dump(p, recs[2:], append=True)
    assert p.read_bytes() == _by_hand(recs)
    d = lldump.read_dump(p)
    assert list(d) == ["l_out-0", "l_out-1"]
    assert [r.tolist() for r in d["l_out-0"]] == [list(range(5)), [3.0] * 5]
    assert d["l_out-1"][0].tolist() == [-1.5, 2.25]


def test_lldump_rejects_bad_files(tmp_path):
    p = tmp_path / "bad.bin"
    p.write_bytes(b"LLDUMP2\x00")
    with pytest.raises(ValueError):
        lldump.read_dump(p)
    whole = _by_hand([("ffn_out-3", np.ones(4, np.float32))])
    for cut in (9, 12, len(whole) - 1):   # inside the name length, the name, the values
        p.write_bytes(whole[:cut])
        with pytest.raises(EOFError):
            lldump.read_dump(p)


def test_lldump_metric_closed_forms():
    rng = np.random.default_rng(0)
    a = rng.standard_normal(64).astype(np.float32)
    o = rng.standard_normal(64).astype(np.float32)
    o -= (o @ a) / (a @ a) * a                       # orthogonal to a
    o *= np.linalg.norm(a) / np.linalg.norm(o)      # same length
    assert lldump.agreement([a], [a])[1:] == (pytest.approx(1.0), 0.0)
    _, c, r = lldump.agreement([a], [-a])
    assert c == pytest.approx(-1.0) and r == pytest.approx(2.0)
    _, c, r = lldump.agreement([a], [2 * a])
    assert c == pytest.approx(1.0) and r == pytest.approx(1.0)
    _, c, r = lldump.agreement([a], [o])
    assert abs(c) < 1e-6 and r == pytest.approx(math.sqrt(2.0), rel=1e-6)
    # two records pool their sums: the same as one record of both
    n, c, r = lldump.agreement([a, 2 * a], [o, 2 * a])
    n1, c1, r1 = lldump.agreement([np.concatenate([a, 2 * a])], [np.concatenate([o, 2 * a])])
    assert (n, c, r) == (n1, pytest.approx(c1), pytest.approx(r1))
    # a zero reference has no direction: nan, not a division error
    assert all(math.isnan(v) for v in lldump.agreement([np.zeros(4)], [np.ones(4)])[1:])
    with pytest.raises(lldump.DumpMismatch):
        lldump.agreement([a], [a[:3]])
    with pytest.raises(lldump.DumpMismatch):
        lldump.agreement([a, a], [a])


def test_lldump_compare_rows_and_error_growth(tmp_path):
    a = np.array([1.0, 0.0], np.float32)
    b = np.array([1.0, 1.0], np.float32) / np.sqrt(np.float32(2))   # 45 degrees from a
    # the reference's write order is graph order; "only_ref" has no candidate and no row
    ref = [("ffn_out-0", a), ("l_out-0", a), ("ffn_out-1", a), ("l_out-1", a), ("only_ref", a), ("l_out-10", a)]
    cand = [("l_out-10", -a), ("l_out-1", b), ("ffn_out-1", b), ("l_out-0", a), ("ffn_out-0", a)]
    pr, pc = tmp_path / "ref.bin", tmp_path / "cand.bin"
    lldump.write_dump(pr, ref)
    lldump.write_dump(pc, cand)
    rows = lldump.compare(lldump.LayerDump(pr), lldump.LayerDump(pc))
    assert [r[1] for r in rows] == ["ffn_out-0", "l_out-0", "ffn_out-1", "l_out-1", "l_out-10"]
    assert [r[0] for r in rows] == [0, 0, 1, 1, 10]
    e1 = 1.0 - math.sqrt(0.5)
    # (1 - cosine) of the l_out rows is 0, e1, 2: its growth row to row is 0, e1, 2 - e1
    assert rows[0][5] is None and rows[2][5] is None
    assert rows[1][5] == pytest.approx(0.0) and rows[3][5] == pytest.approx(e1) and rows[4][5] == pytest.approx(2 - e1)
    text = lldump.format_rows(rows)
    assert text.splitlines()[0] == "layer,tensor,values,cosine,relative_l2,cumulative_error_delta"
    assert text.splitlines()[3].startswith("1,ffn_out-1,2,") and text.splitlines()[3].endswith(",")
    assert text.splitlines()[5].startswith("10,l_out-10,2,-1,2,")
    # the command line prints the same CSV
    out = tmp_path / "cmp.csv"
    lldump.main([str(pr), str(pc), "--output", str(out)])
    assert out.read_text() == text


def test_lldump_header_only_and_layer_names(tmp_path):
    p = tmp_path / "empty.bin"
    lldump.write_dump(p, [])
    assert lldump.LayerDump(p).names == [] and lldump.read_dump(p) == {}
    assert [lldump._layer(n) for n in ("l_out-12", "result_norm", "attn-x", "ffn_out-0")] == [12, -1, -1, 0]


def test_smooth_scale_file_parser(tmp_path):
    """The library's own parser on files written the way the scale tool writes them
    (numpy '<f4' tofile of a [layers, hidden] array)."""
    import ggml_mi355x as mi
    rng = np.random.default_rng(3)
    s = np.clip(rng.lognormal(0.0, 1.0, (3, 40)), 1e-3, 1e3).astype("<f4")
    p = tmp_path / "sq-scales-a05.bin"
    s.tofile(p)
    got = mi.read_smooth_scales(p, 3, 40)
    assert got.tobytes() == s.tobytes()
    with pytest.raises(mi.MiError, match="holds 480 bytes, expected 492"):
        mi.read_smooth_scales(p, 3, 41)
    bad = s.copy()
    bad[2, 7] = np.nan
    bad.tofile(p)
    with pytest.raises(mi.MiError, match="layer 2, channel 7"):
        mi.read_smooth_scales(p, 3, 40)
    bad[2, 7] = 0.0
    bad.tofile(p)
    with pytest.raises(mi.MiError, match="not a positive"):
        mi.read_smooth_scales(p, 3, 40)
    with pytest.raises(mi.MiError, match="cannot open"):
        mi.read_smooth_scales(tmp_path / "missing.bin", 3, 40)
