"""LLDUMP1 layer dumps: read, write and compare.

The format is the layer-dump file of the reference's llama-eval-callback
(patches/ascend310b4-llama-cpp.patch:825-892 writes it; its reader and comparison
script are patch:2800-2890, scripts/compare-layer-dumps.py): the 8-byte magic
b"LLDUMP1\\0", then records of a little-endian u16 name length, the UTF-8 name, a u64
value count and that many little-endian fp32 values.  A name may repeat (one record per
decode step); records keep their file order.

`compare` gives, per tensor name present in both dumps, the value count, the cosine and
the relative L2 error of the candidate against the reference over all of that name's
records, and for l_out-<layer> rows the growth of (1 - cosine) since the previous
l_out row: the columns of the reference's comparison
(layer,tensor,values,cosine,relative_l2,cumulative_error_delta).
"""

import math
import re
import struct

import numpy as np

MAGIC = b"LLDUMP1\0"


def write_dump(path, records, append=False):
    """records: iterable of (name, array); values are written as fp32."""
    with open(path, "ab" if append else "wb") as f:
        if f.tell() == 0:
            f.write(MAGIC)
        for name, values in records:
            raw = name.encode("utf-8")
            v = np.ascontiguousarray(values, dtype="<f4").reshape(-1)
            f.write(struct.pack("<H", len(raw)))
            f.write(raw)
            f.write(struct.pack("<Q", v.size))
            f.write(v.tobytes())


def read_dump(path):
    """-> dict name -> list of fp32 arrays (one per record, in file order)."""
    out = {}
    with open(path, "rb") as f:
        if f.read(8) != MAGIC:
            raise ValueError(f"{path}: not an LLDUMP1 file")
        while True:
            head = f.read(2)
            if not head:
                break
            if len(head) != 2:
                raise EOFError(f"{path}: truncated record header")
            (nl,) = struct.unpack("<H", head)
            name = f.read(nl)
            cnt = f.read(8)
            if len(name) != nl or len(cnt) != 8:
                raise EOFError(f"{path}: truncated record header")
            (n,) = struct.unpack("<Q", cnt)
            raw = f.read(4 * n)
            if len(raw) != 4 * n:
                raise EOFError(f"{path}: truncated values of {name.decode('utf-8', 'replace')}")
            out.setdefault(name.decode("utf-8"), []).append(np.frombuffer(raw, dtype="<f4").astype(np.float32))
    return out


def layer_of(name):
    m = re.search(r"-(\d+)$", name)
    return int(m.group(1)) if m else -1


def metric(ref, cand):
    """(values, cosine, relative L2) of cand against ref over lists of records, in float64."""
    if len(ref) != len(cand):
        raise ValueError("record count mismatch")
    dot = r2 = c2 = d2 = 0.0
    count = 0
    for a, b in zip(ref, cand):
        if a.size != b.size:
            raise ValueError("tensor size mismatch")
        a = a.astype(np.float64)
        b = b.astype(np.float64)
        dot += float(a @ b)
        r2 += float(a @ a)
        c2 += float(b @ b)
        d2 += float((b - a) @ (b - a))
        count += a.size
    cos = dot / math.sqrt(r2 * c2) if r2 and c2 else float("nan")
    rel = math.sqrt(d2 / r2) if r2 else float("nan")
    return count, cos, rel


def compare(reference, candidate):
    """Rows (layer, name, values, cosine, relative_l2, cumulative_error_delta or None) for
    the names both dumps hold, by layer then name."""
    names = sorted(set(reference) & set(candidate), key=lambda n: (layer_of(n), n))
    rows, prev = [], 0.0
    for name in names:
        count, cos, rel = metric(reference[name], candidate[name])
        delta = None
        if name.startswith("l_out-"):
            delta = (1.0 - cos) - prev
            prev = 1.0 - cos
        rows.append((layer_of(name), name, count, cos, rel, delta))
    return rows


def format_rows(rows):
    lines = ["layer,tensor,values,cosine,relative_l2,cumulative_error_delta"]
    for layer, name, count, cos, rel, delta in rows:
        lines.append(f"{layer},{name},{count},{cos:.9g},{rel:.9g}," + ("" if delta is None else f"{delta:.9g}"))
    return "\n".join(lines) + "\n"
