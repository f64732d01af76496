"""LLDUMP1 layer dumps: index, read, write and compare.

The byte format is the layer dump of the reference's llama-eval-callback (written at
patches/ascend310b4-llama-cpp.patch:825-892; its comparison tool is
scripts/compare-layer-dumps.py, patch:2800-2890): the 8-byte magic b"LLDUMP1\\0", then
records of a little-endian u16 name length, the UTF-8 name, a little-endian u64 value
count and that many little-endian fp32 values.  A name repeats once per decode step.

Design here: `LayerDump` maps the file and indexes it in one pass (per name, the byte
offset and value count of each record); values are read as views of the mapping and
stacked per name into one [records, values] matrix, so `agreement` takes each of its
float64 sums (dot, both squared norms, squared difference) as a single reduction over
the stacked pair.  `compare` emits one row per name both dumps hold, in the order the
reference dump first wrote them (graph order: ffn_norm-N, ffn_out-N, l_out-N, ...), with
the columns of the reference's tool: layer, tensor, values, cosine, relative_l2, and for
l_out-<layer> rows cumulative_error_delta, the change of (1 - cosine) from the previous
l_out row, which shows the layer where the error grows.

Command line: python lldump.py REFERENCE CANDIDATE [--output FILE] prints the CSV.
"""

import argparse
import os
import struct

import numpy as np

MAGIC = b"LLDUMP1\0"
CSV_HEADER = "layer,tensor,values,cosine,relative_l2,cumulative_error_delta"


class DumpMismatch(ValueError):
    """The two dumps disagree on the shape of a tensor's records."""


def _layer(name):
    """trailing -<digits> of a callback name (l_out-12 -> 12), -1 when there is none"""
    head, sep, tail = name.rpartition("-")
    return int(tail) if sep and tail.isdigit() else -1


class LayerDump:
    """An LLDUMP1 file indexed by tensor name (records in file order)."""

    def __init__(self, path):
        self.path = str(path)
        size = os.path.getsize(self.path)
        self._mem = np.memmap(self.path, dtype=np.uint8, mode="r") if size else np.zeros(0, np.uint8)
        if size < len(MAGIC) or self._mem[:len(MAGIC)].tobytes() != MAGIC:
            raise ValueError(f"{self.path}: not an LLDUMP1 file")
        self.index = {}     # name -> [(value byte offset, value count), ...]
        at = len(MAGIC)
        while at < size:
            at = self._index_record(at, size)

    def _index_record(self, at, size):
        def need(n, what):
            if at + n > size:
                raise EOFError(f"{self.path}: truncated {what} at byte {at}")
        need(2, "name length")
        (name_len,) = struct.unpack_from("<H", self._mem, at)
        at += 2
        need(name_len + 8, "record header")
        name = self._mem[at:at + name_len].tobytes().decode("utf-8")
        (count,) = struct.unpack_from("<Q", self._mem, at + name_len)
        at += name_len + 8
        need(4 * count, f"values of {name}")
        self.index.setdefault(name, []).append((at, count))
        return at + 4 * count

    @property
    def names(self):
        return list(self.index)

    def records(self, name):
        """the records of one name, each a float32 array (copied out of the mapping)"""
        return [np.frombuffer(self._mem, dtype="<f4", count=n, offset=o).astype(np.float32)
                for o, n in self.index[name]]

    def matrix(self, name):
        """[records, values] float64 stack of one name's records"""
        return _stack(self.records(name), name)

    def as_dict(self):
        return {n: self.records(n) for n in self.index}


def read_dump(path):
    """-> dict name -> list of fp32 arrays (one per record, in file order)"""
    return LayerDump(path).as_dict()


def write_dump(path, records, append=False):
    """records: iterable of (name, array); values are written as little-endian fp32"""
    with open(path, "ab" if append else "wb") as f:
        if f.tell() == 0:
            f.write(MAGIC)
        for name, values in records:
            raw = name.encode("utf-8")
            v = np.ascontiguousarray(values, dtype="<f4").ravel()
            f.write(struct.pack("<H", len(raw)) + raw + struct.pack("<Q", v.size) + v.tobytes())


def _stack(recs, name="tensor"):
    sizes = {r.size for r in recs}
    if len(sizes) > 1:
        raise DumpMismatch(f"{name}: records of different lengths {sorted(sizes)}")
    return np.stack([np.asarray(r, np.float64).ravel() for r in recs]) if recs else np.zeros((0, 0))


def agreement(ref_records, cand_records, name="tensor"):
    """(values, cosine, relative L2 error) of the candidate against the reference, pooled
    over every record of one tensor name; nan where a norm is zero"""
    R, C = _stack(ref_records, name), _stack(cand_records, name)
    if R.shape != C.shape:
        raise DumpMismatch(f"{name}: reference holds {R.shape[0]} x {R.shape[1] if R.ndim > 1 else 0} values, "
                           f"candidate {C.shape[0]} x {C.shape[1] if C.ndim > 1 else 0}")
    r, c = R.ravel(), C.ravel()
    rr, cc, rc = float(r @ r), float(c @ c), float(r @ c)
    d = c - r
    dd = float(d @ d)
    cos = rc / np.sqrt(rr * cc) if rr > 0 and cc > 0 else float("nan")
    rel = np.sqrt(dd / rr) if rr > 0 else float("nan")
    return r.size, float(cos), float(rel)


def compare(reference, candidate):
    """Rows (layer, name, values, cosine, relative_l2, cumulative_error_delta or None) for
    the names both dumps hold, in the reference's first-write order.  reference and
    candidate are LayerDump objects or dicts name -> list of records."""
    ref = reference.as_dict() if isinstance(reference, LayerDump) else reference
    cand = candidate.as_dict() if isinstance(candidate, LayerDump) else candidate
    names = [n for n in ref if n in cand]
    stats = [agreement(ref[n], cand[n], n) for n in names]
    is_lout = np.array([n.startswith("l_out-") for n in names], bool)
    err = np.array([1.0 - s[1] for s in stats], np.float64)
    delta = np.full(len(names), np.nan)
    delta[is_lout] = np.diff(err[is_lout], prepend=0.0)
    return [(_layer(n), n, s[0], s[1], s[2], float(dl) if lo else None)
            for n, s, dl, lo in zip(names, stats, delta, is_lout)]


def format_rows(rows):
    out = [CSV_HEADER]
    for layer, name, count, cos, rel, delta in rows:
        tail = "" if delta is None else format(delta, ".9g")
        out.append(",".join([str(layer), name, str(count), format(cos, ".9g"), format(rel, ".9g"), tail]))
    return "\n".join(out) + "\n"


def main(argv=None):
    ap = argparse.ArgumentParser(description="Compare two LLDUMP1 layer dumps tensor by tensor.")
    ap.add_argument("reference")
    ap.add_argument("candidate")
    ap.add_argument("--output")
    a = ap.parse_args(argv)
    text = format_rows(compare(LayerDump(a.reference), LayerDump(a.candidate)))
    if a.output:
        with open(a.output, "w", encoding="utf-8") as f:
            f.write(text)
    print(text, end="")


if __name__ == "__main__":
    main()
