"""CPU checks of the persistent layer-stack decode's dependency-hop protocol.

tests/persist_sim.cpp runs one thread per workgroup through the walk of k_persist_q8_0
(llama-cpp-ascend310b4-addon_amd/csrc/persist.hip) with the roles, expected-arrival
counts and sync-area layout of csrc/persist_plan.h, the header the kernel and its
launcher compile.  It checks that no wait returns before every producer of its hop has
written, that the walk finishes without timeouts, that the exit leaves the sync area
clean for the next launch, and that a hop that never completes (the kernel's
debug_stall_hop) ends every workgroup through the error word and leaves the next launch
clean.  The GPU memory model (write-through stores, cache lines) is not modelled here;
the GPU tests check the results bit for bit against the per-node launches.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "llama-cpp-ascend310b4-addon_amd", "csrc")
SHAPE = (256, 1536, 12, 2, 128, 8960)  # workgroups, n_embd, heads, kv heads, head dim, n_ff


@pytest.fixture(scope="module")
def sim(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("persist_sim") / "persist_sim")
    subprocess.run(["g++", "-O1", "-std=c++17", "-pthread", "-I", CSRC, os.path.join(ROOT, "tests", "persist_sim.cpp"),
                    "-o", exe], check=True)
    return exe


def _run(exe, n_layer, splits, launches=2, spin=2_000_000, stall=-1, seed=1, shape=SHAPE):
    args = [str(v) for v in (*shape, n_layer, splits, launches, spin, stall, seed)]
    r = subprocess.run([exe, *args], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    fields = dict(kv.split("=") for kv in r.stdout.split()[1:])
    return {k: int(v) for k, v in fields.items()}


@pytest.mark.parametrize("splits", [1, 2, 7, 12, 16])
def test_walk_completes_in_order(sim, splits):
    r = _run(sim, n_layer=3, splits=splits, launches=3, seed=splits)
    assert r["violations"] == 0 and r["timeouts"] == 0 and r["err"] == 0
    assert r["residue"] == 0  # every counter back at zero for the next launch
    assert r["arrivals"] == r["expected"]  # every producer arrived exactly once per hop


def test_walk_full_depth(sim):
    r = _run(sim, n_layer=28, splits=12, launches=2, seed=5)
    assert r == {**r, "violations": 0, "timeouts": 0, "err": 0, "residue": 0}
    assert r["arrivals"] == r["expected"]


@pytest.mark.parametrize("hop", range(5))
def test_stalled_hop_ends_every_workgroup(sim, hop):
    # the first launch's waits on this hop can never complete: they give up after the
    # spin limit, every workgroup still reaches the exit (the join returns), and the
    # second launch runs clean on the same sync area
    r = _run(sim, n_layer=2, splits=12, launches=2, spin=2000, stall=hop, seed=11 + hop)
    assert r["timeouts"] >= 1
    assert r["residue"] == 0 and r["err"] == 0


def test_unfit_layouts_are_refused(sim):
    exe = sim
    # 17 splits x 2 kv heads + 128 q/k/v + 96 o tiles exceed 256 workgroups
    args = [str(v) for v in (*SHAPE, 2, 64, 1, 1000, -1, 1)]
    r = subprocess.run([exe, *args], capture_output=True, text=True, timeout=60)
    assert r.returncode == 3 and r.stdout.strip() == "unfit"
