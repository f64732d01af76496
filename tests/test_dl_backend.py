"""The dynamically loadable backend (libggml-mi355x.so, built with GGML_BACKEND_DL) as
ggml's backend loader uses it: dlopen'ed into a process whose libggml-base is already
loaded, with ggml_backend_init / ggml_backend_score resolved by name.  On the CPU: no
device is needed to load it, register it and check its ids against the base library."""
import json
import os
import subprocess
import sys
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "llama-cpp-ascend310b4-addon_amd")
DL = os.path.join(PKG, "libggml-mi355x.so")
BASE = os.path.join(PKG, "libggml-base.so")

LOADER = textwrap.dedent("""
    import ctypes, json, os, sys
    pre, base, dl = sys.argv[1], sys.argv[2], sys.argv[3]
    if pre:
        ctypes.CDLL(pre, mode=os.RTLD_NOW | os.RTLD_GLOBAL)
    ctypes.CDLL(base, mode=os.RTLD_NOW | os.RTLD_GLOBAL)        # the host's libggml-base
    lib = ctypes.CDLL(dl, mode=os.RTLD_NOW | os.RTLD_LOCAL)      # what ggml_backend_load does
    lib.ggml_backend_init.restype = ctypes.c_void_p
    lib.ggml_backend_score.restype = ctypes.c_int
    lib.ggml_backend_mi355x_abi_check.restype = ctypes.c_int
    lib.ggml_backend_mi355x_abi_check.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
    msg = ctypes.create_string_buffer(256)
    ok = lib.ggml_backend_mi355x_abi_check(msg, 256)
    reg = lib.ggml_backend_init()
    out = {"abi_ok": ok, "msg": msg.value.decode(), "reg": bool(reg),
           "api_version": ctypes.c_int.from_address(reg).value if reg else None,
           "score": lib.ggml_backend_score()}
    print(json.dumps(out))
""")


def _load(pre=""):
    r = subprocess.run([sys.executable, "-c", LOADER, pre, BASE, DL], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout.strip().splitlines()[-1]), r.stderr


@pytest.fixture(scope="module")
def built():
    for p in (DL, BASE):
        if not os.path.exists(p):
            pytest.fail(f"{p} is not built (run __graft_entry__.build())")


def test_dl_backend_registers_over_libggml_base(built):
    out, _ = _load()
    assert out["abi_ok"] == 1, out["msg"]
    assert out["reg"] and out["api_version"] == 2     # GGML_BACKEND_API_VERSION of ggml-backend-impl.h
    assert out["score"] in (0, 100)                  # 0 without a gfx950 device


def test_dl_backend_carries_no_ggml_core(built):
    """Its ggml_* symbols come from the host: it exports only its own entry points, and
    what it imports is ggml-base API."""
    nm = lambda *a: subprocess.run(["nm", "-D", *a, DL], capture_output=True, text=True, check=True).stdout
    defined = {ln.split()[-1] for ln in nm("--defined-only").splitlines() if " T " in ln}
    ggml_defined = {s for s in defined if s.startswith("ggml_")}
    own = {"ggml_backend_init", "ggml_backend_score", "ggml_backend_is_mi355x"}
    assert ggml_defined - own == {s for s in ggml_defined if s.startswith("ggml_backend_mi355x_")}
    assert own <= ggml_defined
    undefined = {ln.split()[-1] for ln in nm("--undefined-only").splitlines()}
    imported = {s for s in undefined if s.startswith("ggml_")}
    base_defined = {ln.split()[-1] for ln in subprocess.run(["nm", "-D", "--defined-only", BASE], capture_output=True,
                                                             text=True, check=True).stdout.splitlines()}
    assert imported and imported <= base_defined, imported - base_defined


def test_dl_backend_refuses_a_ggml_with_other_op_ids(built, tmp_path):
    """A libggml-base from another ggml revision numbers its ops differently: stand one in
    whose op table names every id "DIV"; registration must refuse rather than run DIV
    nodes as some other op."""
    src = tmp_path / "other_ids.c"
    src.write_text('const char *ggml_op_name(int op) { (void)op; return "DIV"; }\n')
    so = tmp_path / "libother_ids.so"
    subprocess.run(["gcc", "-shared", "-fPIC", "-o", str(so), str(src)], check=True)
    out, err = _load(str(so))
    assert out["abi_ok"] == 0 and "DIV in the loaded ggml, NONE in this backend's build" in out["msg"]
    assert not out["reg"] and out["score"] == 0
    assert "not registering" in err
