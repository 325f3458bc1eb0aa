"""The C-ABI library on the CPU: it loads, exports every entry point the
headers declare, fails cleanly without a GPU, honours the fault-injection
switch, and its host utilities agree with the oracle."""
import ctypes as C
import os
import pathlib
import re
import subprocess
import sys

import numpy as np
import pytest

import oracle
from ltx_amd import conditioning, synth
from ltx_amd import runtime as rt

ROOT = pathlib.Path(__file__).resolve().parent.parent


def declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(ltx_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    L = rt.lib()
    names = declared_symbols()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def _gpu_present():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.mark.skipif(_gpu_present(), reason="checks the no-GPU error path")
def test_init_without_gpu_fails_cleanly():
    L = rt.lib()
    h = C.c_void_p()
    assert L.ltx_init(0, C.byref(h)) == 0 and not h.value
    assert "hipGetDeviceCount" in L.ltx_last_error(None).decode()


def test_fault_injection_switch():
    """LTX_FAIL_AFTER=1 makes the first checked HIP call fail with a tagged error."""
    code = ("import sys; sys.path.insert(0, %r)\n"
            "import ctypes as C\n"
            "from ltx_amd import runtime as rt\n"
            "h = C.c_void_p(); L = rt.lib()\n"
            "assert L.ltx_init(0, C.byref(h)) == 0\n"
            "print(L.ltx_last_error(None).decode())\n") % str(ROOT / "ltx-zml_amd")
    env = dict(os.environ, LTX_FAIL_AFTER="1")
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert "[LTX_FAIL_AFTER]" in out.stdout or "hipGetDeviceCount" in out.stdout


def test_rope_tables_library_equals_oracle():
    grid = synth.latent_grid(3, 4, 8)
    c_or, s_or = oracle.rope_tables(grid)
    c, s = rt.rope_tables(grid, graph_layout=False)
    assert np.array_equal(c.view(np.uint32), c_or.view(np.uint32))
    assert np.array_equal(s.view(np.uint32), s_or.view(np.uint32))
    cg, sg = rt.rope_tables(grid, graph_layout=True)
    assert np.array_equal(cg, c.transpose(1, 0, 2)) and np.array_equal(sg, s.transpose(1, 0, 2))


def test_null_arguments_are_rejected():
    L = rt.lib()
    assert L.ltx_block_forward(None, None, None, None, 0, None, None, 0, None, None, None, 0, None, 0, None) == 0
    assert L.ltx_rope_tables(None, 0, None, None, 0) == 0


def test_sinusoid_known_answers():
    e = conditioning.sinusoid(np.array([0.0, 0.5], np.float32))
    assert e.shape == (2, 256)
    assert (e[0, :128] == 1.0).all() and (e[0, 128:] == 0.0).all()  # cos half first
    # slot 0 frequency is 1: cos(1000 * 0.5)
    assert np.isclose(e[1, 0], np.cos(np.float32(500.0)), atol=1e-6)


def test_synthetic_inputs_are_deterministic():
    a = synth.make_inputs(64, 16)
    b = synth.make_inputs(64, 16)
    for k in a:
        assert np.array_equal(a[k], b[k])
    assert a["tstab"].shape == (3, 9, 4096) and a["tidx"].max() == 2
    g = synth.latent_grid(14, 32, 64)
    assert g.shape == (3, 28672, 2) and g[0].max() == 13 and g[1].max() == 31 * 32 and g[2].max() == 63 * 32
