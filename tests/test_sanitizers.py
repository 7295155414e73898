"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer (g++ builds of
``make -C navi_amd/csrc asan`` and ``make -C oracle asan``): the record layout, leaf
tables, cell tables, record depths and scene flags (relayout.cpp), the scene compiler
(scene_compiler.cpp) and the CPU oracle, driven by the torch-free CPU test modules,
including the malformed, cyclic, out-of-range and one-leaf DAGs of
tests/test_host_layout.py. The run must be clean; a planted overrun (a record buffer
smaller than the capacity passed for it) must be caught, so a clean run means
something.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
MODULES = ["tests/test_host_layout.py", "tests/test_relayout_leaves.py", "tests/test_compiler.py",
           "tests/test_oracle_codecs.py", "tests/test_oracle_tracer.py", "tests/test_gmdag_io.py"]


@pytest.fixture(scope="module")
def asan_env(tmp_path_factory):
    libasan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    if not libasan or not Path(libasan).exists():
        pytest.skip("gcc's libasan is not installed")
    out = tmp_path_factory.mktemp("asan")
    subprocess.run(["make", "-s", "-C", str(ROOT / "navi_amd" / "csrc"), "asan", f"ASAN_OUT={out}"], check=True)
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "asan", f"ASAN_OUT={out / 'liboracle.so'}"],
                   check=True)
    env = dict(os.environ)
    env.update(LD_PRELOAD=libasan, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               NAVI_HOST_LIB=str(out / "libnavi_host.so"), NAVI_SCENE_LIB=str(out / "libnavi_scene.so"),
               NAVI_ORACLE_LIB=str(out / "liboracle.so"), OMP_NUM_THREADS="4", PYTHONMALLOC="malloc")
    return env, out


def test_host_code_is_clean_under_asan_and_ubsan(asan_env):
    env, out = asan_env
    # the instrumented builds are the ones loaded
    probe = ("import sys; sys.path.insert(0, '.');"
             "from navi_amd import _native, scenes; import oracle;"
             "scenes._scene_lib(); oracle.lib();"
             "maps = open('/proc/self/maps').read();"
             "print(all(p in maps for p in sys.argv[1:]))")
    libs = [str(out / n) for n in ("libnavi_host.so", "libnavi_scene.so", "liboracle.so")]
    r = subprocess.run([sys.executable, "-c", probe, *libs], cwd=ROOT, env=env, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0 and r.stdout.strip() == "True", r.stdout + r.stderr[-3000:]
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", *MODULES],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    report = r.stdout[-4000:] + r.stderr[-4000:]
    assert r.returncode == 0, report
    assert "AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, report
    assert " passed" in r.stdout


def test_a_planted_overrun_is_caught(asan_env):
    """navi_relayout told that a 1-record buffer holds 4096 records writes past its end
    on a 64^3 scene: AddressSanitizer must stop it."""
    env, _ = asan_env
    code = ("import sys, ctypes; sys.path.insert(0, '.'); import numpy as np;"
            "from navi_amd import _native, scenes as S;"
            "w = np.ascontiguousarray(S.box_room(resolution=64).compile());"
            "buf = np.zeros((1, 8), np.uint32); n = ctypes.c_uint64(); root = ctypes.c_uint32();"
            "_native.lib().navi_relayout(w.ctypes.data, w.size, buf.ctypes.data, 4096,"
            " ctypes.byref(n), ctypes.byref(root), None)")
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode != 0 and "AddressSanitizer" in r.stderr, r.stderr[-3000:]
