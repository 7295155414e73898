"""The post-pass log1p for non-negative arguments (navi_amd/csrc/log1p_nonneg.h,
the same source the device compiles) against the correctly rounded log1p on
the host: within one ulp for any reciprocal within one ulp of RN(1/b), see
tests/native/log1p_check.c. Strided here to keep the CPU suite short; stride 1
(every binary32 in [0, 32]) passes with a worst error of 0.92 ulp. The GPU test
test_observe_depth_against_exact_log1p checks the device build end to end."""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).with_name("native") / "log1p_check.c"


@pytest.fixture(scope="module")
def exe(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("needs gcc")
    out = tmp_path_factory.mktemp("log1p") / "log1p_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fopenmp", "-o", str(out), str(SRC), "-lm"], check=True)
    return out


@pytest.mark.parametrize("stride,hi", [(29, "32"), (1001, "3.4e38")])
def test_log1p_within_one_ulp(exe, stride, hi):
    env = dict(os.environ, OMP_NUM_THREADS=str(min(8, os.cpu_count() or 1)))
    out = subprocess.run([str(exe), str(stride), hi], capture_output=True, text=True, timeout=300, env=env)
    assert out.returncode == 0, out.stdout + out.stderr
    assert " 0 over 1.0 ulp" in out.stdout
