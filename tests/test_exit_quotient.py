"""The relaid tracer's void-exit quotient (one Markstein correction of a
product with the correctly rounded reciprocal) against IEEE division, over
the divisors and quotients the tracer can meet; see
tests/native/markstein_check.c. The tracer's bit-exact GPU parity tests cover
it end to end."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).with_name("native") / "markstein_check.c"


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_markstein_quotient_matches_ieee_division(tmp_path):
    exe = tmp_path / "markstein_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(SRC), "-lm"], check=True)
    out = subprocess.run([str(exe), "64"], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert " 0 misses" in out.stdout
