"""The GEMV RMSNorm prologue divides by reciprocal plus one Newton step
(csrc/k_gemv.hip, quotient()).  This compiles a host restatement of that
formula and compares it with IEEE division rounded to fp16/bf16 over every
numerator and a stride of divisors (CHOMIK_QUOTIENT_STRIDE=1 for all of them:
a few minutes)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_quotient_matches_ieee_division(tmp_path):
    exe = tmp_path / "quotient_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-frounding-math", "-o", str(exe),
                    os.path.join(HERE, "native", "quotient_check.c"), "-lm"], check=True)
    stride = os.environ.get("CHOMIK_QUOTIENT_STRIDE", "61")
    run = subprocess.run([str(exe), stride], capture_output=True, text=True, timeout=600)
    print(run.stdout)
    assert run.returncode == 0, run.stdout
    assert "fp16 cases" in run.stdout and "bf16 cases" in run.stdout
    # without the correction step the same comparison must find mismatches
    planted = subprocess.run([str(exe), stride, "plain"], capture_output=True, text=True, timeout=600)
    assert planted.returncode == 1, planted.stdout
    counts = [int(line.split()[-1]) for line in planted.stdout.splitlines() if "mismatches" in line]
    assert len(counts) == 2 and all(c > 0 for c in counts), planted.stdout
