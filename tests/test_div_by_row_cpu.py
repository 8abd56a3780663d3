"""The L2 readout's division by the row norm (nep_rms.h, div_by_row): the reciprocal, one
product and one exact FMA correction give IEEE's correctly rounded quotient bit for bit, over
the range the kernel sends through it (s and 1/s normal, v zero or |v| >= 2^-100, a zero or
normal quotient).  The check is a C program, compiled here with gcc (IEEE single division and
fmaf on the host).  The full run, `div_by_row_check 300000000 1` (2.8e8 random pairs, then
every fp32 v in [2^-100, 2) of both signs for eight divisors: 1.3e10 quotients), found no
difference either; here a sample of it keeps the CPU suite short."""
import pathlib
import shutil
import subprocess

import pytest

SRC = pathlib.Path(__file__).resolve().parent / "csrc" / "div_by_row_check.c"


def test_division_by_the_row_norm_matches_ieee_division(tmp_path):
    cc = shutil.which("gcc")
    if cc is None:
        pytest.skip("gcc not available")
    exe = tmp_path / "div_by_row_check"
    subprocess.run([cc, "-O2", "-std=c11", "-ffp-contract=off", str(SRC), "-o", str(exe), "-lm"],
                   check=True)
    run = subprocess.run([str(exe), "20000000", "61"], capture_output=True, text=True, timeout=240)
    assert run.returncode == 0, run.stdout
    assert "mismatches 0" in run.stdout
