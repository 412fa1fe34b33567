"""The fp32 top-p kernel sums DETEXP_FIX weights in an fp64 form (the
contract's fp32 steps to p and n, then rint(p * 2^(n + 40)) in fp64, the
argument clamped at -30.5).  Pinned here against the oracle's integer form
on a strided sweep of every fp32 d in [-31, 0] plus dense windows around the
cutoff; the full sweep (stride 1, about a minute) found no mismatch either."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_detexp_f64_form_matches_the_oracle(tmp_path):
    exe = tmp_path / "detexp_f64_form"
    subprocess.run(["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-fno-fast-math",
                    "-o", str(exe), os.path.join(HERE, "detexp", "detexp_f64_form.c"),
                    os.path.join(ROOT, "oracle", "tokpath_oracle.c"), "-lm"],
                   check=True)
    out = subprocess.run([str(exe), "509"], capture_output=True, text=True, timeout=300)
    print(out.stdout)
    assert out.returncode == 0, out.stdout
    assert " 0 mismatches" in out.stdout
