"""The certified first conv decides an output's bit from a per-channel
summary of the real fold (csrc/bnn_fold.c:62-77): at most two change points
along the floats of an overflow-free range (real_fold_switches in
bnns_to_c_amd/csrc/bnn_kernels.h).  tests/fold_switch_check.cpp builds that
summary for 20,000 parameter sets (random over 2^-40 .. 2^40, zero,
negative and tiny slopes, signed zeros, denormals, infinities and NaN) and
compares it with the fold itself at about 13 million probe values, the
change points and their neighbours included.  CPU only: the summary is
host code."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc (for the HIP headers) not found")
def test_fold_switches_match_the_fold(tmp_path):
    exe = tmp_path / "fsc"
    subprocess.run([HIPCC, "-O2", "-std=c++17", "-ffp-contract=off", "-I", os.path.join(ROOT, "bnns_to_c_amd", "csrc"),
                    "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "fold_switch_check.cpp"), "-o",
                    str(exe)], check=True, capture_output=True, timeout=300)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.startswith("ok "), r.stdout + r.stderr
    cases, probes = (int(v) for v in r.stdout.split()[1:3])
    assert cases == 20000 and probes > 10_000_000
