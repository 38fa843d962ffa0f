"""CPU check of the quantizer rounding the GPU kernels use
(mimir-model_amd/csrc/quant_rne.hpp): the same source built with g++ against
an exact integer evaluation of RoundToEven(127 x / amax), on random inputs
over the whole float range, exact ties (127 x / amax = k + 1/2) and their
neighbours."""
import os
import subprocess

from conftest import ROOT


def test_quant_rne_matches_exact_rounding(tmp_path):
    exe = tmp_path / "quant_rne_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-fno-fast-math",
                    os.path.join(ROOT, "tests", "quant_rne_check.cpp"), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe), "300000"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0" in r.stdout
