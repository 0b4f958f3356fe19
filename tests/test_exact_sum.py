"""CPU check of the exact parallel running-sum method used by the exact path
(ax-engine_amd/csrc/axs_exact_sum.h): tests/exact_sum_selftest.cpp simulates
the kernel's tiled transducer scan and compares every prefix with the
sequential f32 loop, bit for bit."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_exact_running_sum_matches_sequential_f32(tmp_path):
    exe = tmp_path / "es"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-I",
                    os.path.join(ROOT, "ax-engine_amd", "csrc"),
                    os.path.join(ROOT, "tests", "exact_sum_selftest.cpp"), "-o", str(exe)],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failures" in r.stdout
