"""CPU check of the device's f32 exp (ax-engine_amd/csrc/axs_expf.h).

The reference's probabilities are f32::exp, i.e. the host libm's expf
(crates/ax-engine-mlx/src/sampling.rs:248-251,274-277).  The device restates
that function; tests/expf_libm_selftest.cpp compares the restatement with the
host expf over all 2^32 f32 inputs (bit for bit) and checks monotonicity on
x <= 0.  A one-bit slip in the table, a coefficient or the reduction shows up
as mismatches.
"""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_expf_restatement_equals_host_expf_everywhere(tmp_path):
    exe = tmp_path / "expf_selftest"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-pthread", "-I",
                    os.path.join(ROOT, "ax-engine_amd", "csrc"),
                    os.path.join(ROOT, "tests", "expf_libm_selftest.cpp"), "-o", str(exe), "-lm"],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 mismatches, 0 inversions" in r.stdout
