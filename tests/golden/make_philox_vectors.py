"""Writes tests/golden/philox_torch.json: Philox4x32-10 outputs produced by
torch's own engine (ATen/core/PhiloxRNGEngine.h, compiled here with g++), used
to pin the oracle's and the kernel's Philox.

philox_engine(seed, subsequence, offset) runs counter (offset_lo, offset_hi,
subsequence_lo, subsequence_hi) with key (seed_lo, seed_hi); its first four
draws are the four output words of one Philox4x32-10 block.
Run:  python tests/golden/make_philox_vectors.py
"""
import json
import os
import subprocess
import tempfile

import numpy as np
import torch.utils.cpp_extension as ext

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = r"""
#include <ATen/core/PhiloxRNGEngine.h>
#include <cstdio>
#include <cstdint>
int main() {
  uint64_t ctr_lo, ctr_hi, key;
  while (std::scanf("%lu %lu %lu", &ctr_lo, &ctr_hi, &key) == 3) {
    at::philox_engine e(key, ctr_hi, ctr_lo);
    uint32_t a = e(), b = e(), c = e(), d = e();
    std::printf("%u %u %u %u\n", a, b, c, d);
  }
  return 0;
}
"""


def main():
    rs = np.random.default_rng(20261201)
    cases = []
    for i in range(24):
        ctr = [int(x) for x in rs.integers(0, 2**32, 4, dtype=np.uint64)]
        key = [int(x) for x in rs.integers(0, 2**32, 2, dtype=np.uint64)]
        if i == 0:
            ctr, key = [0, 0, 0, 0], [0, 0]
        cases.append({"ctr": ctr, "key": key})
    inc = ext.include_paths()
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "p.cpp")
        exe = os.path.join(d, "p")
        with open(src, "w") as f:
            f.write(SRC)
        cmd = ["g++", "-O1", "-std=c++17", src, "-o", exe] + [f"-I{p}" for p in inc]
        subprocess.run(cmd, check=True)
        lines = []
        for c in cases:
            lo = c["ctr"][0] | (c["ctr"][1] << 32)
            hi = c["ctr"][2] | (c["ctr"][3] << 32)
            k = c["key"][0] | (c["key"][1] << 32)
            lines.append(f"{lo} {hi} {k}")
        out = subprocess.run([exe], input="\n".join(lines) + "\n", capture_output=True,
                             text=True, check=True).stdout.split("\n")
    for c, line in zip(cases, out):
        c["out"] = [int(x) for x in line.split()]
    with open(os.path.join(HERE, "philox_torch.json"), "w") as f:
        json.dump({"source": "torch ATen/core/PhiloxRNGEngine.h philox_engine, 10 rounds",
                   "cases": cases}, f, indent=1)


if __name__ == "__main__":
    main()
