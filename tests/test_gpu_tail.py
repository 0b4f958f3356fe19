"""GPU parity for rows whose probability mass lies mostly below 2^-14 of the
maximum's, against the CPU oracle, through the C ABI.

On the exact path the keys with p < 2^-14 are summed per p bucket while the
running sum stays in one binade; a bucket that the sum leaves its binade in,
a bucket that holds its own top value (a p whose 14 low bits are zero), and
a bucket that a nucleus cut, top-k edge or draw falls inside are sorted and
summed element by element.  These rows put all of that in the tail:
  * a bulk of ~150k logits 10.5..16.5 below the maximum, so the running sum
    crosses 2 or 4 inside the tail;
  * copies of logits whose libm expf is a bucket's top value;
  * top-p 0.5..0.99, top-k edges inside the tail, min-p with top-p, and
    uniforms near 1, so the cut and the draw land in tail buckets.
Run with kept lists (the tail is then ordered in full for them) and without
(only the buckets the decisions read are ordered), in both launch shapes
(listed rows and the exact path in place).  Same bar as the other parity
tests: ids equal on every row, kept lists exact, logprobs within 1e-5.
"""
import ctypes
import ctypes.util

import numpy as np
import pytest

from ax_sampler.synth import DTYPE_F32, Workload, _params

from gpu_common import compare, log, run_gpu, run_oracle

pytestmark = pytest.mark.gpu

V = 151936


def _libm_expf():
    lib = ctypes.CDLL(ctypes.util.find_library("m"))
    f = lib.expf
    f.restype = ctypes.c_float
    f.argtypes = [ctypes.c_float]
    return f


def _top_valued(count: int, start: float = -10.75):
    """f32 x below `start` whose host expf has a bit pattern with its 14 low
    bits zero: the top value of a tail bucket when the row maximum is 0 and
    T = 1 (the oracle and the device both use that expf)."""
    expf = _libm_expf()
    b = int(np.array([start], np.float32).view(np.uint32)[0])
    out = []
    while len(out) < count:
        b += 1  # negative floats: one step further from zero
        x = np.array([b], np.uint32).view(np.float32)[0]
        pb = int(np.array([expf(float(x))], np.float32).view(np.uint32)[0])
        if pb & 0x3FFF == 0:
            out.append(x)
    return np.array(out, np.float32)


@pytest.fixture(scope="module")
def tail_workload():
    B = 96
    rng = np.random.default_rng(2024)
    tops = _top_valued(12)
    x = np.empty((B, V), np.float32)
    p = _params(B, temperature=1.0, seed=0, step=5)
    laws = [
        dict(top_p=0.9), dict(top_p=0.5), dict(top_p=0.99), dict(top_p=0.97, top_k=60000),
        dict(top_k=90000), dict(top_p=0.95, min_p=2.0 ** -19, has_min_p=1), dict(top_p=0.0), dict(top_k=3),
    ]
    for r in range(B):
        shift = np.float32(rng.uniform(-1.0, 1.5))
        x[r] = rng.uniform(-16.5, -10.5, V).astype(np.float32) + shift
        x[r] = np.minimum(x[r], np.float32(-10.4))
        nh = int(rng.integers(0, 40))  # a few head entries
        x[r, rng.choice(V, nh, replace=False)] = rng.uniform(-9.0, -0.5, nh).astype(np.float32)
        if r % 3 != 2:  # copies of bucket-top values
            for t in rng.choice(tops, 4, replace=False):
                x[r, rng.choice(V, int(rng.integers(1, 300)), replace=False)] = t
        x[r, int(rng.integers(0, V))] = 0.0  # the maximum, p = 1
        for k, v in laws[r % len(laws)].items():
            p[r][k] = v
    p["seed"] = 977 + np.arange(B, dtype=np.uint64)
    w = Workload("tail", DTYPE_F32, B, V, x, p)
    us = rng.random(B).astype(np.float32)
    us[::5] = np.float32(0.9995)  # draws deep into the kept set
    us[1::7] = np.float32(1.0)
    return w, us


def _rows(w: Workload, rows) -> Workload:
    return Workload(w.name, w.dtype, len(rows), w.V, np.ascontiguousarray(w.logits[rows]),
                    np.ascontiguousarray(w.params[rows]))


@pytest.fixture(scope="module")
def sampler():
    from ax_sampler import HipSampler

    s = HipSampler(0, max_batch=128, max_vocab=V)
    yield s
    s.close()


@pytest.mark.parametrize("kept_cap", [0, 64])
@pytest.mark.parametrize("rows", ["inplace", "listed"])
def test_tail_mass_rows(sampler, oracle, tail_workload, kept_cap, rows):
    w, us = tail_workload
    if rows == "listed":  # fewer rows than the in-place threshold: k_exact_mat + k_exact_row
        sel = np.arange(0, w.B, 6)
        w, us = _rows(w, sel), np.ascontiguousarray(us[sel])
    gpu = run_gpu(sampler, w, us, kept_cap=kept_cap)
    cpu = run_oracle(oracle, w, us, kept_cap=kept_cap)
    summ = compare(w, gpu, cpu, f"tail-{rows}-{kept_cap}")
    log(f"tail mass rows ({rows}, kept_cap={kept_cap}): {summ}")
    assert summ["exact_path_rows"] == w.B
