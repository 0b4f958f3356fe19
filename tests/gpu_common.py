"""Helpers shared by the GPU parity tests: run a workload through the HIP
library (C ABI) and through the CPU oracle, and compare."""
import os
import sys

import numpy as np

from ax_sampler import _abi
from ax_sampler.synth import DTYPE_BF16, Workload


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def to_device(w: Workload):
    import torch

    if w.dtype == DTYPE_BF16:
        t = torch.from_numpy(np.ascontiguousarray(w.logits).view(np.int16)).view(torch.bfloat16)
    else:
        t = torch.from_numpy(np.ascontiguousarray(w.logits))
    return t.to("cuda:0")


def hist_rows(w: Workload):
    if w.hist is None:
        return None
    return [w.hist[w.hist_off[r]:w.hist_off[r + 1]] for r in range(w.B)]


def bias_rows(w: Workload):
    if w.bias_ids is None:
        return None
    return [(w.bias_ids[w.bias_off[r]:w.bias_off[r + 1]], w.bias_vals[w.bias_off[r]:w.bias_off[r + 1]])
            for r in range(w.B)]


def run_gpu(sampler, w: Workload, uniforms=None, kept_cap=0, logprobs=True, logits=None):
    import torch

    t = to_device(w) if logits is None else logits
    res = sampler.sample(t, w.params, history=hist_rows(w), mask_words=w.mask, bias=bias_rows(w),
                         uniforms=uniforms, logprobs=logprobs, kept_cap=kept_cap)
    torch.cuda.synchronize()
    return res.numpy()


def run_oracle(oracle, w: Workload, uniforms=None, kept_cap=0, nthreads=8):
    ms = w.mask.shape[1] if w.mask is not None else 0
    return oracle.sample_batch(w.logits, w.dtype, w.B, w.V, w.V, w.params, w.hist, w.hist_off,
                               w.mask, ms, w.bias_ids, w.bias_vals, w.bias_off, uniforms,
                               kept_cap=kept_cap, nthreads=nthreads)


def boundary_allowance(rows: int, frac: float = 0.02) -> int:
    """Most near-boundary MTP sequences a parity test excuses: 2% of them, at
    least 1."""
    return max(1, int(np.ceil(frac * rows)))


def compare(w: Workload, gpu, cpu, name="", check_kept=True):
    """Token ids must be equal on EVERY row, boundary rows included: the
    device computes the reference's probabilities with the same libm expf
    and reproduces its sequential f32 sums bit for bit, so a row near a
    nucleus / min-p / draw boundary (which the oracle flags and the summary
    counts) is decided identically on both sides.  Kept lists are compared
    exactly on every row, logprobs within 1e-5 relative.  Returns a summary
    dict."""
    tid, lp, fl, kid, kc = gpu
    want, ex, kept = cpu
    mism = np.nonzero(tid != want)[0]
    bnd = ex["boundary"] != 0
    assert mism.size == 0, (
        f"{name}: token mismatch on rows {mism[:10].tolist()} (boundary: {bnd[mism[:10]].tolist()}): "
        f"gpu {tid[mism[:10]]} cpu {want[mism[:10]]} "
        f"flags {[hex(int(f)) for f in fl[mism[:10]]]}"
    )
    assert not np.any(fl & np.uint32(_abi.FLAG_ERROR)), f"{name}: error flag set"
    nk = 0
    if check_kept and kid is not None and kept is not None:
        for r in range(w.B):
            n = min(int(ex[r]["n_kept"]), kid.shape[1])
            assert int(kc[r]) == int(ex[r]["n_kept"]), (name, r, int(kc[r]), int(ex[r]["n_kept"]))
            # the exact path lists never-drawn entries (p < 2^-24 of the
            # maximum's) as 0xFFFFFFFF after its ordered prefix
            row = kid[r, :n]
            none = np.nonzero(row == np.uint32(0xFFFFFFFF))[0]
            m = int(none[0]) if none.size else n
            assert np.all(row[m:] == np.uint32(0xFFFFFFFF)), (name, r, "unlisted entries not a suffix")
            assert m == n or (fl[r] & np.uint32(_abi.FLAG_EXACT_PATH)), (name, r, "unlisted kept ids")
            assert m >= 1, (name, r, "empty kept prefix")
            assert np.array_equal(row[:m], kept[r, :m]), (name, r)
            nk += 1
    drew = ex["drew"] != 0
    if lp is not None:
        sel = drew
        if sel.any():
            np.testing.assert_allclose(lp[sel], ex["logprob"][sel], rtol=1e-5, atol=2e-6)
    return {
        "rows": w.B,
        "mismatch": int(mism.size),
        "boundary_rows": int(bnd.sum()),
        "gpu_near_rows": int(np.count_nonzero(fl & np.uint32(_abi.FLAG_NEAR_ANY))),
        "exact_path_rows": int(np.count_nonzero(fl & np.uint32(_abi.FLAG_EXACT_PATH))),
        "kept_checked": nk,
    }
