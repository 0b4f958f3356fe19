"""GPU parity: the HIP sampler (through the C ABI) against the CPU oracle.

Token ids must be bit-exact on EVERY row, including the rows the oracle flags
as boundary rows (|cum - threshold| < 1e-6 of the mass at the nucleus edge or
the draw point, |p - min_p| < 1e-6 min_p, or a probability tie within 2 ulp
at the top-k cut): the device uses the host libm's expf bit for bit and
reproduces the reference's sequential f32 sums, so even those rows are
decided identically.  Boundary rows are counted and printed.  Greedy ids and
kept (top-k / nucleus) sets must match exactly; logprobs within 1e-5
relative.
"""
import math

import numpy as np
import pytest

from ax_sampler import MlxSamplingParams, pack_params
from ax_sampler import _abi
from ax_sampler.synth import (DTYPE_BF16, DTYPE_F32, Workload, f32_to_bf16_bits, make_c1, make_c2,
                              make_c3, make_c4, make_mixed)

from gpu_common import compare, log, run_gpu, run_oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sampler():
    from ax_sampler import HipSampler

    s = HipSampler(0, max_batch=256, max_vocab=262144)
    yield s
    s.close()


def _uniforms(B, seed):
    return np.random.default_rng(seed).random(B).astype(np.float32)


def test_argmax_batch_matches_oracle(sampler, oracle):
    import torch

    rs = np.random.default_rng(0)
    for dt, V in [(DTYPE_F32, 151936), (DTYPE_BF16, 262144), (DTYPE_F32, 1), (DTYPE_F32, 4099)]:
        B = 16
        x = rs.normal(0, 3, (B, V)).astype(np.float32)
        x[1, :] = 2.0                      # all tie → id 0
        x[2, V // 2:] = 1e9 if V > 1 else x[2, 0]
        x[3, :] = np.nan                   # all NaN → 0
        x[4, :] = -np.inf
        if V > 3:
            x[5, [1, 3]] = 50.0            # tie → lower id
            x[6, 0] = np.nan
            x[6, 2] = 40.0
        log(f"argmax dtype={dt} V={V}")
        if dt == DTYPE_BF16:
            bits = f32_to_bf16_bits(x)
            xf = oracle.bf16_to_f32(bits)
            t = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda()
        else:
            xf = x
            t = torch.from_numpy(x).cuda()
        ids, lp = sampler.argmax(t)
        ids2, lp2 = sampler.argmax(t)
        torch.cuda.synchronize()
        ids = ids.cpu().numpy().view(np.uint32)
        lp = lp.cpu().numpy()
        # reproducible: a second call gives the same bits
        assert np.array_equal(ids2.cpu().numpy().view(np.uint32), ids)
        assert np.array_equal(lp2.cpu().numpy().view(np.uint32), lp.view(np.uint32)), (dt, V)
        for r in range(B):
            assert ids[r] == oracle.argmax_f32(xf[r]), (dt, V, r)
            core = oracle.core_argmax_logprob(xf[r], pack_params([MlxSamplingParams()]))
            if core is not None:
                # the fast path's -ln sum exp(l - max) against its float64
                # value (the core sampler's own sequential f32 sum is what
                # axs_sample_batch reproduces: test_greedy_logprob_is_the_core_sum)
                l64 = xf[r][np.isfinite(xf[r])].astype(np.float64)
                want = -math.log(np.sum(np.exp(l64 - l64.max())))
                assert abs(lp[r] - want) <= 1e-5 * max(1.0, abs(want)), (r, lp[r], want)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_c1_single_row(sampler, oracle, seed):
    for greedy in (False, True):
        w = make_c1(seed, greedy=greedy)
        for us in (np.array([u], np.float32) for u in (0.03, 0.5, 0.97)):
            gpu = run_gpu(sampler, w, us, kept_cap=64)
            cpu = run_oracle(oracle, w, us, kept_cap=64)
            s = compare(w, gpu, cpu, f"C1 seed={seed} greedy={greedy}")
            log(f"C1 seed={seed} greedy={greedy} u={us[0]}: {s}")


def test_c2_full_config(sampler, oracle):
    w = make_c2(2)
    us = _uniforms(w.B, 22)
    gpu = run_gpu(sampler, w, us, kept_cap=64)
    cpu = run_oracle(oracle, w, us, kept_cap=64)
    log(f"C2: {compare(w, gpu, cpu, 'C2')}")
    # Philox draws: same uniforms on both sides
    gpu = run_gpu(sampler, w, None, kept_cap=64)
    ph = np.array([oracle.philox_uniform(int(w.params[r]['seed']), r, int(w.params[r]['step']))
                   for r in range(w.B)], dtype=np.float32)
    cpu = run_oracle(oracle, w, ph, kept_cap=64)
    log(f"C2 philox: {compare(w, gpu, cpu, 'C2-philox')}")


def test_c3_rows(sampler, oracle):
    w = make_c3(3, B=48)
    us = _uniforms(w.B, 33)
    gpu = run_gpu(sampler, w, us, kept_cap=64)
    cpu = run_oracle(oracle, w, us, kept_cap=64)
    log(f"C3 (48 rows): {compare(w, gpu, cpu, 'C3')}")


def test_c4_constrained(sampler, oracle):
    w = make_c4(4, B=48)
    us = _uniforms(w.B, 44)
    gpu = run_gpu(sampler, w, us, kept_cap=64)
    cpu = run_oracle(oracle, w, us, kept_cap=64)
    log(f"C4 (48 rows): {compare(w, gpu, cpu, 'C4')}")
    allowed = w.extra["allowed"]
    tid = gpu[0]
    assert all(allowed[r, tid[r]] for r in range(w.B)), "a masked id was emitted"


@pytest.mark.parametrize("dtype,V", [(DTYPE_BF16, 151936), (DTYPE_F32, 4099)])
def test_mixed_laws_segmented(sampler, oracle, dtype, V):
    """Every row law, masks, bias lists and bans on 40 rows: k_row, with the
    rows that need the exact second pass listed for k_exact_mat /
    k_exact_row."""
    w = make_mixed(21 + V % 89, 40, V, dtype, hist_len=512, mask=True, bias=True, ngram=True)
    us = _uniforms(w.B, 2000 + V)
    gpu = run_gpu(sampler, w, us, kept_cap=32)
    cpu = run_oracle(oracle, w, us, kept_cap=32)
    log(f"mixed segmented dtype={dtype} V={V}: {compare(w, gpu, cpu, f'mixed-seg-{V}')}")


@pytest.mark.parametrize("dtype,B,V", [(DTYPE_F32, 1, 151936), (DTYPE_BF16, 8, 151936),
                                       (DTYPE_F32, 70, 4099), (DTYPE_BF16, 64, 262144)])
def test_greedy_logprob_is_the_core_sum(sampler, oracle, dtype, B, V):
    """Greedy rows of axs_sample_batch return the core sampler's logprob,
    -ln of its sequential f32 sum of exp(l - max) in index order
    (crates/ax-engine-core/src/sampling.rs:177-190), with repetition penalty
    and n-gram ban applied first: the exact path's running sum reproduces the
    f32 sum bit for bit, so the two agree to the last ulp of ln (the device
    rounds ln once from double; the host's logf is within 0.52 ulp of it).
    Shapes: one row (k_stream + listed exact rows), 8 and 70 rows (k_row,
    listed), 64 rows at V = 262,144 (k_row in place)."""
    import torch

    rs = np.random.default_rng([B, V])
    x = (rs.standard_normal((B, V), dtype=np.float32) * np.float32(3.0))
    if dtype == DTYPE_BF16:
        bits = f32_to_bf16_bits(x)
        xf = oracle.bf16_to_f32(bits)
        t = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda()
    else:
        xf = x
        t = torch.from_numpy(x).cuda()
    mps, hist = [], []
    for r in range(B):
        mp = MlxSamplingParams.greedy()
        if r % 3 == 1:
            mp = mp.with_repetition_penalty(1.3, None)
        if r % 4 == 2:
            mp = mp.with_no_repeat_ngram(3, 64)
        mps.append(mp)
        hist.append(rs.integers(0, V, 96).astype(np.uint32))
    res = sampler.sample(t, pack_params(mps), history=hist, logprobs=True)
    torch.cuda.synchronize()
    tid, lp, fl, _, _ = res.numpy()
    worst = 0.0
    for r in range(B):
        core = oracle.core_argmax_logprob(xf[r], pack_params([mps[r]]), recent=hist[r])
        assert core is not None
        # token: the MLX law's first maximum (the core keeps the last; the
        # rows have no ties at their maximum)
        assert tid[r] == oracle.sample_row(xf[r], pack_params([mps[r]]), hist[r], u=0.5)[0]
        assert fl[r] & np.uint32(_abi.FLAG_GREEDY)
        ulp = float(np.spacing(np.float32(abs(core[1]))))
        worst = max(worst, abs(float(lp[r]) - core[1]) / ulp)
        assert abs(float(lp[r]) - core[1]) <= ulp, (r, float(lp[r]), core[1])
    log(f"greedy logprob dtype={dtype} B={B} V={V}: worst {worst:.2f} ulp of the core value")


@pytest.mark.parametrize("dtype,B,V", [(DTYPE_F32, 1, 151936), (DTYPE_BF16, 24, 151936), (DTYPE_F32, 80, 4099)])
def test_token_logprob_matches_full_vocab_token_logprob(sampler, oracle, dtype, B, V):
    """axs_token_logprob_batch against the oracle's full_vocab_token_logprob
    (crates/ax-engine-mlx/src/sampling.rs:761-787): the normaliser is the
    reference's index-order f32 sum reproduced bit for bit, so values agree
    to the last ulp of ln.  Covers the argmax, a random and the least likely
    token, T <= 0, an out-of-range id, an all -inf row and a NaN token."""
    import torch

    rs = np.random.default_rng([7, B, V])
    x = (rs.standard_normal((B, V), dtype=np.float32) * np.float32(3.0))
    temps = rs.choice(np.array([0.6, 1.0, 1.7], np.float32), B)
    toks = rs.integers(0, V, B).astype(np.uint32)
    if B > 3:
        x[1, :] = -np.inf
        x[2, toks[2]] = np.nan
        temps[3] = 0.0
        toks[0] = V + 5
    for r in range(4, B, 3):
        toks[r] = int(np.argmax(x[r]))
    if dtype == DTYPE_BF16:
        bits = f32_to_bf16_bits(x)
        xf = oracle.bf16_to_f32(bits)
        t = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda()
    else:
        xf = x
        t = torch.from_numpy(x).cuda()
    got = sampler.token_logprob(t, toks, temps).cpu().numpy()
    worst = 0.0
    for r in range(B):
        want = oracle.full_vocab_token_logprob(xf[r], int(toks[r]), float(temps[r]))
        if math.isinf(want):
            assert got[r] == want, (r, got[r], want)
            continue
        ulp = float(np.spacing(np.float32(abs(want))))
        worst = max(worst, abs(float(got[r]) - want) / ulp)
        assert abs(float(got[r]) - want) <= ulp, (r, float(got[r]), want)
    log(f"token logprob dtype={dtype} B={B} V={V}: worst {worst:.2f} ulp")
