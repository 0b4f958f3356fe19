"""GPU tests of the engine-level boundary: ``HipTokenSampler`` (the
``TokenSampler`` plug-in, crates/ax-engine-core/src/sampling.rs:90-92) over
the host-pointer entry point ``axs_sample_batch_host``, and the runner-level
wrappers ``sample_batched`` / ``argmax_batched``
(crates/ax-engine-mlx/src/batched_sampling.rs:102-149), all checked against
the CPU oracle.

The first six tests transcribe the core sampler's own unit tests
(crates/ax-engine-core/src/sampling.rs:280-439) onto the GPU sampler.
"""
import math

import numpy as np
import pytest

from ax_sampler import (HipTokenSampler, MlxSamplingParams, SamplerInput, SamplerRequest, SamplingParams,
                        StopReason, argmax_batched, pack_params, sample_batched)
from ax_sampler.philox import philox_uniforms

from gpu_common import log

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sampler():
    from ax_sampler import HipSampler

    s = HipSampler(0, max_batch=64, max_vocab=151936)
    yield s
    s.close()


@pytest.fixture(scope="module")
def ts(sampler):
    return HipTokenSampler(sampler)


def req(rid, prev, logits, recent=(), gen=0, max_out=4, params=None):
    return SamplerRequest(rid, prev, None if logits is None else list(map(float, logits)),
                          list(recent), gen, max_out, params or SamplingParams())


def test_marks_max_output_boundary(ts):
    out = ts.sample(SamplerInput([req(1, 10, None, max_out=1), req(2, 20, None, max_out=4)]))
    assert (out[0].token_id, out[0].stop_reason) == (11, StopReason.MAX_OUTPUT_TOKENS)
    assert (out[1].token_id, out[1].stop_reason) == (21, None)
    assert out[0].logprob == 0.0 and out[1].logprob == 0.0


def test_prefers_argmax_logits_when_present(ts):
    out = ts.sample(SamplerInput([req(1, 99, [0.25, 1.5, -0.5, 0.75])]))
    assert out[0].token_id == 1 and out[0].stop_reason is None
    assert out[0].logprob is not None and math.isfinite(out[0].logprob) and out[0].logprob < 0.0


def test_marks_non_finite_logits_as_error(ts):
    out = ts.sample(SamplerInput([req(1, 99, [float("nan"), float("inf")])]))
    assert (out[0].token_id, out[0].stop_reason, out[0].logprob) == (0, StopReason.ERROR, None)


def test_applies_repetition_penalty_to_recent_tokens(ts):
    out = ts.sample(SamplerInput([req(1, 99, [1.0, 1.8, 0.9], recent=[1],
                                      params=SamplingParams(repetition_penalty=2.0))]))
    assert out[0].token_id == 0


def test_bans_token_that_would_repeat_ngram(ts):
    out = ts.sample(SamplerInput([req(1, 99, [0.5, 0.4, 2.0, 0.3], recent=[1, 2, 2, 1, 2],
                                      params=SamplingParams(no_repeat_ngram_size=3, ngram_window=16))]))
    assert out[0].token_id == 0


def test_ignores_invalid_repetition_penalty_with_ngram_processor(ts):
    p = SamplingParams(repetition_penalty=float("nan"), no_repeat_ngram_size=3, ngram_window=16)
    out = ts.sample(SamplerInput([req(1, 99, [0.5, 1.5, 2.0, 0.3], recent=[1, 2, 2, 1, 2], params=p)]))
    assert out[0].token_id == 1 and out[0].stop_reason is None


def test_contract_edges(ts):
    """Saturating stub and budget, total_cmp validity (+NaN invalid, -NaN
    skipped), empty logits, first-maximum ties, mixed widths in one input."""
    neg_nan = np.frombuffer(np.array([0xFFC00000], np.uint32).tobytes(), np.float32)[0]
    reqs = [
        req(1, 0xFFFFFFFF, None, gen=0xFFFFFFFF, max_out=0xFFFFFFFF),   # saturates, at budget
        req(2, 5, [neg_nan, 1.0, 0.5]),                                   # -NaN: valid, token 1
        req(3, 5, [float("nan"), 1.0, 0.5]),                              # +NaN: invalid
        req(4, 5, []),                                                    # empty: invalid
        req(5, 5, [2.0, 5.0, 5.0, 1.0]),                                  # tie: first maximum
        req(6, 5, [-np.inf, -np.inf]),                                    # no finite maximum
        req(7, 5, [0.1, 0.2, 3.0]),                                       # a different width
    ]
    out = ts.sample(SamplerInput(reqs))
    assert [o.request_id for o in out] == [1, 2, 3, 4, 5, 6, 7]
    assert (out[0].token_id, out[0].stop_reason) == (0xFFFFFFFF, StopReason.MAX_OUTPUT_TOKENS)
    assert out[1].token_id == 1 and out[1].stop_reason is None
    for o in (out[2], out[3], out[5]):
        assert (o.token_id, o.stop_reason, o.logprob) == (0, StopReason.ERROR, None)
    assert out[4].token_id == 1
    assert out[6].token_id == 2


def test_greedy_and_sampled_requests_match_the_oracle(ts, oracle):
    """A step of 24 requests over V = 151,936: greedy ones (core logprob
    within an ulp of ln), sampled ones (token = the MLX law with the
    request's Philox uniform, Philox(seed, request_id, generated_len))."""
    rs = np.random.default_rng(31)
    V = 151936
    reqs = []
    for i in range(24):
        lg = (rs.standard_normal(V, dtype=np.float32) * np.float32(3.0))
        recent = [int(x) for x in rs.integers(0, V, 64)]
        if i % 2 == 0:
            p = SamplingParams(repetition_penalty=1.1 if i % 4 == 0 else 1.0)
        else:
            p = SamplingParams(temperature=0.8, top_p=0.9, top_k=int(rs.choice([0, 40])), seed=1000 + i,
                               min_p=0.05 if i % 3 == 0 else None, repetition_penalty=1.1)
        reqs.append(SamplerRequest(100 + i, 7, lg.tolist(), recent, 3 + i, 64, p))
    out = ts.sample(SamplerInput(reqs))
    for i, (rq, o) in enumerate(zip(reqs, out)):
        lg = np.asarray(rq.logits, np.float32)
        mp = rq.sampling_params.to_mlx()
        mp.repetition_context_size = None
        pp = pack_params([mp])
        if i % 2 == 0:
            core = oracle.core_argmax_logprob(lg, pp, recent=rq.recent_tokens)
            assert o.token_id == core[0]  # no ties at these maxima
            assert abs(o.logprob - core[1]) <= float(np.spacing(np.float32(abs(core[1])))), (i, o.logprob, core)
        else:
            u = float(philox_uniforms([rq.sampling_params.seed], [rq.request_id], [rq.generated_len])[0])
            tok, ex, _ = oracle.sample_row(lg, pp, rq.recent_tokens, u=u)
            assert o.token_id == tok, (i, o.token_id, tok)
            assert o.logprob == pytest.approx(float(ex["logprob"]), rel=1e-5, abs=2e-6)
        assert o.stop_reason is None


def test_sample_batched_matches_per_row_sample(sampler, oracle):
    """crates/ax-engine-mlx/src/batched_sampling.rs:214-240 on the GPU: row r
    of sample_batched is the single-row law of row r with its own params,
    recent tokens and draw (Philox(seed, r, step) here, the row's Xorshift
    stream in the reference)."""
    import torch

    data = np.array([[0.1, 5.0, 1.0, 2.0, 0.5], [4.0, 4.5, 0.2, 0.3, 0.1], [1.0, 1.1, 0.9, 3.0, 0.4]],
                    np.float32)
    params = [MlxSamplingParams.greedy(), MlxSamplingParams.greedy().with_repetition_penalty(2.0, None),
              MlxSamplingParams.new(0.8, 1.0, 0)]
    recent = [[], [1], []]
    seeds, steps = [7, 11, 23], [0, 0, 5]
    got = sample_batched(sampler, torch.from_numpy(data).cuda(), params, recent, seeds, steps)
    for r in range(3):
        u = oracle.philox_uniform(seeds[r], r, steps[r])
        want = oracle.sample_row(data[r], pack_params([params[r]]), recent[r], u=u)[0]
        assert got[r] == want, r
    assert got[:2] == [1, 0]


def test_argmax_batched_accepts_b1v_shape(sampler):
    """crates/ax-engine-mlx/src/batched_sampling.rs:199-208."""
    import torch

    data = np.array([[0.0, 1.0, 0.5, 0.2], [3.0, 0.1, 0.2, 0.3]], np.float32).reshape(2, 1, 4)
    assert argmax_batched(sampler, torch.from_numpy(data).cuda()) == [1, 0]


def test_host_entry_matches_device_entry(sampler, oracle):
    """axs_sample_batch_host (host logits, copied on the context's stream)
    gives the same outputs as axs_sample_batch on the same data, bf16 and
    f32, with mask, bias and kept lists."""
    import torch

    from ax_sampler.synth import DTYPE_BF16, make_mixed

    from gpu_common import bias_rows, hist_rows, to_device

    for dtype, V, seed in ((DTYPE_BF16, 151936, 5), (0, 4099, 6)):
        w = make_mixed(seed, 40, V, dtype, hist_len=256, mask=True, bias=True, ngram=True)
        us = np.random.default_rng(seed).random(w.B).astype(np.float32)
        dev = sampler.sample(to_device(w), w.params, history=hist_rows(w), mask_words=w.mask,
                             bias=bias_rows(w), uniforms=us, logprobs=True, kept_cap=16)
        torch.cuda.synchronize()
        d = dev.numpy()
        h = sampler.sample_host(w.logits, w.params, history=hist_rows(w), mask_words=w.mask,
                                bias=bias_rows(w), uniforms=us, logprobs=True, kept_cap=16,
                                bf16=dtype == DTYPE_BF16)
        for a, b, name in zip(d[:3] + d[4:], h[:3] + h[4:], ("ids", "logprobs", "flags", "kept_count")):
            assert np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32)), (V, name)
        for r in range(w.B):  # kept lists: the written prefix of each row
            n = min(int(d[4][r]), 16)
            assert np.array_equal(d[3][r, :n], h[3][r, :n]), (V, r)
        log(f"host entry == device entry, dtype={dtype} V={V}")
