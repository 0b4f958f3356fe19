"""The reference's own unit tests, transcribed against the CPU oracle.

Each test names the reference test it restates (file:line).  They pin the
oracle's restatement of sample_categorical_into and friends before the oracle
is trusted as the HIP sampler's parity checker.
"""
import math

import numpy as np
import pytest

from ax_sampler.params import MlxSamplingParams, pack_params


def P(mp: MlxSamplingParams) -> np.ndarray:
    return pack_params([mp])


def sample(o, logits, mp, hist=(), rng=None, **kw):
    tok, ex, kept = o.sample_row(logits, P(mp), list(hist), rng=rng, **kw)
    return tok


# --- crates/ax-engine-mlx/src/sampling.rs tests --------------------------------


def test_categorical_with_zero_temperature_is_argmax(oracle):
    # sampling.rs:976-984
    rng = oracle.Xorshift64(42)
    assert sample(oracle, [0.1, 5.0, 1.0, 2.0], MlxSamplingParams.greedy(), rng=rng) == 1


def test_min_p_drops_tokens_below_relative_threshold(oracle):
    # sampling.rs:986-997
    rng = oracle.Xorshift64(3)
    mp = MlxSamplingParams.new(1.0, 1.0, 0).with_min_p(0.05)
    for _ in range(64):
        assert sample(oracle, [10.0, 1.0, 1.0, 1.0, 1.0], mp, rng=rng) == 0


def test_min_p_keeps_comparable_tokens(oracle):
    # sampling.rs:999-1012
    rng = oracle.Xorshift64(11)
    mp = MlxSamplingParams.new(1.0, 1.0, 0).with_min_p(0.2)
    seen = {sample(oracle, [2.0, 1.9, 0.0], mp, rng=rng) for _ in range(400)}
    assert 0 in seen and 1 in seen
    assert 2 not in seen


def test_min_p_extreme_value_falls_back_to_argmax(oracle):
    # sampling.rs:1014-1022
    rng = oracle.Xorshift64(5)
    mp = MlxSamplingParams.new(1.0, 1.0, 0).with_min_p(2.0)
    tok, ex, _ = oracle.sample_row([0.5, 3.0, 1.0], P(mp), [], rng=rng)
    assert tok == 1
    assert ex["path"] == oracle.PATH_FALLBACK


def test_min_p_is_inert_for_greedy_argmax(oracle):
    # sampling.rs:1024-1030
    rng = oracle.Xorshift64(9)
    mp = MlxSamplingParams.greedy().with_min_p(0.9)
    assert sample(oracle, [0.1, 5.0, 1.0], mp, rng=rng) == 1


def test_min_p_none_keeps_exact_prior_distribution(oracle):
    # sampling.rs:1032-1044
    logits = [1.2, 0.8, 2.1, 0.3, 1.7]
    plain = MlxSamplingParams.new(0.7, 1.0, 0)
    with_none = MlxSamplingParams.new(0.7, 1.0, 0).with_min_p(None)
    a, b = oracle.Xorshift64(21), oracle.Xorshift64(21)
    for _ in range(64):
        assert sample(oracle, logits, plain, rng=a) == sample(oracle, logits, with_none, rng=b)


def test_categorical_with_high_temperature_samples_nondeterministically(oracle):
    # sampling.rs:1046-1065
    rng = oracle.Xorshift64(1)
    seen = {sample(oracle, [1.0] * 10, MlxSamplingParams.new(1.0, 1.0, 0), rng=rng) for _ in range(200)}
    assert len(seen) >= 5


def test_categorical_with_peaked_distribution_samples_mode(oracle):
    # sampling.rs:1067-1079
    logits = [0.0] * 10
    logits[3] = 20.0
    rng = oracle.Xorshift64(7)
    for _ in range(50):
        assert sample(oracle, logits, MlxSamplingParams.new(1.0, 1.0, 0), rng=rng) == 3


def test_categorical_top_k_limits_candidates(oracle):
    # sampling.rs:1081-1091
    rng = oracle.Xorshift64(11)
    for _ in range(100):
        assert sample(oracle, [1.0] * 6, MlxSamplingParams.new(1.0, 1.0, 2), rng=rng) < 2


def test_categorical_top_p_limits_candidates(oracle):
    # sampling.rs:1093-1103
    rng = oracle.Xorshift64(17)
    for _ in range(100):
        assert sample(oracle, [1.0] * 6, MlxSamplingParams.new(1.0, 0.5, 0), rng=rng) < 3


def test_categorical_applies_top_p_before_top_k(oracle):
    # sampling.rs:1247-1257
    logits = np.array([0.6, 0.2, 0.1, 0.1], dtype=np.float32)
    logits = np.log(logits).astype(np.float32)
    ids, probs = oracle.token_distribution(logits, P(MlxSamplingParams.new(1.0, 0.7, 2)))
    d = dict(zip(ids.tolist(), probs.tolist()))
    assert d.get(0, 0.0) > 0.0
    assert d.get(1, 0.0) > 0.0
    assert d.get(2, 0.0) == 0.0
    assert d.get(3, 0.0) == 0.0


def test_residual_distribution_removes_draft_mass(oracle):
    # sampling.rs:1272-1284
    target = oracle.distribution_new([(1, 0.6), (2, 0.3), (3, 0.1)])
    draft = oracle.distribution_new([(1, 0.6), (2, 0.4)])
    rng = oracle.Xorshift64(41)
    for _ in range(50):
        u = rng.next_f32()
        tok = oracle.sample_residual([t for t, _ in target], [p for _, p in target],
                                     [t for t, _ in draft], [p for _, p in draft], u)
        assert tok == 3


def test_deterministic_delta_speculation_preserves_target_distribution(oracle):
    # sampling.rs:1286-1307 (50k trials, +-0.01)
    target = oracle.distribution_new([(0, 0.6), (1, 0.3), (2, 0.1)])
    draft = oracle.distribution_new([(0, 1.0)])
    tid = [t for t, _ in target]
    tp = [p for _, p in target]
    p0 = oracle.distribution_prob(tid, tp, 0)
    rng = oracle.Xorshift64(43)
    counts = [0, 0, 0]
    trials = 50_000
    for _ in range(trials):
        if rng.next_f32() < p0:
            tok = 0
        else:
            tok = oracle.sample_residual(tid, tp, [0], [1.0], rng.next_f32())
        counts[tok] += 1
    for c, e in zip(counts, [0.6, 0.3, 0.1]):
        assert abs(c / trials - e) < 0.01


def test_xorshift_produces_distinct_values(oracle):
    # sampling.rs:1309-1315
    rng = oracle.Xorshift64(1)
    vals = [rng.next_u64() for _ in range(10)]
    assert len(set(vals)) == 10


def test_categorical_falls_back_to_argmax_on_nan_logits(oracle):
    # sampling.rs:1317-1324
    rng = oracle.Xorshift64(99)
    tok = sample(oracle, [math.nan] * 3, MlxSamplingParams.new(1.0, 1.0, 0), rng=rng)
    assert tok < 3


def test_categorical_argmax_ignores_nan_and_keeps_first_tie(oracle):
    # sampling.rs:1326-1334
    rng = oracle.Xorshift64(99)
    assert sample(oracle, [math.nan, 4.0, 4.0, 3.0], MlxSamplingParams.greedy(), rng=rng) == 1


def test_token_distribution_discards_invalid_mass_before_normalizing(oracle):
    # sampling.rs:1336-1342
    d = oracle.distribution_new([(1, 1.0), (2, -0.5), (3, math.nan), (4, 3.0)])
    assert d == [(1, 0.25), (4, 0.75)]


def test_categorical_falls_back_to_argmax_on_all_neg_inf(oracle):
    # sampling.rs:1344-1351
    rng = oracle.Xorshift64(3)
    tok, ex, _ = oracle.sample_row([-math.inf] * 4, P(MlxSamplingParams.new(1.0, 1.0, 0)), [], rng=rng)
    assert tok < 4
    assert ex["path"] == oracle.PATH_FALLBACK


def test_repetition_penalty_demotes_recent_tokens_before_argmax(oracle):
    # sampling.rs:1353-1360
    rng = oracle.Xorshift64(1)
    mp = MlxSamplingParams.greedy().with_repetition_penalty(2.0, None)
    assert sample(oracle, [1.0, 1.8, 0.9], mp, [1], rng=rng) == 0


def test_repetition_penalty_respects_context_window(oracle):
    # sampling.rs:1362-1369
    rng = oracle.Xorshift64(1)
    mp = MlxSamplingParams.greedy().with_repetition_penalty(2.0, 1)
    assert sample(oracle, [1.0, 1.8, 0.9], mp, [1, 2], rng=rng) == 1


def test_no_repeat_ngram_bans_repeated_continuation_before_greedy_argmax(oracle):
    # sampling.rs:1371-1381
    rng = oracle.Xorshift64(1)
    mp = MlxSamplingParams.greedy().with_no_repeat_ngram(3, 16)
    assert sample(oracle, [0.5, 0.4, 2.0, 0.3], mp, [1, 2, 2, 1, 2], rng=rng) == 0


def test_no_repeat_ngram_respects_recent_history_window(oracle):
    # sampling.rs:1383-1393
    rng = oracle.Xorshift64(1)
    mp = MlxSamplingParams.greedy().with_no_repeat_ngram(3, 3)
    assert sample(oracle, [0.5, 0.4, 2.0, 0.3], mp, [1, 2, 2, 1, 2], rng=rng) == 2


# --- crates/ax-engine-mlx/src/batched_sampling.rs tests ------------------------


def test_sample_batched_host_matches_per_row_sample(oracle):
    # batched_sampling.rs:214-243: batched row r == the single-row call with the
    # same params, history and RNG (here: the same supplied uniform).
    data = np.array(
        [[0.1, 5.0, 1.0, 2.0, 0.5], [4.0, 4.5, 0.2, 0.3, 0.1], [1.0, 1.1, 0.9, 3.0, 0.4]],
        dtype=np.float32,
    )
    mps = [
        MlxSamplingParams.greedy(),
        MlxSamplingParams.greedy().with_repetition_penalty(2.0, None),
        MlxSamplingParams.new(0.8, 1.0, 0),
    ]
    params = pack_params(mps)
    hist = np.array([1], dtype=np.uint32)
    hoff = np.array([0, 0, 1, 1], dtype=np.int64)
    seeds = [7, 11, 23]
    us = np.array([oracle.Xorshift64(s).next_f32() for s in seeds], dtype=np.float32)
    got, ex, _ = oracle.sample_batch(data, 0, 3, 5, 5, params, hist, hoff, uniforms=us)
    for r in range(3):
        rng = oracle.Xorshift64(seeds[r])
        want = sample(oracle, data[r], mps[r], [1] if r == 1 else [], rng=rng)
        assert got[r] == want
        # greedy rows consume no uniform; the sampled row consumes one
        assert ex[r]["drew"] == (1 if r == 2 else 0)


def test_sample_batched_host_greedy_tie_matches_single_path(oracle):
    # batched_sampling.rs:245-262 (host argmax on an all-tie row: first max)
    data = np.full((1, 4), 0.1, dtype=np.float32)
    got, _, _ = oracle.sample_batch(data, 0, 1, 4, 4, pack_params([MlxSamplingParams.greedy()]),
                                    uniforms=np.zeros(1, np.float32))
    assert got[0] == sample(oracle, data[0], MlxSamplingParams.greedy(), rng=oracle.Xorshift64(1)) == 0


# --- crates/ax-engine-core/src/sampling.rs tests --------------------------------


def test_core_deterministic_sampler_prefers_argmax_logits(oracle):
    # core sampling.rs:314-335
    r = oracle.core_argmax_logprob([0.25, 1.5, -0.5, 0.75], P(MlxSamplingParams()))
    assert r is not None
    assert r[0] == 1 and math.isfinite(r[1]) and r[1] < 0


def test_core_deterministic_sampler_marks_non_finite_logits_as_error(oracle):
    # core sampling.rs:337-354
    assert oracle.core_argmax_logprob([math.nan, math.inf], P(MlxSamplingParams())) is None


def test_core_repetition_penalty_applies_to_recent_tokens(oracle):
    # core sampling.rs:370-391
    mp = MlxSamplingParams(repetition_penalty=2.0)
    assert oracle.core_argmax_logprob([1.0, 1.8, 0.9], P(mp), [1])[0] == 0


def test_core_bans_token_that_would_repeat_ngram(oracle):
    # core sampling.rs:393-415
    mp = MlxSamplingParams(no_repeat_ngram_size=3, ngram_window=16)
    assert oracle.core_argmax_logprob([0.5, 0.4, 2.0, 0.3], P(mp), [1, 2, 2, 1, 2])[0] == 0


def test_core_ignores_invalid_repetition_penalty_with_ngram(oracle):
    # core sampling.rs:417-440
    mp = MlxSamplingParams(repetition_penalty=math.nan, no_repeat_ngram_size=3, ngram_window=16)
    assert oracle.core_argmax_logprob([0.5, 1.5, 2.0, 0.3], P(mp), [1, 2, 2, 1, 2])[0] == 1


def test_core_ties_go_to_last_max(oracle):
    # core sampling.rs:172-175 (Iterator::max_by keeps the last maximum) — the
    # documented divergence from the MLX sampler's first-max argmax.
    r = oracle.core_argmax_logprob([3.0, 7.0, 7.0, 1.0], P(MlxSamplingParams()))
    assert r[0] == 2
    assert oracle.argmax_f32([3.0, 7.0, 7.0, 1.0]) == 1


# --- crates/ax-engine-mlx/src/runner/mod.rs MTP tests ---------------------------


def test_mtp_accept_count_ngram_pseudo_logprob_rejection_samples(oracle):
    # runner/mod.rs:14948-14993
    r = oracle.mtp_accept_count([17], [0.0], [], [oracle.SRC_NGRAM], [1.0], None, [17],
                                oracle.Xorshift64(42), 1.0, 0.8, oracle.MODEL_GREEDY, oracle.NGRAM_DELTA)
    assert r == (1, True, None)
    r = oracle.mtp_accept_count([17], [0.0], [], [oracle.SRC_NGRAM], [0.0], None, [17],
                                oracle.Xorshift64(99), 1.0, 0.8, oracle.MODEL_GREEDY, oracle.NGRAM_DELTA)
    assert r[0] == 0 and r[1] is False


def test_mtp_accept_count_ngram_greedy_mode_uses_argmax_match(oracle):
    # runner/mod.rs:15039-15077
    r = oracle.mtp_accept_count([17], [0.0], [], [oracle.SRC_NGRAM], [0.0], None, [17],
                                oracle.Xorshift64(42), 1.0, 0.8, oracle.MODEL_GREEDY, oracle.NGRAM_GREEDY)
    assert r[0] == 1 and r[1]
    r = oracle.mtp_accept_count([17], [0.0], [], [oracle.SRC_NGRAM], [1.0], None, [99],
                                oracle.Xorshift64(42), 1.0, 0.8, oracle.MODEL_GREEDY, oracle.NGRAM_GREEDY)
    assert r == (0, False, 99)


def test_mtp_accept_count_ngram_nan_logprob_falls_back_to_greedy(oracle):
    # runner/mod.rs:15079-15100
    r = oracle.mtp_accept_count([17], [math.nan], [], [oracle.SRC_NGRAM], [0.0], None, [17],
                                oracle.Xorshift64(42), 1.0, 0.8, oracle.MODEL_GREEDY,
                                oracle.NGRAM_CONFIDENCE)
    assert r == (1, True, None)


def test_mtp_accept_count_ngram_rejection_ignores_draft_distribution(oracle):
    # runner/mod.rs:15102-15129
    r = oracle.mtp_accept_count([17], [math.log(0.9)], [([17], [1.0])], [oracle.SRC_NGRAM], [0.0],
                                [([99], [1.0])], [17], oracle.Xorshift64(42), 1.0, 0.8,
                                oracle.MODEL_GREEDY, oracle.NGRAM_CONFIDENCE)
    assert r == (0, False, None)


def test_mtp_model_accept_count_defaults_to_argmax_verification(oracle):
    # runner/mod.rs:15131-15152
    r = oracle.mtp_accept_count([17], [math.log(0.01)], [], [oracle.SRC_MTP], [1.0], None, [99],
                                oracle.Xorshift64(42), 1.0, 0.8, oracle.MODEL_GREEDY,
                                oracle.NGRAM_CONFIDENCE)
    assert r == (0, False, 99)


def test_mtp_accept_count_aligns_hybrid_tail_distribution_after_ngram_prefix(oracle):
    # runner/mod.rs:15154-15181
    r = oracle.mtp_accept_count(
        [10, 20], [math.nan, 0.0], [([20], [1.0])], [oracle.SRC_NGRAM, oracle.SRC_HYBRID],
        [1.0, 0.0], [([10], [1.0]), ([99], [1.0])], [10, 20], oracle.Xorshift64(7), 1.0, 0.8,
        oracle.MODEL_REJECTION, oracle.NGRAM_CONFIDENCE)
    assert r == (1, False, 99)


def test_mtp_accept_count_temperature_rescaling(oracle):
    # runner/mod.rs:15183-15245
    lp = float(np.log(np.float32(0.8)))
    r = oracle.mtp_accept_count([5], [lp], [], [oracle.SRC_MTP], [1.0], None, [5], oracle.Xorshift64(1),
                                0.7, 0.6, oracle.MODEL_REJECTION, oracle.NGRAM_CONFIDENCE)
    assert r[0] == 1
    r = oracle.mtp_accept_count([5], [lp], [], [oracle.SRC_MTP], [1.0], None, [5], oracle.Xorshift64(1),
                                0.7, 0.7, oracle.MODEL_REJECTION, oracle.NGRAM_CONFIDENCE)
    assert r[0] == 1
    ulp = float(np.log(np.float32(0.001)))
    for seed in range(10):
        r = oracle.mtp_accept_count([7], [ulp], [], [oracle.SRC_NGRAM], [0.001], None, [7],
                                    oracle.Xorshift64(seed), 0.7, 2.0, oracle.MODEL_GREEDY,
                                    oracle.NGRAM_CONFIDENCE)
        assert r[0] == 1, seed


def test_filtered_target_probs_four_sevenths(oracle):
    # runner/mod.rs:20086-20125: row = ln(.4,.3,.2,.1), top_p 0.55, top_k 2 →
    # p(0) = 4/7, p(1) = 3/7 under the filtered, renormalised law.
    row = np.log(np.array([0.4, 0.3, 0.2, 0.1], dtype=np.float32)).astype(np.float32)
    ids, probs = oracle.token_distribution(row, P(MlxSamplingParams.new(1.0, 0.55, 2)))
    d = dict(zip(ids.tolist(), probs.tolist()))
    assert abs(d[0] - 4.0 / 7.0) < 1e-6
    assert abs(d[1] - 3.0 / 7.0) < 1e-6


def test_filtered_target_probability_applies_min_p(oracle):
    # runner/mod.rs:14070-14082: probs .9/.05/.05, min_p .1 → token0 prob 1, token1 0;
    # without min-p the renormalised mass is unchanged.
    row = np.log(np.array([0.9, 0.05, 0.05], dtype=np.float32)).astype(np.float32)
    ids, probs = oracle.token_distribution(row, P(MlxSamplingParams.new(1.0, 1.0, 0).with_min_p(0.1)))
    d = dict(zip(ids.tolist(), probs.tolist()))
    assert abs(d[0] - 1.0) < 1e-5 and d.get(1, 0.0) == 0.0
    ids, probs = oracle.token_distribution(row, P(MlxSamplingParams.new(1.0, 1.0, 0)))
    d = dict(zip(ids.tolist(), probs.tolist()))
    assert abs(d[0] - 0.9) < 1e-5


def test_soft_close_probe_membership_by_rank(oracle):
    # ngram_accel.rs:1766-1776: top-3 of these logits are ids 1, 3, 2
    logits = [0.1, 5.0, 3.0, 4.0, 0.5]
    assert oracle.soft_close_in_top_k(logits, 1, 3)
    assert oracle.soft_close_in_top_k(logits, 2, 3)
    assert oracle.soft_close_in_top_k(logits, 3, 3)
    assert not oracle.soft_close_in_top_k(logits, 0, 3)
    assert not oracle.soft_close_in_top_k(logits, 4, 3)
    assert oracle.soft_close_in_top_k(logits, 1, 1)
    assert not oracle.soft_close_in_top_k(logits, 3, 1)


def test_soft_close_probe_edge_cases(oracle):
    # ngram_accel.rs:1778-1786
    assert not oracle.soft_close_in_top_k([], 0, 3)
    assert not oracle.soft_close_in_top_k([1.0, 2.0], 0, 0)
    assert not oracle.soft_close_in_top_k([1.0, 2.0], 9, 3)
    assert oracle.soft_close_in_top_k([1.0, 2.0], 0, 3)


def test_production_target_law_four_sevenths(oracle):
    # runner/mod.rs:20086-20125 (filtered_target_probs_match_gpu_topk_full_probability_sampler):
    # row ln(.4,.3,.2,.1), target top_p 0.55, top_k 2 -> p(0) = 4/7, p(1) = 3/7
    row = np.log(np.array([0.4, 0.3, 0.2, 0.1], dtype=np.float32)).astype(np.float32)
    assert abs(oracle.mtp_target_prob(row, 0, 1.0, top_p=0.55, top_k=2) - 4.0 / 7.0) < 1e-6
    assert abs(oracle.mtp_target_prob(row, 1, 1.0, top_p=0.55, top_k=2) - 3.0 / 7.0) < 1e-6


def test_production_target_law_out_of_top_k_set_is_zero(oracle):
    # runner/mod.rs:20032-20083 (topk_target_softmax_returns_zero_for_out_of_set_tokens)
    row = np.zeros(100, np.float32)
    row[:3] = [10.0, 9.0, 8.0]
    assert oracle.mtp_target_prob(row, 99, 0.8, topk_opt=3) == 0.0
    assert oracle.mtp_target_prob(row, 0, 0.8, topk_opt=3) > 0.5


def test_production_target_law_top_k_option_approximates_full(oracle):
    # runner/mod.rs:19937-20029 (topk_target_softmax_approximates_full_softmax_for_dominant_tokens)
    vocab = 100
    rows = np.zeros((3, vocab), np.float32)
    rows[0, 10], rows[0, 20] = 5.0, 4.0
    rows[1, 25], rows[1, 30] = 6.0, 3.0
    rows[2, 55], rows[2, 60] = 7.0, 2.0
    for i, tok in enumerate([10, 25, 55]):
        full = oracle.mtp_target_prob(rows[i], tok, 0.8)
        topk = oracle.mtp_target_prob(rows[i], tok, 0.8, topk_opt=32)
        assert full > 0.0 and topk > 0.0
        assert 0.85 <= topk / full < 1.15


def test_production_target_law_min_p_full_rows(oracle):
    # runner/mod.rs:14069-14080 (filtered_target_token_probability_applies_min_p):
    # probs .9/.05/.05, min_p .1 -> p(0) = 1, p(1) = 0; without min_p, .9
    row = np.log(np.array([0.9, 0.05, 0.05], dtype=np.float32)).astype(np.float32)
    assert abs(oracle.mtp_target_prob(row, 0, 1.0, min_p=0.1) - 1.0) < 1e-5
    assert oracle.mtp_target_prob(row, 1, 1.0, min_p=0.1) == 0.0
    assert abs(oracle.mtp_target_prob(row, 0, 1.0) - 0.9) < 1e-5
    assert np.isnan(oracle.mtp_target_prob(row, 0, 0.0))
