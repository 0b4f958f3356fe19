"""Pins for the CPU oracle beyond the reference's own unit tests.

* Philox4x32-10 against the Random123 known-answer vectors (Salmon et al.,
  SC'11) and against vectors written by torch's PhiloxRNGEngine
  (tests/golden/philox_torch.json, made by tests/golden/make_philox_vectors.py).
* Xorshift64 against an independent integer restatement.
* The sampling law against a float64 brute force on tiny vocabularies,
  evaluated only where every decision has a margin > 1e-4 (so f32 rounding
  cannot matter): filter order, draw order, tie rules and min-p semantics are
  fixed by this, and a swapped filter order, a wrong tie rule or an index
  versus sorted draw order fails it.
* Closed forms and invariants: top_k = 1 == argmax, T -> 0+, the presence /
  frequency closed form, masked ids never drawn, distribution sums, residual of
  identical laws, the empirical law of many draws.
"""
import json
import math
import os

import numpy as np
import pytest

from ax_sampler.params import MlxSamplingParams, pack_params

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def P(mp):
    return pack_params([mp])


# --- RNGs ----------------------------------------------------------------------

RANDOM123_KAT = [
    # (ctr, key, out) — Random123 kat_vectors, philox4x32 10 rounds
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    (
        (0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344),
        (0xA4093822, 0x299F31D0),
        (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1),
    ),
]


@pytest.mark.parametrize("ctr,key,out", RANDOM123_KAT)
def test_philox_known_answers(oracle, ctr, key, out):
    assert oracle.philox4x32_10(ctr, key) == out


def test_philox_matches_torch_engine_vectors(oracle):
    with open(os.path.join(GOLDEN, "philox_torch.json")) as f:
        vec = json.load(f)
    assert len(vec["cases"]) >= 16
    for c in vec["cases"]:
        assert oracle.philox4x32_10(c["ctr"], c["key"]) == tuple(c["out"])


def test_philox_uniform_mapping(oracle):
    # uniform = (word >> 8) * 2^-24, counter = (row, step_lo, step_hi, purpose)
    seed, row, step = 0x1234_5678_9ABC_DEF0, 17, (3 << 32) | 5
    words = oracle.philox4x32_10((row, 5, 3, 0), (seed & 0xFFFFFFFF, seed >> 32))
    for w in range(4):
        u = oracle.philox_uniform(seed, row, step, 0, w)
        assert u == (words[w] >> 8) * 2.0 ** -24
        assert 0.0 <= u < 1.0


def xorshift_py(seed, n):
    M = (1 << 64) - 1
    s = (seed + 0x9E3779B97F4A7C15) & M
    s = 1 if s == 0 else s
    out = []
    for _ in range(n):
        s ^= (s << 13) & M
        s ^= s >> 7
        s ^= (s << 17) & M
        out.append(s)
    return out


@pytest.mark.parametrize("seed", [0, 1, 42, 0x61C8864680B583EB, 2**64 - 1])
def test_xorshift64_matches_integer_restatement(oracle, seed):
    want = xorshift_py(seed, 200)
    r = oracle.Xorshift64(seed)
    assert [r.next_u64() for _ in range(200)] == want
    r = oracle.Xorshift64(seed)
    for w in want:
        assert r.next_f32() == float(np.float32(w >> 11) * np.float32(2.0 ** -53))


def test_xorshift_next_f32_can_return_one(oracle):
    # (x >> 11) rounds to nearest f32, so 2^53 - 1 maps to 2^53 → 1.0 exactly
    assert float(np.float32((1 << 53) - 1) * np.float32(2.0 ** -53)) == 1.0


# --- float64 brute force of the law ---------------------------------------------


def law64(logits, mp):
    """Independent float64 statement of the reference law: returns (order, kept
    ids, cumulative masses, min margin) or None for argmax fallbacks."""
    l = np.asarray(logits, dtype=np.float64)
    V = l.size
    m = np.max(l)
    p = np.exp((l - m) / mp.temperature)
    ids = np.arange(V)
    margin = np.inf
    if mp.uses_min_p():
        margin = min(margin, np.min(np.abs(p - mp.min_p)) / mp.min_p)
        keep = p >= mp.min_p
        ids, p = ids[keep], p[keep]
    sorted_order = mp.top_k > 0 or mp.top_p < 1.0
    if sorted_order:
        o = np.lexsort((ids, -p))
        ids, p = ids[o], p[o]
        if 0.0 < mp.top_p < 1.0:
            total = p.sum()
            cum = np.cumsum(p)
            cut = mp.top_p * total
            n = int(np.argmax(cum >= cut - 1e-300)) + 1
            margin = min(margin, abs(cum[n - 1] - cut) / total)
            if n >= 2:
                margin = min(margin, abs(cut - cum[n - 2]) / total)
            ids, p = ids[:n], p[:n]
        if mp.top_k > 0:
            ids, p = ids[: mp.top_k], p[: mp.top_k]
    return ids, p, margin


def draw64(ids, p, u):
    F = p.sum()
    cum = np.cumsum(p)
    j = int(np.argmax(cum >= u * F))
    lo = cum[j - 1] if j > 0 else -np.inf
    margin = min(abs(cum[j] - u * F), abs(u * F - lo)) / F
    return int(ids[j]), margin


@pytest.mark.parametrize("seed", range(40))
def test_law_matches_float64_brute_force_on_tiny_vocab(oracle, seed):
    rs = np.random.default_rng(seed)
    V = int(rs.integers(2, 9))
    logits = rs.normal(0, 2.0, V).astype(np.float32)
    T = float(rs.choice([0.5, 0.8, 1.0, 1.7]))
    top_k = int(rs.choice([0, 0, 1, 2, 3]))
    top_p = float(rs.choice([1.0, 0.9, 0.6, 0.3]))
    min_p = rs.choice([None, 0.05, 0.3])
    mp = MlxSamplingParams.new(T, top_p, top_k).with_min_p(None if min_p is None else float(min_p))
    ids, p, margin = law64(logits, mp)
    checked = 0
    for u in np.linspace(0.0005, 0.9995, 97, dtype=np.float32):
        tok_ref, dm = draw64(ids, p, float(u))
        if margin < 1e-4 or dm < 1e-4:
            continue
        tok, ex, kept = oracle.sample_row(logits, P(mp), [], u=float(u), kept_cap=16)
        assert tok == tok_ref, (seed, float(u))
        assert kept.tolist() == ids.tolist()
        checked += 1
    assert checked > 0 or margin < 1e-4


def test_min_p_only_draws_in_index_order(oracle):
    # min-p alone leaves the survivors in index order (retain keeps order,
    # apply_top_k_top_p is a no-op): with survivors {0: p=0.5, 2: p=1} a draw at
    # u just above 1/3 lands on id 2 only in index order.
    logits = np.array([math.log(0.5), -20.0, 0.0], dtype=np.float32)
    mp = MlxSamplingParams.new(1.0, 1.0, 0).with_min_p(0.1)
    tok, ex, kept = oracle.sample_row(logits, P(mp), [], u=0.34, kept_cap=4)
    assert kept.tolist() == [0, 2] and ex["sorted"] == 0
    assert tok == 2
    # with top_k the same row is sorted (2 first) and u=0.34 lands on id 2 too,
    # but u=0.9 lands on id 0
    mp2 = MlxSamplingParams.new(1.0, 1.0, 2).with_min_p(0.1)
    tok, ex, kept = oracle.sample_row(logits, P(mp2), [], u=0.9, kept_cap=4)
    assert kept.tolist() == [2, 0] and ex["sorted"] == 1 and tok == 0


def test_top_k_set_is_the_stable_sorted_prefix(oracle):
    rs = np.random.default_rng(5)
    for _ in range(20):
        V = 300
        logits = np.round(rs.normal(0, 2, V), 1).astype(np.float32)  # many exact ties
        k = int(rs.integers(1, 40))
        tok, ex, kept = oracle.sample_row(logits, P(MlxSamplingParams.new(1.0, 1.0, k)), [], u=0.5,
                                          kept_cap=64)
        p = np.exp((logits.astype(np.float64) - logits.max()))
        order = np.lexsort((np.arange(V), -p))
        assert kept.tolist() == order[:k].tolist()


def test_top_k_one_is_argmax_for_every_uniform(oracle):
    rs = np.random.default_rng(9)
    logits = rs.normal(0, 3, 1000).astype(np.float32)
    a = int(np.argmax(logits))
    for u in [0.0, 0.3, 0.999, 1.0]:
        assert oracle.sample_row(logits, P(MlxSamplingParams.new(0.7, 0.95, 1)), [], u=u)[0] == a


def test_temperature_to_zero_plus_is_argmax_and_subnormal_falls_back(oracle):
    logits = np.array([0.1, 3.0, 2.9, -1.0], dtype=np.float32)
    for T in (1e-30, 1e-38):
        tok, ex, _ = oracle.sample_row(logits, P(MlxSamplingParams.new(T, 1.0, 0)), [], u=0.99)
        assert tok == 1
    # T so small that 1/T overflows: every p is NaN→0 → argmax fallback
    tok, ex, _ = oracle.sample_row(logits, P(MlxSamplingParams.new(1e-45, 1.0, 0)), [], u=0.5)
    assert tok == 1 and ex["path"] == oracle.PATH_FALLBACK and ex["drew"] == 0


def test_presence_frequency_closed_form(oracle):
    # build extension: a history holding id 1 three times and id 2 once ⇒
    # l1 - 3*freq - presence, l2 - freq - presence (presence/frequency window =
    # the repetition window).
    row = np.array([1.0, 2.0, 3.0, 0.5], dtype=np.float32)
    mp = MlxSamplingParams.greedy()
    mp.presence_penalty, mp.frequency_penalty = 0.5, 0.25
    out = row.copy()
    hist = np.array([1, 2, 1, 1, 9], dtype=np.uint32)  # 9 >= V is ignored
    oracle.lib().axo_apply_processors(out.ctypes.data, 4, P(mp).ctypes.data, hist.ctypes.data, 5,
                                      None, None, None, 0)
    want = [1.0, np.float32(np.float32(2.0) - np.float32(0.75)) - np.float32(0.5),
            np.float32(np.float32(3.0) - np.float32(0.25)) - np.float32(0.5), 0.5]
    assert out.tolist() == [float(w) for w in want]


def test_masked_ids_are_never_drawn(oracle):
    rs = np.random.default_rng(11)
    V = 500
    logits = rs.normal(0, 3, V).astype(np.float32)
    allowed = rs.random(V) < 0.2
    words = np.zeros((V + 31) // 32, dtype=np.uint32)
    for t in np.nonzero(allowed)[0]:
        words[t >> 5] |= np.uint32(1 << (t & 31))
    mp = MlxSamplingParams.new(1.0, 0.9, 0)
    for u in np.linspace(0, 1, 200):
        tok, _, _ = oracle.sample_row(logits, P(mp), [], u=float(u), mask_words=words)
        assert allowed[tok]


def test_distribution_sums_to_one_and_residual_of_identical_laws_is_target(oracle):
    rs = np.random.default_rng(2)
    logits = rs.normal(0, 3, 2000).astype(np.float32)
    ids, probs = oracle.token_distribution(logits, P(MlxSamplingParams.new(0.6, 0.95, 0)))
    assert abs(float(np.sum(probs, dtype=np.float64)) - 1.0) < 1e-6
    for u in np.linspace(0.01, 0.99, 25):
        # residual of P against itself is empty → sampled from the target
        r = oracle.sample_residual(ids, probs, ids, probs, float(u))
        assert r == oracle.sample_from_distribution(ids, probs, float(u))


def test_empirical_law_matches_kept_distribution(oracle):
    rs = np.random.default_rng(4)
    logits = rs.normal(0, 1.0, 12).astype(np.float32)
    mp = MlxSamplingParams.new(0.9, 0.8, 5)
    ids, p, _ = law64(logits, mp)
    p = p / p.sum()
    n = 20000
    us = rs.random(n).astype(np.float32)
    counts = {}
    for u in us:
        t = oracle.sample_row(logits, P(mp), [], u=float(u))[0]
        counts[t] = counts.get(t, 0) + 1
    assert set(counts) <= set(ids.tolist())
    chi2 = sum((counts.get(int(i), 0) - n * q) ** 2 / (n * q) for i, q in zip(ids, p))
    assert chi2 < 30.0  # 4 dof, p ~ 1e-5


def test_core_logprob_closed_form(oracle):
    rs = np.random.default_rng(8)
    logits = rs.normal(0, 2, 5000).astype(np.float32)
    tok, lp = oracle.core_argmax_logprob(logits, P(MlxSamplingParams()))
    l64 = logits.astype(np.float64)
    assert tok == int(np.argmax(logits))
    assert abs(lp - (-math.log(np.sum(np.exp(l64 - l64.max()))))) < 1e-5
