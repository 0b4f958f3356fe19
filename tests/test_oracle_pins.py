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


def _apply(oracle, row, mp, hist=(), mask=None, bias=None):
    out = np.array(row, dtype=np.float32)
    h = np.array(list(hist) if len(hist) else [0], dtype=np.uint32)
    bi = bv = None
    nb = 0
    if bias is not None:
        bi = np.array([b[0] for b in bias], dtype=np.uint32)
        bv = np.array([b[1] for b in bias], dtype=np.float32)
        nb = len(bias)
    oracle.lib().axo_apply_processors(out.ctypes.data, out.size, P(mp).ctypes.data, h.ctypes.data,
                                      len(hist), None if mask is None else mask.ctypes.data,
                                      None if bi is None else bi.ctypes.data,
                                      None if bv is None else bv.ctypes.data, nb)
    return out


def test_logit_bias_closed_form(oracle):
    """Build extension: each bias entry is added to its id in list order (so
    duplicates add one after another in f32), ids >= V are ignored, the bias
    comes after repetition and presence / frequency, and the mask after the
    bias.  The values are chosen so that every plausible other order gives a
    different f32 result."""
    f = np.float32
    row = [1.0, 1.0, 3.0, 0.5, -1.0]
    mp = MlxSamplingParams.greedy()
    mp.repetition_penalty = 2.0
    mp.presence_penalty, mp.frequency_penalty = 0.5, 0.25
    hist = [2, 2, 1]
    bias = [(0, 1e8), (0, -1e8), (0, 1.0),   # id 0: ((1 + 1e8) - 1e8) + 1 = 1 in f32
            (7, 5.0),                         # id 7 >= V: ignored
            (1, 1e-8),                        # id 1: after rep / presence: 1e-8
            (2, -0.25), (3, 4.0)]
    words = np.array([0b10111], dtype=np.uint32)  # id 3 disallowed
    out = _apply(oracle, row, mp, hist, mask=words, bias=bias)
    l0 = f(f(f(f(1.0) + f(1e8)) - f(1e8)) + f(1.0))
    assert l0 == f(1.0)  # list order; summing the biases first would give 2, reversed 0
    # id 1: history count 1 → rep 1/2 = 0.5, - 0.25 - 0.5 = -0.25 ... then + 1e-8
    l1 = f(f(f(f(1.0) / f(2.0)) - f(0.25)) - f(0.5))
    l1 = f(l1 + f(1e-8))
    # id 2: count 2 → 3 / 2 = 1.5, - 0.5 - 0.5 = 0.5, + (-0.25) = 0.25
    l2 = f(f(f(f(f(3.0) / f(2.0)) - f(f(0.25) * f(2.0))) - f(0.5)) + f(-0.25))
    want = [l0, l1, l2, -np.inf, f(-1.0)]
    assert out.tolist() == [float(w) for w in want], out
    # rep before presence: presence first would give (3 - 0.5 - 0.5) / 2 = 1.0
    assert l2 == f(0.25)
    # bias after presence / frequency: adding 1e-8 to 1.0 first would be lost
    assert l1 == f(-0.25) + f(1e-8) and l1 != f(-0.25)


def test_logit_bias_decides_the_draw(oracle):
    """A bias large enough to make an id the maximum makes it the greedy
    token and the only survivor of top_k = 1; an out-of-vocabulary bias id
    changes nothing."""
    rs = np.random.default_rng(12)
    V = 300
    logits = rs.normal(0, 2, V).astype(np.float32)
    t = int(np.argmin(logits))
    bias_ids = np.array([t, V + 3], dtype=np.uint32)
    bias_vals = np.array([100.0, 1e9], dtype=np.float32)
    for mp in (MlxSamplingParams.greedy(), MlxSamplingParams.new(0.8, 1.0, 1)):
        tok, _, _ = oracle.sample_row(logits, P(mp), [], u=0.5, bias_ids=bias_ids, bias_vals=bias_vals)
        assert tok == t
    tok, _, _ = oracle.sample_row(logits, P(MlxSamplingParams.greedy()), [], u=0.5,
                                  bias_ids=bias_ids[1:], bias_vals=bias_vals[1:])
    assert tok == int(np.argmax(logits))


def test_full_vocab_token_logprob_closed_form(oracle):
    """full_vocab_token_logprob (crates/ax-engine-mlx/src/sampling.rs:761-787)
    against float64 log-softmax, plus its special cases."""
    rs = np.random.default_rng(13)
    V = 5000
    logits = rs.normal(0, 3, V).astype(np.float32)
    l64 = logits.astype(np.float64)
    for T in (0.7, 1.0, 1.6):
        z = (l64 - l64.max()) / T
        lse = math.log(np.sum(np.exp(z)))
        for t in [int(np.argmax(logits)), int(np.argmin(logits)), 17, 4999]:
            want = max(z[t] - lse, -30.0)
            got = oracle.full_vocab_token_logprob(logits, t, T)
            assert abs(got - want) <= 2e-5 * max(1.0, abs(want)), (T, t, got, want)
    # floor at -30: an id 200 nats below the maximum
    x = np.array([0.0, -200.0, 0.0], dtype=np.float32)
    assert oracle.full_vocab_token_logprob(x, 1, 1.0) == -30.0
    assert oracle.full_vocab_token_logprob(x, 0, 1.0) == float(np.float32(math.log(0.5)))
    # out of range id, greedy temperature
    assert oracle.full_vocab_token_logprob(x, 3, 1.0) == -30.0
    assert oracle.full_vocab_token_logprob(x, 0, 0.0) == 0.0        # first maximum
    assert oracle.full_vocab_token_logprob(x, 2, 0.0) == -np.inf    # tie loses to id 0
    # -inf logits contribute nothing; an all -inf row has no finite mass → -30
    y = np.array([-np.inf, 1.0, -np.inf], dtype=np.float32)
    assert oracle.full_vocab_token_logprob(y, 1, 0.9) == 0.0
    assert oracle.full_vocab_token_logprob(np.full(4, -np.inf, np.float32), 1, 1.0) == -30.0


# --- MTP verify: float64 statement of the function-level law --------------------


def _dist64(logits, mp):
    ids, p, margin = law64(logits, mp)
    return ids, p / p.sum(), margin


def mtp64(tgt, dft, dids, tmp, dmp, us):
    """Float64 statement of one sequence's verify step: accept iff
    u < min(1, P(d) / q') with q' = exp(ln q * Td/Tt) (temperatures differing
    by > 1e-6), ln q = max(ln max(Q(d), 1e-37), -30)
    (crates/ax-engine-mlx/src/runner/mod.rs:12388-12419); on reject the
    residual max(P - Q, 0) over the ascending-id union, normalised, drawn with
    the tail uniform, or the target itself when the residual is empty
    (crates/ax-engine-mlx/src/sampling.rs:733-752); all accepted: the bonus
    draw of target row D (runner/mod.rs:9732-9775).  Returns (ids, smallest
    decision margin)."""
    D = len(dids)
    Tt, Td = tmp.temperature, dmp.temperature
    out, margin = [], np.inf
    for i in range(D):
        tid, tp, tm = _dist64(tgt[i], tmp)
        did, dq, dm = _dist64(dft[i], dmp)
        margin = min(margin, tm, dm)
        d = int(dids[i])
        q = float(dq[did == d].sum())
        p = float(tp[tid == d].sum())
        lnq = max(math.log(max(q, 1e-37)), -30.0)
        lps = lnq * (Td / Tt) if (Td > 0 and Tt > 0 and abs(Td - Tt) > 1e-6) else lnq
        acc = min(p / max(math.exp(lps), 1e-37), 1.0)
        u = float(us[i])
        if u < 1.0:
            margin = min(margin, abs(u - acc))
        if u < acc:
            out.append(d)
            continue
        P = dict(zip(tid.tolist(), tp.tolist()))
        Q = dict(zip(did.tolist(), dq.tolist()))
        keys = sorted(set(P) | set(Q))
        r = []
        for k in keys:
            diff = P.get(k, 0.0) - Q.get(k, 0.0)
            if k in P and k in Q and diff != 0.0:
                margin = min(margin, abs(diff))
            r.append(max(diff, 0.0))
        r = np.array(r)
        if r.sum() > 0.0:
            tok, m2 = draw64(np.array(keys), r, float(us[D]))
        else:
            tok, m2 = draw64(tid, tp, float(us[D]))
        return out + [tok], min(margin, m2)
    bid, bp, bm = law64(tgt[D], tmp)
    tok, m2 = draw64(bid, bp, float(us[D]))
    return out + [tok], min(margin, bm, m2)


def _rand_mp(rs):
    mp = MlxSamplingParams.new(float(rs.choice([0.6, 0.9, 1.3])), float(rs.choice([1.0, 0.95, 0.7])),
                               int(rs.choice([0, 0, 2, 3])))
    return mp.with_min_p(None if rs.random() < 0.6 else float(rs.choice([0.05, 0.2])))


@pytest.mark.parametrize("seed", range(30))
def test_mtp_verify_matches_float64_law(oracle, seed):
    """axo_mtp_verify_seq on V <= 8 against the float64 statement above, over
    random uniforms, wherever every decision has a margin > 1e-4."""
    from ax_sampler.params import pack_params

    rs = np.random.default_rng(1000 + seed)
    V = int(rs.integers(3, 9))
    D = int(rs.integers(1, 4))
    tgt = rs.normal(0, 1.5, (D + 1, V)).astype(np.float32)
    if seed % 5 == 0:
        dft = tgt[:D].copy()           # draft == target: residual empty → target
    else:
        dft = (tgt[:D] + rs.normal(0, 0.7, (D, V))).astype(np.float32)
    tmp = _rand_mp(rs)
    dmp = tmp if seed % 5 == 0 else _rand_mp(rs)
    N = 400
    dids = rs.integers(0, V, (N, D)).astype(np.uint32)
    us = rs.random((N, D + 1)).astype(np.float32)
    us[: N // 8, :D] = 0.0            # accept everything → bonus
    us[N // 8: N // 4, 0] = 1.0       # reject the first draft
    T = np.ascontiguousarray(np.broadcast_to(tgt, (N, D + 1, V)))
    Dr = np.ascontiguousarray(np.broadcast_to(dft, (N, D, V)))
    out_ids, out_n, acc, fl = oracle.mtp_verify_batch(T, Dr, 0, N, D, V, V, dids,
                                                      pack_params([tmp] * N), pack_params([dmp] * N),
                                                      uniforms=us, nthreads=4)
    checked = 0
    for b in range(N):
        want, margin = mtp64(tgt, dft, dids[b], tmp, dmp, us[b])
        if margin < 1e-4:
            continue
        got = out_ids[b, : out_n[b]].tolist()
        assert got == want, (seed, b, got, want, us[b].tolist(), dids[b].tolist())
        assert int(acc[b]) == min(len(want) - 1, D) and fl[b] & 0x80000000 == 0
        checked += 1
    assert checked >= N // 2, (seed, checked)


@pytest.mark.parametrize("filtered", [False, True])
def test_mtp_first_token_follows_the_target_law(oracle, filtered):
    """Speculative sampling's defining property: with equal temperatures and
    the draft token drawn from Q, the first emitted token (accepted draft or
    residual) is distributed as the target law P.  chi^2 over 40,000
    sequences."""
    from ax_sampler.params import pack_params

    rs = np.random.default_rng(77 + filtered)
    V, D, N = 6, 2, 40000
    tgt = rs.normal(0, 1.0, (D + 1, V)).astype(np.float32)
    dft = (tgt[:D] + rs.normal(0, 0.8, (D, V))).astype(np.float32)
    mp = MlxSamplingParams.new(0.8, 0.9 if filtered else 1.0, 4 if filtered else 0)
    qi, qp = oracle.token_distribution(dft[0], P(mp))
    qi1, qp1 = oracle.token_distribution(dft[1], P(mp))
    ud = rs.random((N, 2)).astype(np.float32)
    dids = np.zeros((N, D), np.uint32)
    for b in range(N):
        dids[b, 0] = oracle.sample_from_distribution(qi, qp, float(ud[b, 0]))
        dids[b, 1] = oracle.sample_from_distribution(qi1, qp1, float(ud[b, 1]))
    us = rs.random((N, D + 1)).astype(np.float32)
    T = np.ascontiguousarray(np.broadcast_to(tgt, (N, D + 1, V)))
    Dr = np.ascontiguousarray(np.broadcast_to(dft, (N, D, V)))
    pp = pack_params([mp] * N)
    out_ids, out_n, _, _ = oracle.mtp_verify_batch(T, Dr, 0, N, D, V, V, dids, pp, pp, uniforms=us,
                                                   nthreads=8)
    pid, pv, _ = _dist64(tgt[0], mp)
    first = out_ids[:, 0]
    assert set(np.unique(first).tolist()) <= set(pid.tolist())
    chi2 = sum((np.count_nonzero(first == i) - N * q) ** 2 / (N * q) for i, q in zip(pid, pv))
    assert chi2 < 25.0, chi2  # <= 5 dof, p ~ 1e-4


@pytest.mark.parametrize("seed", range(6))
def test_soft_close_probe_is_a_rank_count(oracle, seed):
    """ngram_accel.rs:1609-1640 without NaN or signed zeros: the running top
    set replaces its last entry only on a strictly larger logit, so the final
    set is the top `rank` by (logit desc, id asc): the target is in it iff
    fewer than `rank` logits beat it (larger, or equal at a lower id).
    Repeated values (bf16-like quantisation) exercise the tie rule."""
    rng = np.random.default_rng([seed, 91])
    for trial in range(40):
        n = int(rng.integers(1, 300))
        x = np.round(rng.standard_normal(n) * 2.0, int(rng.integers(0, 3))).astype(np.float32)
        x[x == 0] = np.float32(0.25)  # no zeros: +0 and -0 compare equal but sort apart
        rank = int(rng.integers(0, 12))
        for t in rng.integers(0, n, 5):
            beats = int(np.count_nonzero(x > x[t]) + np.count_nonzero(x[:t] == x[t]))
            assert oracle.soft_close_in_top_k(x, int(t), rank) == (rank > 0 and beats < rank), (seed, trial, t)


def test_soft_close_probe_nan_and_signed_zero(oracle):
    """Worked by hand from the reference's loop: the first `rank` logits sort
    by total order (+NaN above +inf, -NaN below -inf, -0 below +0), later
    ones enter only on IEEE `>`, which no value passes against a NaN and +0
    does not pass against -0."""
    nan = np.float32(np.nan)
    neg_nan = np.array([0xFFC00000], np.uint32).view(np.float32)[0]
    assert oracle.soft_close_in_top_k([nan, 1.0, 2.0], 0, 1)
    assert not oracle.soft_close_in_top_k([nan, 1.0, 2.0], 2, 1)
    # -NaN sorts last and then blocks every replacement
    assert not oracle.soft_close_in_top_k([1.0, neg_nan, 3.0], 2, 2)
    assert oracle.soft_close_in_top_k([1.0, neg_nan, 3.0], 1, 2)
    # a later +0 does not replace an earlier -0
    assert oracle.soft_close_in_top_k([-0.0, 0.0], 0, 1)
    assert not oracle.soft_close_in_top_k([-0.0, 0.0], 1, 1)
    # +0 sorts above -0 in the first rank entries, so -0 is the one replaced
    assert oracle.soft_close_in_top_k([0.0, -0.0, 1.0], 0, 2)
    assert not oracle.soft_close_in_top_k([0.0, -0.0, 1.0], 1, 2)


@pytest.mark.parametrize("seed", range(4))
def test_top_logprobs_follow_full_vocab_token_logprob(oracle, seed):
    """The top-N list is the full_vocab_token_logprob ranking: with every
    listed log-probability above the -30 clamp, the ids are the first n of
    all ids ordered by (log-probability desc, id asc) — log-probabilities
    from the function pinned by its closed form above — and the values are
    that function's.  Repeated logits exercise the lower-id tie rule."""
    rng = np.random.default_rng([seed, 17])
    for trial in range(6):
        V = int(rng.integers(1, 400))
        x = np.round(rng.standard_normal(V) * 2.0, 1).astype(np.float32)
        T = float(rng.choice([0.5, 1.0, 1.7]))
        n = int(rng.integers(1, 25))
        ids, lp = oracle.top_logprobs(x, T, n)
        full = np.array([oracle.full_vocab_token_logprob(x, i, T) for i in range(V)], np.float32)
        order = np.lexsort((np.arange(V), -full))
        k = min(n, V)
        if full[order[k - 1]] > -30.0:
            assert ids[:k].tolist() == order[:k].tolist(), (seed, trial)
        assert np.array_equal(lp[:k], full[ids[:k]])
        assert np.all(ids[k:] == 0xFFFFFFFF) and np.all(np.isneginf(lp[k:]))


def test_top_logprobs_edge_cases(oracle):
    x = np.array([1.0, 3.0, 3.0, -np.inf, np.nan], np.float32)
    ids, lp = oracle.top_logprobs(x, 0.0, 3)  # T <= 0: the first maximum only
    assert ids.tolist() == [1, 0xFFFFFFFF, 0xFFFFFFFF] and lp[0] == 0.0
    ids, lp = oracle.top_logprobs(x, 1.0, 5)  # ties to the lower id; p(NaN) = p(-inf) = 0
    assert ids.tolist() == [1, 2, 0, 3, 4]
    assert lp[3] == -30.0 and lp[4] == -30.0


def _log_softmax64(x, T):
    z = x.astype(np.float64) / T
    z = z - z.max()
    return z - np.log(np.exp(z).sum())


@pytest.mark.parametrize("seed", range(3))
def test_mtp_draft_sampled_mode_is_argmax_with_full_softmax_logprob(oracle, seed):
    """mtp_draft_tokens_sampled: the argmax and ln softmax(l / T) of it (float64
    closed form, within 1e-5)."""
    rng = np.random.default_rng([seed, 31])
    for trial in range(5):
        V = int(rng.integers(2, 3000))
        x = (rng.standard_normal(V) * 3.0).astype(np.float32)
        T = float(rng.choice([0.6, 1.0, 1.3]))
        tok, lnq, ex = oracle.mtp_draft(x, T, oracle.MTP_DRAFT_SAMPLED, 0.5)
        assert ex is None and tok == int(np.argmax(x))
        assert abs(lnq - max(_log_softmax64(x, T)[tok], -30.0)) < 1e-5


@pytest.mark.parametrize("seed", range(3))
def test_mtp_draft_stochastic_mode_inverts_the_softmax_cdf(oracle, seed):
    """mtp_draft_tokens_stochastic at T > 0: the token whose float64 CDF
    interval holds u (draws within 1e-5 of an interval end skipped), with
    ln softmax(l / T) of it; at T <= 0 the argmax with ln q at T = 1."""
    rng = np.random.default_rng([seed, 37])
    V = 500
    x = (rng.standard_normal(V) * 2.0).astype(np.float32)
    T = 0.8
    p = np.exp(_log_softmax64(x, T))
    cdf = np.cumsum(p)
    checked = 0
    for u in np.linspace(0.001, 0.999, 200).astype(np.float32):
        tok, lnq, ex = oracle.mtp_draft(x, T, oracle.MTP_DRAFT_STOCHASTIC, float(u))
        lo = cdf[tok] - p[tok]
        if min(abs(float(u) - lo), abs(float(u) - cdf[tok])) > 1e-5:
            assert lo <= float(u) < cdf[tok], (u, tok)
            checked += 1
        assert abs(lnq - max(_log_softmax64(x, T)[tok], -30.0)) < 1e-5
    assert checked > 190
    tok, lnq, _ = oracle.mtp_draft(x, 0.0, oracle.MTP_DRAFT_STOCHASTIC, 0.3)
    assert tok == int(np.argmax(x))
    assert abs(lnq - _log_softmax64(x, 1.0)[tok]) < 1e-5


def _prod_law64(x, tok, T, top_p, top_k, min_p, topk_opt):
    """The production target law in float64 (runner/mod.rs:11836-12159), for
    tiny rows; returns (P, margin of the top-p cut)."""
    z = (x.astype(np.float64) - x.max()) / T
    p = np.exp(z) / np.exp(z).sum()
    if topk_opt == 0 and top_k == 0 and not top_p < 1.0 and min_p is None:
        return p[tok], np.inf
    V = x.size
    K = min(topk_opt, V) if topk_opt else (min(top_k, V) if (top_k and top_k < V) else V)
    tp = top_p if (topk_opt or top_k or top_p < 1.0) else 1.0
    order = np.lexsort((np.arange(V), -p))[:K]
    if min_p is not None:
        order = order[p[order] >= min_p * p[order[0]]]
    margin = np.inf
    if 0.0 < tp < 1.0:
        cum = np.cumsum(p[order])
        k = int(np.searchsorted(cum, tp))  # first cum >= tp
        k = min(k, order.size - 1)
        margin = np.min(np.abs(cum - tp))
        order = order[: k + 1]
    return (p[tok] / p[order].sum() if tok in order else 0.0), margin


@pytest.mark.parametrize("seed", range(4))
def test_production_target_law_matches_float64_statement(oracle, seed):
    """Random tiny rows and laws: the oracle's f32 law within 1e-5 of its
    float64 statement (rows whose top-p cut lies within 1e-5 skipped)."""
    rng = np.random.default_rng([seed, 41])
    checked = 0
    for trial in range(60):
        V = int(rng.integers(2, 40))
        x = np.round(rng.standard_normal(V) * 2.0, 2).astype(np.float32)
        T = float(rng.choice([0.5, 1.0, 1.5]))
        top_p = float(rng.choice([1.0, 0.9, 0.6, 0.3]))
        top_k = int(rng.choice([0, 0, 3, 10]))
        min_p = [None, 0.05, 0.3][int(rng.integers(0, 3))]
        topk_opt = int(rng.choice([0, 0, 0, 5]))
        tok = int(rng.integers(0, V))
        want, margin = _prod_law64(x, tok, T, top_p, top_k, min_p, topk_opt)
        if margin < 1e-5:
            continue
        got = oracle.mtp_target_prob(x, tok, T, top_p, top_k, min_p, topk_opt)
        assert abs(got - want) < 1e-5, (seed, trial, got, want)
        checked += 1
    assert checked > 50
