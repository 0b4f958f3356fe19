"""GPU parity of the MTP speculative verify step (axs_mtp_verify, kernel
k_mtp_verify over the pipeline's kept lists) against the CPU oracle's
function-level law (crates/ax-engine-mlx/src/runner/mod.rs:12333-12462,
crates/ax-engine-mlx/src/sampling.rs:647-752).

Kept sets of any size are verified on the device (lists longer than
2,048 ids are read from the rows' own buffers).

Per sequence the emitted ids (accepted prefix + residual / bonus tail), their
count and the accept count must equal the oracle's, except on sequences the
oracle flags as near a decision boundary (|u - p/q| < 1e-6 with u < 1, or a
near flag in one of the sequence's distributions), which are counted and
bounded (at most 2% of the sequences, at least 1).  u = 1 never accepts on
either side, so the empty-residual fallback of draft == target is held
exactly.  Draft ids are drawn
from the draft law by the oracle with its own uniforms (config C5).
"""
import math

import numpy as np
import pytest

from ax_sampler import _abi
from ax_sampler.synth import DTYPE_BF16, DTYPE_F32, bf16_bits_to_f32, f32_to_bf16_bits, make_c5

from gpu_common import boundary_allowance, log

pytestmark = pytest.mark.gpu

NEAR = _abi.MTP_FLAG_NEAR_ACCEPT | _abi.MTP_FLAG_NEAR


@pytest.fixture(scope="module")
def sampler():
    from ax_sampler import HipSampler

    s = HipSampler(0, max_batch=256, max_vocab=262144)
    yield s
    s.close()


def _draft_ids(oracle, draft, dtype, B, D, V, dparams, seed):
    """One token per draft row from the draft law (sample_categorical_into)."""
    rows = draft.reshape(B * D, V)
    p = np.repeat(dparams, D)
    us = np.random.default_rng(seed).random(B * D).astype(np.float32)
    ids, _, _ = oracle.sample_batch(rows, dtype, B * D, V, V, p, uniforms=us, nthreads=8,
                                    explain=False)
    return ids.reshape(B, D).astype(np.uint32)


def _to_dev(a, dtype):
    import torch

    if dtype == DTYPE_BF16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _run(sampler, oracle, tgt, dft, dtype, tp, dp, dids, us, name, strict=False):
    """strict: every sequence equal except those near an accept decision
    (|u - p/q| < 1e-6): a distribution's near flags excuse nothing, since the
    device forms the distributions exactly."""
    import torch

    B, D1, V = tgt.shape
    D = D1 - 1
    res = sampler.mtp_verify(_to_dev(tgt, dtype), _to_dev(dft, dtype), dids, tp, dp, uniforms=us)
    torch.cuda.synchronize()
    g_ids = res.out_ids.cpu().numpy().view(np.uint32)
    g_n = res.out_count.cpu().numpy().view(np.uint32)
    g_ac = res.accept_count.cpu().numpy().view(np.uint32)
    g_fl = res.flags.cpu().numpy().view(np.uint32)
    c_ids, c_n, c_ac, c_fl = oracle.mtp_verify_batch(tgt, dft, dtype, B, D, V, V, dids, tp, dp,
                                                     uniforms=us, nthreads=8)
    near = (c_fl & np.uint32(_abi.MTP_FLAG_NEAR_ACCEPT if strict else NEAR)) != 0
    assert int(near.sum()) <= boundary_allowance(B), (
        f"{name}: {int(near.sum())} of {B} sequences near a boundary")
    bad = []
    for b in range(B):
        same = g_n[b] == c_n[b] and g_ac[b] == c_ac[b] and np.array_equal(g_ids[b, :g_n[b]],
                                                                           c_ids[b, :c_n[b]])
        if not same and not near[b]:
            bad.append(b)
    assert not bad, (f"{name}: sequences {bad[:8]} differ: gpu n={g_n[bad[:8]]} ac={g_ac[bad[:8]]} "
                     f"ids={g_ids[bad[:8]].tolist()} | cpu n={c_n[bad[:8]]} ac={c_ac[bad[:8]]} "
                     f"ids={c_ids[bad[:8]].tolist()} flags gpu={g_fl[bad[:8]]} cpu={c_fl[bad[:8]]}")
    assert not np.any(g_fl & np.uint32(_abi.MTP_FLAG_ERROR)), f"{name}: error flag"
    tail = (g_fl & np.uint32(_abi.MTP_FLAG_RESIDUAL | _abi.MTP_FLAG_BONUS)) != 0
    summ = {"seqs": B, "near": int(near.sum()), "accepted": int(g_ac.sum()),
            "residual": int(np.count_nonzero(g_fl & np.uint32(_abi.MTP_FLAG_RESIDUAL))),
            "bonus": int(np.count_nonzero(g_fl & np.uint32(_abi.MTP_FLAG_BONUS))), "tail": int(tail.sum())}
    log(f"{name}: {summ}")
    return summ, g_ac


def test_c5_full(sampler, oracle):
    t, d, tp, dp = make_c5(5)
    B, D1, V = t.shape
    D = D1 - 1
    dids = _draft_ids(oracle, d, DTYPE_BF16, B, D, V, dp, 55)
    us = np.random.default_rng(505).random((B, D + 1)).astype(np.float32)
    s, _ = _run(sampler, oracle, t, d, DTYPE_BF16, tp, dp, dids, us, "C5")
    assert s["accepted"] > 0 and s["residual"] + s["bonus"] == B


def test_c5_philox(sampler, oracle):
    t, d, tp, dp = make_c5(15)
    B, D1, V = t.shape
    dids = _draft_ids(oracle, d, DTYPE_BF16, B, D1 - 1, V, dp, 56)
    _run(sampler, oracle, t, d, DTYPE_BF16, tp, dp, dids, None, "C5-philox")


def test_accept_all_and_reject_first(sampler, oracle):
    t, d, tp, dp = make_c5(25, B=16, V=32768)
    B, D1, V = t.shape
    D = D1 - 1
    dids = _draft_ids(oracle, d, DTYPE_BF16, B, D, V, dp, 57)
    us = np.zeros((B, D + 1), np.float32)
    us[:, D] = np.linspace(0.02, 0.98, B)
    s, ac = _run(sampler, oracle, t, d, DTYPE_BF16, tp, dp, dids, us, "accept-all")
    assert s["bonus"] == B and np.all(ac == D)
    us[:, :D] = 1.0  # u < min(1, p/q) never holds for u = 1: every first draft rejected
    s, ac = _run(sampler, oracle, t, d, DTYPE_BF16, tp, dp, dids, us, "reject-first")
    assert np.all(ac == 0) and s["residual"] == B


def test_draft_equals_target(sampler, oracle):
    """q == p: the residual max(p - q, 0) is empty and falls back to the target."""
    t, _, tp, dp = make_c5(35, B=8, V=16384)
    B, D1, V = t.shape
    D = D1 - 1
    d = np.ascontiguousarray(t[:, :D, :])
    dp = tp.copy()
    dids = _draft_ids(oracle, d, DTYPE_BF16, B, D, V, dp, 58)
    us = np.random.default_rng(508).random((B, D + 1)).astype(np.float32)
    us[: B // 2, 0] = 1.0
    _run(sampler, oracle, t, d, DTYPE_BF16, tp, dp, dids, us, "draft==target")


@pytest.mark.parametrize("dtype,B,D,V", [(DTYPE_F32, 24, 1, 4099), (DTYPE_BF16, 8, 7, 8192),
                                         (DTYPE_F32, 12, 2, 50000)])
def test_depths_and_dtypes(sampler, oracle, dtype, B, D, V):
    rng = np.random.default_rng([B, D, V])
    t = (rng.standard_normal((B, D + 1, V), dtype=np.float32) * np.float32(3.0))
    d = t[:, :D, :] + rng.standard_normal((B, D, V), dtype=np.float32) * np.float32(0.5)
    if dtype == DTYPE_BF16:
        t, d = f32_to_bf16_bits(t), f32_to_bf16_bits(d)
    _, _, tp, dp = make_c5(45, B=B, depth=D, V=16)
    tp["temperature"] = rng.choice(np.array([0.6, 1.0, 1.4], np.float32), B)
    tp["top_k"] = rng.choice(np.array([20, 40], np.uint32), B)
    dp["temperature"] = tp["temperature"] * np.float32(0.9)
    dp["top_k"] = tp["top_k"]
    dids = _draft_ids(oracle, d, dtype, B, D, V, dp, 59)
    us = rng.random((B, D + 1)).astype(np.float32)
    _run(sampler, oracle, t, d, dtype, tp, dp, dids, us, f"mtp dtype={dtype} B={B} D={D} V={V}")


@pytest.mark.parametrize("V,law", [(8192, "sorted"), (151936, "sorted"), (151936, "index"), (8192, "mixed")])
def test_kept_sets_beyond_the_list_capacity(sampler, oracle, V, law):
    """Distributions keeping more than 2,048 ids (the short kept lists'
    capacity) are verified on the device from the rows' own buffers (sorted
    keys, or the dense row of an index-order law), held to the oracle like
    every other sequence: flat logits at T = 1 with top-p 0.95 keep ~90% of
    the vocabulary; without filters every id is kept.  Each sequence's
    rejection draws a residual over the full id range; draft == target
    sequences exercise the empty-residual fallback."""
    rng = np.random.default_rng([V, len(law)])
    B, D = 8, 2
    t = rng.standard_normal((B, D + 1, V), dtype=np.float32) * np.float32(0.3)
    d = t[:, :D, :] + rng.standard_normal((B, D, V), dtype=np.float32) * np.float32(0.1)
    d[B - 1] = t[B - 1, :D]  # draft == target: residual empty on rejection
    _, _, tp, dp = make_c5(48, B=B, depth=D, V=16)
    tp["temperature"], dp["temperature"] = 1.0, 1.0
    tp["has_min_p"], dp["has_min_p"] = 0, 0
    if law == "index":
        tp["top_p"], tp["top_k"], dp["top_p"], dp["top_k"] = 1.0, 0, 1.0, 0
    else:
        tp["top_p"], tp["top_k"], dp["top_p"], dp["top_k"] = 0.95, 0, 0.95, 0
    if law == "mixed":  # long target lists against short draft lists, and the reverse
        tp["top_k"] = np.array([0, 40] * (B // 2), np.uint32)
        dp["top_k"] = np.array([40, 0] * (B // 2), np.uint32)
    dids = _draft_ids(oracle, d, DTYPE_F32, B, D, V, dp, 62)
    us = rng.random((B, D + 1)).astype(np.float32)
    us[:, 0] = np.float32(0.9999)  # reject the first draft: every sequence takes the residual
    us[1, 0] = np.float32(0.0)  # except one
    _run(sampler, oracle, t, d, DTYPE_F32, tp, dp, dids, us, f"long kept lists V={V} {law}", strict=True)


def test_index_order_laws_with_zero_probabilities(sampler, oracle):
    """No top-k / top-p / min-p: the distribution is every id with p > 0 in
    index order (TokenDistribution::new drops p = 0,
    crates/ax-engine-mlx/src/sampling.rs:128-144).  Rows with -inf logits
    (p = 0) are held to the oracle, not declined."""
    rng = np.random.default_rng(88)
    B, D, V = 6, 2, 1500
    t = rng.standard_normal((B, D + 1, V), dtype=np.float32) * np.float32(2.0)
    d = t[:, :D, :] + rng.standard_normal((B, D, V), dtype=np.float32) * np.float32(0.4)
    t[:, :, rng.integers(0, V, 40)] = -np.inf
    d[:, :, rng.integers(0, V, 40)] = -np.inf
    _, _, tp, dp = make_c5(47, B=B, depth=D, V=16)
    tp["temperature"], tp["top_p"], tp["top_k"] = 1.0, 1.0, 0
    dp["temperature"], dp["top_p"], dp["top_k"] = 1.0, 1.0, 0
    tp["has_min_p"] = 0
    dp["has_min_p"] = 0
    dids = _draft_ids(oracle, d, DTYPE_F32, B, D, V, dp, 61)
    us = rng.random((B, D + 1)).astype(np.float32)
    _run(sampler, oracle, t, d, DTYPE_F32, tp, dp, dids, us, "index-order with p = 0")


# --- axs_mtp_verify_ex: mtp_accept_count's modes, sources and tail ----------------


def _mtp_expect(oracle, tf, df, dids, tp, dp, us, opts, D):
    """The reference law for one sequence with the oracle's pieces:
    axo_mtp_accept_count (crates/ax-engine-mlx/src/runner/mod.rs:12333-12462)
    over P_i / Q_i = token_distribution, then the tail
    (runner/mod.rs:9732-9775): correction, bonus draw of row D, or the draw
    of the target row at the rejected position (delta residual for an n-gram
    draft when delta_correction is set).  Returns (ids, accept_count)."""
    from ax_sampler import _abi

    Tt, Td = float(tp["temperature"][0]), float(dp["temperature"][0])
    src = [int(x) if int(x) in (1, 2, 3, 4) else 1 for x in (opts.get("sources") if opts.get("sources") is not None
                                                            else np.ones(D, np.uint32))]
    P = [oracle.token_distribution(tf[i], tp) for i in range(D)]
    Q = [oracle.token_distribution(df[i], dp) for i in range(D)]
    lnq, tests = [], []
    for i in range(D):
        has_dd = src[i] != _abi.MTP_SRC_NGRAM
        if opts.get("pending_log_probs") is not None:
            v = float(opts["pending_log_probs"][i])
        elif not has_dd:
            v = 0.0 if opts.get("ngram_mode") == _abi.MTP_NGRAM_DELTA else float("nan")
        elif opts.get("lnq_mode") == _abi.MTP_LNQ_FULL_SOFTMAX:
            v = oracle.full_vocab_token_logprob(df[i], int(dids[i]), Td)
        else:
            v = oracle.logprob_of(oracle.distribution_prob(Q[i][0], Q[i][1], int(dids[i])))
        lnq.append(v)
        greedy = ((src[i] == _abi.MTP_SRC_NGRAM and opts.get("ngram_mode") == _abi.MTP_NGRAM_GREEDY) or
                  (has_dd and opts.get("model_mode", 1) == _abi.MTP_MODEL_GREEDY))
        tests.append((not greedy) and math.isfinite(v) and Tt > 0)
    pred = (list(map(int, opts["predicted"])) if opts.get("predicted") is not None
            else [oracle.argmax_f32(tf[i]) for i in range(D)])
    if Tt > 0 and opts.get("target_law") == _abi.MTP_TARGET_FILTERED:
        mp = float(tp["min_p"][0]) if int(tp["has_min_p"][0]) else None
        tprobs = [oracle.mtp_target_prob(tf[i], int(dids[i]), Tt, float(tp["top_p"][0]), int(tp["top_k"][0]), mp,
                                         int(opts.get("target_topk", 0))) for i in range(D)]
    else:
        tprobs = [max(oracle.distribution_prob(P[i][0], P[i][1], int(dids[i])), 0.0) for i in range(D)] \
            if Tt > 0 else None
    ac, allacc, corr = oracle.mtp_accept_count(
        list(map(int, dids)), lnq, [Q[i] for i in range(D) if src[i] != _abi.MTP_SRC_NGRAM], src, tprobs, P,
        pred, None, Td, Tt, opts.get("model_mode", 1), opts.get("ngram_mode", 0), uniforms=us)
    k = sum(tests[: min(ac, D - 1) + 1]) if not allacc else sum(tests)
    if allacc:
        tail = oracle.sample_row(tf[D], tp, [], u=float(us[k]))[0]
    elif corr is not None:
        tail = corr
    elif opts.get("delta_correction"):
        tail = oracle.sample_residual(P[ac][0], P[ac][1], [int(dids[ac])], [1.0], float(us[k]))
    else:
        tail = oracle.sample_row(tf[ac], tp, [], u=float(us[k]))[0]
    return list(map(int, dids[:ac])) + [int(tail)], ac


def _ex_case(seed, B=16, D=3, V=4099):
    rng = np.random.default_rng(seed)
    t = rng.standard_normal((B, D + 1, V), dtype=np.float32) * np.float32(2.5)
    d = t[:, :D, :] + rng.standard_normal((B, D, V), dtype=np.float32) * np.float32(0.6)
    _, _, tp, dp = make_c5(48 + seed, B=B, depth=D, V=16)
    tp["temperature"] = rng.choice(np.array([0.7, 1.0], np.float32), B)
    dp["temperature"] = tp["temperature"] * rng.choice(np.array([1.0, 0.9], np.float32), B)
    tp["top_k"], dp["top_k"] = 40, 40
    tp["top_p"], dp["top_p"] = 0.95, 0.95
    return rng, t, d, tp, dp


@pytest.mark.parametrize("case", ["rejection", "modes", "full_lnq", "greedy_target", "supplied"])
def test_mtp_verify_ex_matches_accept_count(sampler, oracle, case):
    import torch

    from ax_sampler import _abi

    rng, t, d, tp, dp = _ex_case({"rejection": 1, "modes": 2, "full_lnq": 3, "greedy_target": 4, "supplied": 5}[case])
    B, D1, V = t.shape
    D = D1 - 1
    dids = _draft_ids(oracle, d, DTYPE_F32, B, D, V, dp, 62)
    opts = {"model_mode": _abi.MTP_MODEL_REJECTION}
    if case == "modes" or case == "supplied":
        opts["sources"] = rng.choice(np.array([0, 1, 2, 3, 4], np.uint32), (B, D))
        opts["ngram_mode"] = int(rng.integers(0, 3))
        opts["model_mode"] = int(rng.integers(0, 2))
        opts["delta_correction"] = bool(rng.integers(0, 2))
        # n-gram drafts: the target's argmax half of the time, else a random id
        am = np.array([[oracle.argmax_f32(t[b, i]) for i in range(D)] for b in range(B)], np.uint32)
        ng = opts["sources"] == 3
        dids = np.where(ng & (rng.random((B, D)) < 0.5), am, np.where(ng, rng.integers(0, V, (B, D)), dids)
                        ).astype(np.uint32)
    if case == "supplied":
        opts["pending_log_probs"] = np.where(rng.random((B, D)) < 0.2, np.nan,
                                             -rng.random((B, D)) * 3).astype(np.float32)
        opts["predicted"] = rng.integers(0, V, (B, D)).astype(np.uint32)
    if case == "full_lnq":
        opts["lnq_mode"] = _abi.MTP_LNQ_FULL_SOFTMAX
    if case == "greedy_target":
        tp["temperature"][: B // 2] = 0.0
    us = rng.random((B, D + 1)).astype(np.float32)
    res = sampler.mtp_verify(_to_dev(t, DTYPE_F32), _to_dev(d, DTYPE_F32), dids, tp, dp, uniforms=us,
                             options=opts)
    torch.cuda.synchronize()
    g_ids, g_n, g_ac, g_fl = res.numpy()
    near = 0
    for b in range(B):
        ob = {k: (v[b] if isinstance(v, np.ndarray) else v) for k, v in opts.items()}
        want, ac = _mtp_expect(oracle, t[b], d[b], dids[b], tp[b:b + 1], dp[b:b + 1], us[b], ob, D)
        got = g_ids[b, : g_n[b]].tolist()
        assert not g_fl[b] & np.uint32(_abi.MTP_FLAG_ERROR), (case, b)
        if g_fl[b] & np.uint32(_abi.MTP_FLAG_NEAR_ACCEPT):
            near += 1
            continue
        assert got == want and g_ac[b] == ac, (case, b, got, want, int(g_ac[b]), ac, hex(int(g_fl[b])))
    assert near <= boundary_allowance(B), near
    log(f"mtp_verify_ex {case}: {B} sequences, near {near}, accepted {int(g_ac.sum())}")


def test_mtp_verify_ex_every_mode(sampler, oracle):
    """Every (model mode, n-gram mode, delta correction) combination, mixed
    sources per position, against the oracle's mtp_accept_count + tail."""
    import itertools

    import torch

    from ax_sampler import _abi

    for mm, nm, dc in itertools.product((0, 1), (0, 1, 2), (False, True)):
        rng, t, d, tp, dp = _ex_case(100 + mm * 10 + nm * 2 + int(dc), B=8)
        B, D1, V = t.shape
        D = D1 - 1
        dids = _draft_ids(oracle, d, DTYPE_F32, B, D, V, dp, 63)
        src = rng.choice(np.array([1, 2, 3, 4], np.uint32), (B, D))
        am = np.array([[oracle.argmax_f32(t[b, i]) for i in range(D)] for b in range(B)], np.uint32)
        ng = src == 3
        dids = np.where(ng & (rng.random((B, D)) < 0.6), am, np.where(ng, rng.integers(0, V, (B, D)), dids)
                        ).astype(np.uint32)
        opts = {"sources": src, "model_mode": mm, "ngram_mode": nm, "delta_correction": dc}
        us = rng.random((B, D + 1)).astype(np.float32)
        res = sampler.mtp_verify(_to_dev(t, DTYPE_F32), _to_dev(d, DTYPE_F32), dids, tp, dp, uniforms=us,
                                 options=opts)
        torch.cuda.synchronize()
        g_ids, g_n, g_ac, g_fl = res.numpy()
        for b in range(B):
            if g_fl[b] & np.uint32(_abi.MTP_FLAG_NEAR_ACCEPT):
                continue
            ob = {k: (v[b] if isinstance(v, np.ndarray) else v) for k, v in opts.items()}
            want, ac = _mtp_expect(oracle, t[b], d[b], dids[b], tp[b:b + 1], dp[b:b + 1], us[b], ob, D)
            assert g_ids[b, : g_n[b]].tolist() == want and g_ac[b] == ac, (mm, nm, dc, b)
    log("mtp_verify_ex: all 12 mode combinations match")


LAWS = ["topk_topp", "topp_only", "minp_only", "unfiltered", "topk_option", "wide_bf16", "flat_wide",
        "topp_zero", "minp_above_one", "greedy_target"]


@pytest.mark.parametrize("law", LAWS)
def test_mtp_verify_production_target_law(sampler, oracle, law):
    """axs_mtp_verify_ex with AXS_MTP_TARGET_FILTERED: the acceptance test's
    p(d) is the runner's production law (compute_mtp_target_probs +
    extract_cpu_into + filtered_target_token_probability) in each of its
    cases — the top-k set (the target's top_k or the target_topk option),
    top-p only (the whole sorted row), min-p only (FullRows) and no filter
    (the softmax value) — against the oracle's mtp_accept_count with the
    oracle's mtp_target_prob."""
    import torch

    from ax_sampler import _abi

    V = 151936 if law in ("wide_bf16", "flat_wide") else 4099
    rng, t, d, tp, dp = _ex_case(70 + LAWS.index(law), B=12 if law != "flat_wide" else 4, V=V)
    if law == "topp_zero":
        # every p within 2^-24 of the maximum: a sorted law that cuts nothing
        # keeps ids the exact path lists only above that floor (such an MTP
        # sequence on a wider row is declined, AXS_MTP_FLAG_ERROR)
        t = (t * np.float32(0.3)).astype(np.float32)
        d = (d * np.float32(0.3)).astype(np.float32)
    if law == "flat_wide":
        # nearly flat rows: the 0.95 nucleus holds ~140k values (the sorted
        # walk runs ~35 chunks)
        t = (t * np.float32(0.05)).astype(np.float32)
        d = (t[:, :-1, :] + rng.standard_normal(d.shape, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    dtype = DTYPE_BF16 if law == "wide_bf16" else DTYPE_F32
    if dtype == DTYPE_BF16:
        t, d = f32_to_bf16_bits(t), f32_to_bf16_bits(d)
    opts = {"model_mode": _abi.MTP_MODEL_REJECTION, "target_law": _abi.MTP_TARGET_FILTERED}
    for pp in (tp, dp):
        if law in ("topp_only", "wide_bf16", "flat_wide"):
            pp["top_k"] = 0
        elif law == "minp_only":
            pp["top_k"], pp["top_p"], pp["has_min_p"], pp["min_p"] = 0, 1.0, 1, 0.05
        elif law == "unfiltered":
            pp["top_k"], pp["top_p"] = 0, 1.0
        elif law == "topk_option":
            pp["top_k"] = 0
        elif law == "topp_zero":
            # top_p < 1 selects the filtered law, but 0 cuts nothing there
            # (0 < top_p < 1 gates the cut): every p renormalised
            pp["top_k"], pp["top_p"] = 0, 0.0
        elif law == "minp_above_one":
            # min_p * max p above every p: nothing kept, p(d) = 0
            pp["top_k"], pp["top_p"], pp["has_min_p"], pp["min_p"] = 0, 1.0, 1, 1.5
    if law == "greedy_target":
        tp["temperature"][::2] = 0.0  # no target probabilities: greedy comparisons
    if law == "topk_option":
        opts["target_topk"] = 32
    B, D1, _ = t.shape
    D = D1 - 1
    dids = _draft_ids(oracle, d, dtype, B, D, V, dp, 63)
    us = rng.random((B, D + 1)).astype(np.float32)
    res = sampler.mtp_verify(_to_dev(t, dtype), _to_dev(d, dtype), dids, tp, dp, uniforms=us, options=opts)
    torch.cuda.synchronize()
    g_ids, g_n, g_ac, g_fl = res.numpy()
    near = 0
    tf = bf16_bits_to_f32(t) if dtype == DTYPE_BF16 else t
    df = bf16_bits_to_f32(d) if dtype == DTYPE_BF16 else d
    for b in range(B):
        ob = {k: (v[b] if isinstance(v, np.ndarray) else v) for k, v in opts.items()}
        want, ac = _mtp_expect(oracle, tf[b], df[b], dids[b], tp[b:b + 1], dp[b:b + 1], us[b], ob, D)
        assert not g_fl[b] & np.uint32(_abi.MTP_FLAG_ERROR), (law, b, "declined")
        if g_fl[b] & np.uint32(_abi.MTP_FLAG_NEAR_ACCEPT):
            near += 1
            continue
        got = g_ids[b, : g_n[b]].tolist()
        assert got == want and g_ac[b] == ac, (law, b, got, want, int(g_ac[b]), ac, hex(int(g_fl[b])))
    assert near <= boundary_allowance(B), near
    log(f"mtp production target law {law}: {B} sequences, near {near}, accepted {int(g_ac.sum())}")
