"""ctypes binding of the CPU oracle (oracle/libax_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
bench.py's cpu_baseline leg, as the parity checker — never as a product path.
The functions restate the reference's Rust sampler; see ax_oracle.c for the
file:line each one follows.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional, Sequence, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libax_oracle.so")

EXPLAIN_DTYPE = np.dtype(
    [
        ("token", "<u4"),
        ("path", "<u4"),
        ("drew", "<u4"),
        ("sorted", "<u4"),
        ("n_cand", "<u4"),
        ("n_nucleus", "<u4"),
        ("n_kept", "<u4"),
        ("boundary", "<u4"),
        ("m", "<f4"),
        ("total", "<f4"),
        ("cutoff", "<f4"),
        ("F", "<f4"),
        ("u", "<f4"),
        ("thr", "<f4"),
        ("logprob", "<f4"),
        ("pad0", "<f4"),
        ("margin_draw", "<f8"),
        ("margin_nucleus", "<f8"),
        ("margin_minp", "<f8"),
        ("margin_tie", "<f8"),
    ]
)
assert EXPLAIN_DTYPE.itemsize == 96

PATH_EMPTY, PATH_GREEDY, PATH_FALLBACK, PATH_FAST, PATH_FILTERED = range(5)
NONE_U32 = 0xFFFFFFFF

_lib = None


def build() -> None:
    """Compiles the oracle with its Makefile (gcc, -ffp-contract=off)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp, u32, u64, i32, f32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int, C.c_float
        L.axo_xorshift64_new.restype = u64
        L.axo_xorshift64_new.argtypes = [u64]
        L.axo_xorshift64_next_u64.restype = u64
        L.axo_xorshift64_next_u64.argtypes = [vp]
        L.axo_xorshift64_next_f32.restype = f32
        L.axo_xorshift64_next_f32.argtypes = [vp]
        L.axo_philox4x32_10.restype = None
        L.axo_philox4x32_10.argtypes = [vp, vp, vp]
        L.axo_philox_uniform.restype = f32
        L.axo_philox_uniform.argtypes = [u64, u32, u64, u32, u32]
        L.axo_argmax_f32.restype = u32
        L.axo_argmax_f32.argtypes = [vp, u32]
        L.axo_apply_processors.restype = i32
        L.axo_apply_processors.argtypes = [vp, u32, vp, vp, u32, vp, vp, vp, u32]
        L.axo_sample_row.restype = u32
        L.axo_sample_row.argtypes = [vp, u32, vp, vp, u32, vp, vp, vp, u32, vp, vp, vp, vp, u32]
        L.axo_sample_batch.restype = i32
        L.axo_sample_batch.argtypes = [
            vp, i32, u32, u32, u64, vp, vp, vp, vp, u64, vp, vp, vp, vp, vp, vp, vp, u32, i32,
        ]
        L.axo_token_distribution.restype = i32
        L.axo_token_distribution.argtypes = [vp, u32, vp, vp, vp, u32]
        L.axo_distribution_new.restype = i32
        L.axo_distribution_new.argtypes = [vp, vp, u32]
        L.axo_sample_from_distribution.restype = u32
        L.axo_sample_from_distribution.argtypes = [vp, vp, u32, f32]
        L.axo_sample_residual.restype = u32
        L.axo_sample_residual.argtypes = [vp, vp, u32, vp, vp, u32, f32]
        L.axo_distribution_prob.restype = f32
        L.axo_distribution_prob.argtypes = [vp, vp, u32, u32]
        L.axo_logprob_of.restype = f32
        L.axo_logprob_of.argtypes = [f32]
        L.axo_full_vocab_token_logprob.restype = f32
        L.axo_full_vocab_token_logprob.argtypes = [vp, u32, u32, f32]
        L.axo_top_logprobs.restype = None
        L.axo_top_logprobs.argtypes = [vp, u32, f32, u32, vp, vp]
        L.axo_mtp_target_prob.restype = f32
        L.axo_mtp_target_prob.argtypes = [vp, u32, f32, f32, u32, i32, f32, u32, u32]
        L.axo_soft_close_in_top_k.restype = C.c_int
        L.axo_soft_close_in_top_k.argtypes = [vp, u32, u32, u32]
        L.axo_mtp_accept_count.restype = u32
        L.axo_mtp_accept_count.argtypes = [
            u32, vp, vp, u32, vp, vp, vp, u32, vp, u32, vp, vp, vp, vp, u32, vp, vp, vp, u32,
            f32, f32, i32, i32, vp, vp,
        ]
        L.axo_mtp_verify_seq.restype = u32
        L.axo_mtp_verify_seq.argtypes = [vp, vp, u32, u32, vp, vp, vp, vp, vp, vp, vp]
        L.axo_mtp_verify_batch.restype = i32
        L.axo_mtp_verify_batch.argtypes = [
            vp, vp, i32, u32, u32, u32, u64, vp, vp, vp, vp, vp, vp, vp, vp, i32,
        ]
        L.axo_core_argmax_logprob.restype = i32
        L.axo_core_argmax_logprob.argtypes = [vp, u32, vp, vp, u32, vp, vp]
        L.axo_bf16_to_f32.restype = None
        L.axo_bf16_to_f32.argtypes = [vp, vp, u64]
        _lib = L
    return _lib


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


def _u32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.uint32))


class Xorshift64:
    """Xorshift64 (crates/ax-engine-mlx/src/sampling.rs:15-37) on the C side."""

    def __init__(self, seed: int):
        self.state = np.array([lib().axo_xorshift64_new(seed & 0xFFFFFFFFFFFFFFFF)], dtype=np.uint64)

    @property
    def ptr(self):
        return self.state.ctypes.data

    def next_u64(self) -> int:
        return int(lib().axo_xorshift64_next_u64(self.ptr))

    def next_f32(self) -> float:
        return float(lib().axo_xorshift64_next_f32(self.ptr))

    @property
    def value(self) -> int:
        return int(self.state[0])


def philox4x32_10(ctr: Sequence[int], key: Sequence[int]) -> Tuple[int, int, int, int]:
    c = _u32(ctr)
    k = _u32(key)
    o = np.zeros(4, dtype=np.uint32)
    lib().axo_philox4x32_10(c.ctypes.data, k.ctypes.data, o.ctypes.data)
    return tuple(int(v) for v in o)


def philox_uniform(seed: int, row: int, step: int, purpose: int = 0, word: int = 0) -> float:
    return float(lib().axo_philox_uniform(seed, row, step, purpose, word))


def argmax_f32(logits) -> int:
    a = _f32(logits)
    return int(lib().axo_argmax_f32(a.ctypes.data, a.size))


def sample_row(
    logits,
    params: np.ndarray,
    history=None,
    *,
    u: Optional[float] = None,
    rng: Optional[Xorshift64] = None,
    mask_words=None,
    bias_ids=None,
    bias_vals=None,
    kept_cap: int = 0,
):
    """``sample_categorical_into`` for one row.  ``params`` is a 1-element
    PARAMS_DTYPE array.  Returns (token, explain record, kept ids)."""
    a = _f32(logits)
    h = _u32([] if history is None else history)
    m = None if mask_words is None else _u32(mask_words)
    bi = None if bias_ids is None else _u32(bias_ids)
    bv = None if bias_vals is None else _f32(bias_vals)
    nb = 0 if bi is None else bi.size
    ex = np.zeros(1, dtype=EXPLAIN_DTYPE)
    uu = None if u is None else np.array([u], dtype=np.float32)
    kept = np.zeros(max(kept_cap, 1), dtype=np.uint32)
    tok = lib().axo_sample_row(
        a.ctypes.data, a.size, params.ctypes.data, h.ctypes.data, h.size, _p(m), _p(bi), _p(bv),
        nb, _p(uu), None if rng is None else rng.ptr, ex.ctypes.data,
        kept.ctypes.data if kept_cap else None, kept_cap,
    )
    n = int(ex[0]["n_kept"])
    return int(tok), ex[0], kept[: min(n, kept_cap)]


def sample_batch(
    logits: np.ndarray,
    dtype: int,
    B: int,
    V: int,
    stride: int,
    params: np.ndarray,
    hist: Optional[np.ndarray] = None,
    hist_off: Optional[np.ndarray] = None,
    mask: Optional[np.ndarray] = None,
    mask_stride: int = 0,
    bias_ids: Optional[np.ndarray] = None,
    bias_vals: Optional[np.ndarray] = None,
    bias_off: Optional[np.ndarray] = None,
    uniforms: Optional[np.ndarray] = None,
    kept_cap: int = 0,
    nthreads: int = 1,
    explain: bool = True,
):
    out = np.zeros(B, dtype=np.uint32)
    ex = np.zeros(B, dtype=EXPLAIN_DTYPE) if explain else None
    kept = np.zeros((B, kept_cap), dtype=np.uint32) if kept_cap else None
    rc = lib().axo_sample_batch(
        logits.ctypes.data, dtype, B, V, stride, params.ctypes.data, _p(hist), _p(hist_off),
        _p(mask), mask_stride, _p(bias_ids), _p(bias_vals), _p(bias_off), _p(uniforms),
        out.ctypes.data, _p(ex), _p(kept), kept_cap, nthreads,
    )
    if rc != 0:
        raise RuntimeError("oracle sample_batch failed")
    return out, ex, kept


def token_distribution(logits, params: np.ndarray, cap: Optional[int] = None):
    a = _f32(logits)
    cap = a.size if cap is None else cap
    ids = np.zeros(max(cap, 1), dtype=np.uint32)
    probs = np.zeros(max(cap, 1), dtype=np.float32)
    n = lib().axo_token_distribution(a.ctypes.data, a.size, params.ctypes.data, ids.ctypes.data,
                                     probs.ctypes.data, cap)
    if n < 0:
        return None
    return ids[:n].copy(), probs[:n].copy()


def distribution_new(entries):
    """TokenDistribution::new; returns list of (id, prob) or None."""
    ids = _u32([e[0] for e in entries] or [0])
    probs = _f32([e[1] for e in entries] or [0.0])
    n = lib().axo_distribution_new(ids.ctypes.data, probs.ctypes.data, len(entries))
    if n < 0:
        return None
    return [(int(ids[i]), float(probs[i])) for i in range(n)]


def sample_from_distribution(ids, probs, u: float) -> Optional[int]:
    i = _u32(ids)
    p = _f32(probs)
    t = lib().axo_sample_from_distribution(i.ctypes.data, p.ctypes.data, i.size, u)
    return None if t == NONE_U32 else int(t)


def sample_residual(t_ids, t_probs, d_ids, d_probs, u: float) -> Optional[int]:
    ti, tp, di, dp = _u32(t_ids), _f32(t_probs), _u32(d_ids), _f32(d_probs)
    t = lib().axo_sample_residual(ti.ctypes.data, tp.ctypes.data, ti.size, di.ctypes.data,
                                  dp.ctypes.data, di.size, u)
    return None if t == NONE_U32 else int(t)


def distribution_prob(ids, probs, token: int) -> float:
    i, p = _u32(ids), _f32(probs)
    return float(lib().axo_distribution_prob(i.ctypes.data, p.ctypes.data, i.size, token))


def logprob_of(prob: float) -> float:
    return float(lib().axo_logprob_of(prob))


def full_vocab_token_logprob(logits, token: int, temperature: float) -> float:
    a = _f32(logits)
    return float(lib().axo_full_vocab_token_logprob(a.ctypes.data, a.size, token, temperature))


def top_logprobs(logits, temperature: float, n: int):
    """(ids uint32[n], logprobs f32[n]): the n largest full-softmax
    probabilities, ties to the lower id, with full_vocab_token_logprob."""
    a = _f32(logits)
    ids = np.zeros(max(n, 1), np.uint32)
    lp = np.zeros(max(n, 1), np.float32)
    lib().axo_top_logprobs(a.ctypes.data, a.size, temperature, n, ids.ctypes.data, lp.ctypes.data)
    return ids[:n], lp[:n]


def mtp_target_prob(logits, token: int, temperature: float, top_p: float = 1.0, top_k: int = 0,
                    min_p: Optional[float] = None, topk_opt: int = 0) -> float:
    """The production law's target probability of a draft token
    (compute_mtp_target_probs + extract_cpu_into +
    filtered_target_token_probability, crates/ax-engine-mlx/src/runner/mod.rs:
    11836-12159; see axo_mtp_target_prob).  NaN when T <= 0."""
    a = _f32(logits)
    return float(lib().axo_mtp_target_prob(a.ctypes.data, a.size, temperature, top_p, top_k,
                                           0 if min_p is None else 1, 0.0 if min_p is None else min_p,
                                           topk_opt, token))


MTP_DRAFT_SAMPLED, MTP_DRAFT_STOCHASTIC = 0, 1


def mtp_draft(logits, temperature: float, mode: int, u: float):
    """The draft side of one MTP depth on one draft row: (token, ln q, explain
    record of the draw or None).

    mode MTP_DRAFT_SAMPLED, mtp_draft_tokens_sampled
    (crates/ax-engine-mlx/src/mtp.rs:1454-1552): the token is the argmax
    (lazy_argmax_logits, mtp.rs:192-196) and ln q its full-softmax log-prob at
    the draft temperature (gpu_draft_log_prob_lazy, mtp.rs:203-220).

    mode MTP_DRAFT_STOCHASTIC, mtp_draft_tokens_stochastic (mtp.rs:1554-1640):
    for T > 0 a categorical draw from softmax(logits / T) (lazy_random_sample,
    mtp.rs:228-233), ln q at T; for T <= 0 the argmax, ln q at T = 1
    (mtp.rs:1614-1623).  The reference draws with MLX's own RNG (not
    reproducible); the draw here is sample_categorical_into with no filters
    (crates/ax-engine-mlx/src/sampling.rs:204-271, the index-order law) on the
    supplied uniform u.  ln q is full_vocab_token_logprob
    (crates/ax-engine-mlx/src/sampling.rs:761-787), the CPU statement of
    gpu_draft_log_prob_lazy's value."""
    a = _f32(logits)
    T = float(np.float32(temperature))
    ex = None
    if mode == MTP_DRAFT_SAMPLED or T <= 0.0:
        tok = argmax_f32(a)
    else:
        p = np.zeros(1, dtype=_params_dtype())
        p["temperature"] = T
        p["top_p"] = 1.0
        p["repetition_penalty"] = 1.0
        p["repetition_context_size"] = NONE_U32
        p["ngram_window"] = 128
        tok, ex, _ = sample_row(a, p, u=u)
    lp_t = T if (mode == MTP_DRAFT_SAMPLED or T > 0.0) else 1.0
    return tok, full_vocab_token_logprob(a, tok, lp_t), ex


def _params_dtype():
    from ax_sampler.params import PARAMS_DTYPE

    return PARAMS_DTYPE


def soft_close_in_top_k(logits, target: int, rank: int) -> bool:
    a = _f32(logits)
    if a.size == 0:
        return False
    return bool(lib().axo_soft_close_in_top_k(a.ctypes.data, a.size, target, rank))


def _csr(dists):
    if dists is None:
        return None, None, None, 0
    ids = np.concatenate([_u32(d[0]) for d in dists]) if dists else np.zeros(0, np.uint32)
    probs = np.concatenate([_f32(d[1]) for d in dists]) if dists else np.zeros(0, np.float32)
    off = np.zeros(len(dists) + 1, dtype=np.int64)
    for i, d in enumerate(dists):
        off[i + 1] = off[i] + len(d[0])
    return _u32(ids if ids.size else [0]), _f32(probs if probs.size else [0]), off, len(dists)


SRC_NONE, SRC_MTP, SRC_GEMMA, SRC_NGRAM, SRC_HYBRID = range(5)
MODEL_GREEDY, MODEL_REJECTION = 0, 1
NGRAM_CONFIDENCE, NGRAM_DELTA, NGRAM_GREEDY = 0, 1, 2


def mtp_accept_count(
    pending, pending_log_probs, draft_dists, sources, target_probs, target_dists, predicted,
    rng: Optional[Xorshift64], draft_temperature, target_temperature, model_mode, ngram_mode,
    uniforms=None,
):
    """mtp_accept_count (crates/ax-engine-mlx/src/runner/mod.rs:12333-12462).
    Returns (accept_count, all_accepted, correction or None)."""
    pend = _u32(pending)
    lps = _f32(pending_log_probs if len(pending_log_probs) else [0.0])
    di, dp, doff, nd = _csr(draft_dists)
    src = _u32(sources if len(sources) else [0])
    tp = None if target_probs is None else _f32(target_probs)
    ti, tpp, toff, nt = _csr(target_dists)
    pred = _u32(predicted)
    un = None if uniforms is None else _f32(uniforms)
    allacc = np.zeros(1, dtype=np.uint32)
    corr = np.zeros(1, dtype=np.uint32)
    ac = lib().axo_mtp_accept_count(
        pend.size, pend.ctypes.data, lps.ctypes.data, len(pending_log_probs), _p(di), _p(dp),
        _p(doff), nd, src.ctypes.data, len(sources), _p(tp), _p(ti), _p(tpp), _p(toff), nt,
        pred.ctypes.data, None if rng is None else rng.ptr, _p(un), 0 if un is None else un.size,
        draft_temperature, target_temperature, model_mode, ngram_mode, allacc.ctypes.data,
        corr.ctypes.data,
    )
    c = int(corr[0])
    return int(ac), bool(allacc[0]), (None if c == NONE_U32 else c)


def mtp_verify_batch(target, draft, dtype, B, depth, V, stride, draft_ids, tparams, dparams,
                     uniforms=None, nthreads=1):
    out_ids = np.zeros((B, depth + 1), dtype=np.uint32)
    out_count = np.zeros(B, dtype=np.uint32)
    acc = np.zeros(B, dtype=np.uint32)
    flags = np.zeros(B, dtype=np.uint32)
    lib().axo_mtp_verify_batch(
        target.ctypes.data, draft.ctypes.data, dtype, B, depth, V, stride, draft_ids.ctypes.data,
        tparams.ctypes.data, dparams.ctypes.data, _p(uniforms), out_ids.ctypes.data,
        out_count.ctypes.data, acc.ctypes.data, flags.ctypes.data, nthreads,
    )
    return out_ids, out_count, acc, flags


def core_argmax_logprob(logits, params: np.ndarray, recent=()):
    a = _f32(logits)
    r = _u32(list(recent) if len(recent) else [0])
    tok = np.zeros(1, dtype=np.uint32)
    lp = np.zeros(1, dtype=np.float32)
    ok = lib().axo_core_argmax_logprob(a.ctypes.data, a.size, params.ctypes.data, r.ctypes.data,
                                       len(recent), tok.ctypes.data, lp.ctypes.data)
    if not ok:
        return None
    return int(tok[0]), float(lp[0])


def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a.view(np.uint16))
    out = np.empty(a.shape, dtype=np.float32)
    lib().axo_bf16_to_f32(a.ctypes.data, out.ctypes.data, a.size)
    return out
