"""GPU parity of the MTP draft side (axs_mtp_draft) against the CPU oracle's
mtp_draft, through the C ABI.

Per draft row the token must equal the oracle's on every row (argmax for the
sampled mode and for T <= 0; the index-order categorical draw on the same
uniform for the stochastic mode, boundary rows included) and ln q must be
full_vocab_token_logprob of it within 1e-5 (the device reproduces that
function's sequential sum).  Rows mix temperatures 0.6 / 1.0 / 1.4 / 0 / -1,
a row of NaN and a row with -inf logits,
bf16 and f32 logits, supplied uniforms (with 0 and 1) and Philox draws, and
the drafted rows then feed axs_mtp_verify_ex as pending_log_probs.
"""
import numpy as np
import pytest

from ax_sampler.synth import DTYPE_BF16, DTYPE_F32, _params

from gpu_common import log

pytestmark = pytest.mark.gpu

TEMPS = [0.6, 1.0, 1.4, 0.0, -1.0, 0.6, 1.0, 0.3]


@pytest.fixture(scope="module")
def sampler():
    from ax_sampler import HipSampler

    s = HipSampler(0, max_batch=128, max_vocab=151936)
    yield s
    s.close()


def _rows(B, V, dtype, seed):
    rng = np.random.default_rng([seed, 77])
    x = (rng.standard_normal((B, V)) * 3.0).astype(np.float32)
    x[2] = np.nan          # no finite logit: argmax 0, ln q -30
    x[3, ::2] = -np.inf    # zero-probability ids
    if dtype == DTYPE_BF16:
        bits = x.view(np.uint32)
        bits = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000  # round to bf16
        x = bits.astype(np.uint32).view(np.float32)
    p = _params(B, seed=1000 + seed, step=9)
    p["temperature"] = [TEMPS[r % len(TEMPS)] for r in range(B)]
    p["seed"] = 31 + np.arange(B, dtype=np.uint64) * 7
    return x, p


def _device(x, dtype):
    import torch

    if dtype == DTYPE_BF16:
        return torch.from_numpy((x.view(np.uint32) >> 16).astype(np.uint16).view(np.int16)).view(
            torch.bfloat16).to("cuda:0")
    return torch.from_numpy(x).to("cuda:0")


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("dtype,V,B", [(DTYPE_BF16, 151936, 40), (DTYPE_F32, 50021, 24)])
@pytest.mark.parametrize("uniform_src", ["supplied", "philox"])
def test_mtp_draft_matches_oracle(sampler, oracle, mode, dtype, V, B, uniform_src):
    import torch

    log(f"mtp_draft mode={mode} dtype={dtype} V={V} B={B} uniforms={uniform_src}")
    x, p = _rows(B, V, dtype, seed=3 + mode)
    rng = np.random.default_rng(5)
    if uniform_src == "supplied":
        us = rng.random(B).astype(np.float32)
        us[0], us[1] = np.float32(0.0), np.float32(1.0)
    else:
        us = None
    ids, lnq = sampler.mtp_draft(_device(x, dtype), p, mode, uniforms=us)
    torch.cuda.synchronize()
    got_ids = ids.cpu().numpy().view(np.uint32)
    got_lnq = lnq.cpu().numpy()
    n_draw = 0
    for r in range(B):
        T = float(p[r]["temperature"])
        u = float(us[r]) if us is not None else oracle.philox_uniform(int(p[r]["seed"]), r, int(p[r]["step"]))
        tok, want_lnq, ex = oracle.mtp_draft(x[r], T, mode, u)
        n_draw += ex is not None
        assert got_ids[r] == tok, (r, T, got_ids[r], tok)
        assert abs(float(got_lnq[r]) - want_lnq) <= 1e-5 * max(1.0, abs(want_lnq)), (r, got_lnq[r], want_lnq)
    log(f"mtp_draft: {B} rows, {n_draw} categorical draws")


def test_drafts_feed_the_verify_step(sampler, oracle):
    """Draft every position with axs_mtp_draft (stochastic, the draft's own
    temperature), then verify with the drafted ln q as pending_log_probs: the
    outcome equals the oracle's mtp_accept_count + tail on the same draft ids
    and log-probs."""
    import torch

    from ax_sampler import _abi
    from test_gpu_mtp import _ex_case, _mtp_expect, _to_dev

    rng, t, d, tp, dp = _ex_case(11, B=12)
    B, D1, V = t.shape
    D = D1 - 1
    drow_p = np.repeat(dp, D)
    ud = rng.random(B * D).astype(np.float32)
    ids, lnq = sampler.mtp_draft(_to_dev(d.reshape(B * D, V), DTYPE_F32), drow_p, _abi.MTP_DRAFT_STOCHASTIC,
                                 uniforms=ud)
    torch.cuda.synchronize()
    dids = ids.cpu().numpy().view(np.uint32).reshape(B, D)
    lq = lnq.cpu().numpy().reshape(B, D)
    for r in range(B * D):
        tok, want, _ = oracle.mtp_draft(d.reshape(B * D, V)[r], float(drow_p[r]["temperature"]),
                                        _abi.MTP_DRAFT_STOCHASTIC, float(ud[r]))
        assert dids.flat[r] == tok and abs(float(lq.flat[r]) - want) <= 1e-5 * max(1.0, abs(want)), r
    opts = {"model_mode": _abi.MTP_MODEL_REJECTION, "pending_log_probs": lq}
    us = rng.random((B, D + 1)).astype(np.float32)
    res = sampler.mtp_verify(_to_dev(t, DTYPE_F32), _to_dev(d, DTYPE_F32), dids, tp, dp, uniforms=us,
                             options=opts)
    torch.cuda.synchronize()
    g_ids, g_n, g_ac, g_fl = res.numpy()
    near = 0
    for b in range(B):
        ob = {k: (v[b] if isinstance(v, np.ndarray) else v) for k, v in opts.items()}
        want, ac = _mtp_expect(oracle, t[b], d[b], dids[b], tp[b:b + 1], dp[b:b + 1], us[b], ob, D)
        if g_fl[b] & np.uint32(_abi.MTP_FLAG_NEAR_ACCEPT):
            near += 1
            continue
        assert g_ids[b, : g_n[b]].tolist() == want and g_ac[b] == ac, (b, g_ids[b, : g_n[b]].tolist(), want)
    assert near <= 1, near
    log(f"draft -> verify: {B} sequences, near {near}, accepted {int(g_ac.sum())}")
