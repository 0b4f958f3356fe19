"""GPU parity of the top-N log-probabilities (axs_top_logprobs) against the
oracle's axo_top_logprobs, through the C ABI: ids bit-exact, values equal to
the oracle's full_vocab_token_logprob (crates/ax-engine-mlx/src/sampling.rs:
761-787) within 1e-5 (the device's ln is rounded once from double; glibc's
logf may differ by one ulp).

Rows in f32 and bf16 (bf16 repeats values: ties to the lower id), several
temperatures including T <= 0, n from 1 to AXS_TOP_LOGPROBS_MAX, both
launch shapes (one row; 2..63 listed rows; 64 or more in place), a row of
all-equal logits (every id ties), an all -inf row and a tiny vocabulary."""
import numpy as np
import pytest

from ax_sampler.synth import f32_to_bf16_bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sampler():
    from ax_sampler import HipSampler

    s = HipSampler(0, max_batch=256, max_vocab=262144)
    yield s
    s.close()


def _run(sampler, oracle, x, bf16, temps, n):
    import torch

    B, V = x.shape
    if bf16:
        bits = f32_to_bf16_bits(x)
        dev = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to("cuda:0")
        xf = (bits.astype(np.uint32) << 16).view(np.float32)
    else:
        dev = torch.from_numpy(x).to("cuda:0")
        xf = x
    ids, lp = sampler.top_logprobs(dev, temps, n)
    torch.cuda.synchronize()
    ids = ids.cpu().numpy().view(np.uint32)
    lp = lp.cpu().numpy()
    for r in range(B):
        wi, wl = oracle.top_logprobs(xf[r], float(temps[r]), n)
        assert ids[r].tolist() == wi.tolist(), (r, ids[r][:8].tolist(), wi[:8].tolist())
        fin = np.isfinite(wl)
        assert np.array_equal(np.isneginf(lp[r]), np.isneginf(wl)), r
        np.testing.assert_allclose(lp[r][fin], wl[fin], rtol=1e-5, atol=2e-6)


@pytest.mark.parametrize("B", [1, 17, 96])
@pytest.mark.parametrize("bf16", [False, True])
def test_top_logprobs_match_oracle(sampler, oracle, B, bf16):
    rng = np.random.default_rng([B, int(bf16)])
    V = 151936
    x = (rng.standard_normal((B, V)) * 3.0).astype(np.float32)
    temps = np.array([[0.7, 1.0, 1.6, 0.0][r % 4] for r in range(B)], np.float32)
    for n in (1, 5, 20, 64):
        _run(sampler, oracle, x, bf16, temps, n)


def test_top_logprobs_edge_rows(sampler, oracle):
    V = 4099
    x = np.random.default_rng(5).standard_normal((6, V)).astype(np.float32)
    x[0, :] = 2.0            # every id ties
    x[1, :] = -np.inf        # no finite maximum
    x[2, 17] = 50.0          # one dominant id, the rest underflow to 0 mass
    x[3, ::3] = np.nan
    temps = np.array([1.0, 1.0, 0.05, 0.9, 1e-30, -1.0], np.float32)
    _run(sampler, oracle, x, False, temps, 20)
    _run(sampler, oracle, x[:, :7].copy(), False, temps, 12)  # n > V
