"""GPU parity of the think soft-close rank probe (axs_soft_close_probe)
against the oracle's restatement of think_soft_close_in_top_k
(crates/ax-engine-mlx/src/ngram_accel.rs:1609-1640), through the C ABI.

Rows in f32 and bf16 at V = 151,936 and small vocabularies; targets at the
row maximum, inside and just outside the top ranks, at tied values (the
lower id keeps its place), beyond the vocabulary; rank 0, 1, 3 (the
reference's THINK_SOFT_CLOSE_PROBE_RANK) and rank >= V; rows holding NaN
(+ and -) or both signed zeros, which the device replays literally.
Every row's answer must equal the oracle's."""
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


def _rows(rng, B, V, quantise):
    x = (rng.standard_normal((B, V)) * 3.0).astype(np.float32)
    if quantise:  # repeated values: ties at the cut
        x = np.round(x * 4.0).astype(np.float32) / np.float32(4.0)
    return x


def _targets(rng, x, ranks):
    B, V = x.shape
    t = np.zeros(B, np.uint32)
    for r in range(B):
        order = np.lexsort((np.arange(V), -x[r]))  # (value desc, id asc)
        k = int(ranks[r])
        pick = r % 6
        if pick == 0:
            t[r] = order[0]
        elif pick == 1:
            t[r] = order[max(min(k, V) - 1, 0)]  # the last one in
        elif pick == 2:
            t[r] = order[min(k, V - 1)]  # the first one out
        elif pick == 3:
            t[r] = V + 5  # beyond the vocabulary
        else:
            t[r] = int(rng.integers(0, V))
    return t


def _check(sampler, oracle, x, dtype_bf16, t, ranks):
    import torch

    B, V = x.shape
    if dtype_bf16:
        bits = f32_to_bf16_bits(x)
        dev = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to("cuda:0")
        xf = (bits.astype(np.uint32) << 16).view(np.float32)
    else:
        dev = torch.from_numpy(x).to("cuda:0")
        xf = x
    out = sampler.soft_close_probe(dev, t, ranks).cpu().numpy().view(np.uint32)
    torch.cuda.synchronize()
    want = np.array([oracle.soft_close_in_top_k(xf[r], int(t[r]), int(ranks[r])) for r in range(B)], np.uint32)
    bad = np.nonzero(out != want)[0]
    assert bad.size == 0, (bad[:10].tolist(), out[bad[:10]].tolist(), want[bad[:10]].tolist())
    return int(want.sum())


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("V,quantise", [(151936, False), (151936, True), (4099, True), (7, True)])
def test_probe_matches_oracle(sampler, oracle, bf16, V, quantise):
    rng = np.random.default_rng([V, int(bf16), int(quantise)])
    B = 48
    x = _rows(rng, B, V, quantise)
    ranks = np.array([[0, 1, 3, 3, 5, V + 2][r % 6] for r in range(B)], np.uint32)
    t = _targets(rng, x, ranks)
    hits = _check(sampler, oracle, x, bf16, t, ranks)
    print(f"probe V={V} bf16={bf16} quantised={quantise}: {hits} of {B} rows hit")


def test_probe_nan_and_signed_zero_rows(sampler, oracle):
    rng = np.random.default_rng(77)
    B, V = 24, 4096
    x = _rows(rng, B, V, True)
    neg_nan = np.array([0xFFC00000], np.uint32).view(np.float32)[0]
    for r in range(B):
        if r % 3 == 0:
            x[r, rng.integers(0, V, 3)] = np.nan
        elif r % 3 == 1:
            x[r, int(rng.integers(0, 4))] = neg_nan  # early: inside the first ranks
        else:
            x[r, rng.integers(0, V, 50)] = 0.0
            x[r, rng.integers(0, V, 50)] = -0.0
            x[r, :3] = np.array([0.0, -0.0, -0.0], np.float32)
    x[2, :] = 0.0
    x[2, 1::2] = -0.0  # all zeros
    ranks = np.array([[1, 3, 3, 8][r % 4] for r in range(B)], np.uint32)
    t = _targets(rng, x, ranks)
    t[2] = 1
    _check(sampler, oracle, x, False, t, ranks)
