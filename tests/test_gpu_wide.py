"""GPU parity of the one-workgroup-per-row shape (k_row: batches of 2 rows or
more, V <= 262,144) against the CPU oracle, through the C ABI.

Same bar as test_gpu_parity: token ids bit-exact on every row (boundary rows
included, and counted), kept sets exact, logprobs within 1e-5 relative.
Covers the north-star workload at full size (B=256, V=262,144 bf16) with
supplied and Philox uniforms, every row law with masks, bias lists (duplicate
and out-of-vocabulary ids) and n-gram bans, unaligned and tiny vocabularies,
and the fallback for repetition windows with more distinct ids than the LDS
hash holds.
"""
import numpy as np
import pytest

from ax_sampler.synth import DTYPE_BF16, DTYPE_F32, make_c3, make_c4, make_mixed

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


def test_c3_full_size(sampler, oracle):
    w = make_c3(3)
    us = _uniforms(w.B, 303)
    gpu = run_gpu(sampler, w, us, kept_cap=64)
    cpu = run_oracle(oracle, w, us, kept_cap=64)
    log(f"C3 full (256 rows, k_row): {compare(w, gpu, cpu, 'C3-full')}")
    gpu = run_gpu(sampler, w, None, kept_cap=64)
    ph = np.array([oracle.philox_uniform(int(w.params[r]['seed']), r, int(w.params[r]['step']))
                   for r in range(w.B)], dtype=np.float32)
    cpu = run_oracle(oracle, w, ph, kept_cap=64)
    log(f"C3 full philox: {compare(w, gpu, cpu, 'C3-full-philox')}")


def test_c4_shape_wide(sampler, oracle):
    w = make_c4(4, B=256)
    us = _uniforms(w.B, 404)
    gpu = run_gpu(sampler, w, us, kept_cap=64)
    cpu = run_oracle(oracle, w, us, kept_cap=64)
    log(f"C4 shape, 256 rows: {compare(w, gpu, cpu, 'C4-wide')}")
    allowed = w.extra["allowed"]
    assert all(allowed[r, gpu[0][r]] for r in range(w.B)), "a masked id was emitted"


@pytest.mark.parametrize("dtype,V,mask,bias,ngram", [
    (DTYPE_BF16, 262144, False, False, False),
    (DTYPE_BF16, 151936, True, True, True),
    (DTYPE_F32, 151936, False, True, False),
    (DTYPE_F32, 4099, True, True, True),      # unaligned rows: element loads
    (DTYPE_BF16, 4100, False, True, True),    # length not a multiple of the vector
    (DTYPE_BF16, 8, False, True, False),      # tiny vocabulary
    (DTYPE_F32, 1, False, False, False),
])
def test_mixed_laws_wide(sampler, oracle, dtype, V, mask, bias, ngram):
    w = make_mixed(11 + V % 97, 256, V, dtype, hist_len=768, mask=mask, bias=bias, ngram=ngram)
    us = _uniforms(w.B, 1000 + V)
    us[7] = 1.0  # the reference's generator can return exactly 1.0
    gpu = run_gpu(sampler, w, us, kept_cap=32)
    cpu = run_oracle(oracle, w, us, kept_cap=32)
    log(f"mixed dtype={dtype} V={V} mask={mask} bias={bias} ngram={ngram}: "
        f"{compare(w, gpu, cpu, f'mixed-{V}')}")
    if mask:
        allowed = w.extra["allowed"]
        for r in range(w.B):
            if allowed[r].any() and cpu[1][r]["drew"]:
                assert allowed[r, gpu[0][r]], f"row {r}: masked id {gpu[0][r]} emitted"


def test_greedy_logprob_wide(sampler, oracle):
    w = make_c3(5, B=256, V=65536)
    w.params["temperature"] = 0.0
    gpu = run_gpu(sampler, w, None, kept_cap=4)
    cpu = run_oracle(oracle, w, None, kept_cap=4)
    log(f"greedy wide: {compare(w, gpu, cpu, 'greedy-wide')}")


def test_hash_overflow_fallback(sampler, oracle):
    """Rows whose repetition windows hold more distinct ids than the LDS hash
    (4,096 slots) resolve their special ids from HBM; the result is the same."""
    w = make_c3(6, B=256, V=65536)
    rng = np.random.default_rng(66)
    lens = np.full(w.B, 64, dtype=np.int64)
    lens[:3] = 5000                      # three rows with ~5,000 distinct ids
    hs = [rng.permutation(w.V)[:n].astype(np.uint32) if n > 64 else
          rng.integers(0, w.V, n).astype(np.uint32) for n in lens]
    hs[1][:100] = hs[1][100]             # and repeats
    w.hist = np.concatenate(hs)
    w.hist_off = np.zeros(w.B + 1, dtype=np.int64)
    w.hist_off[1:] = np.cumsum(lens)
    us = _uniforms(w.B, 606)
    gpu = run_gpu(sampler, w, us, kept_cap=64)
    cpu = run_oracle(oracle, w, us, kept_cap=64)
    log(f"hash overflow: {compare(w, gpu, cpu, 'hash-overflow')}")


@pytest.mark.parametrize("B", [256, 16])
def test_min_p_above_one(sampler, oracle, B):
    """min_p > 1 leaves no survivor (the maximum has p = 1): argmax, no draw
    (sampling.rs:290-293), for every draw law, on the one-row-per-workgroup
    shape (B = 256: exact path in place; B = 16: listed)."""
    w = make_c3(8, B=B, V=65536)
    rng = np.random.default_rng(88)
    w.params["min_p"] = rng.choice(np.array([1.5, 0.05, 2.0], np.float32), B)
    w.params["top_k"] = rng.choice(np.array([0, 40], np.uint32), B)
    w.params["top_p"] = rng.choice(np.array([1.0, 0.9], np.float32), B)
    us = _uniforms(w.B, 808)
    gpu = run_gpu(sampler, w, us, kept_cap=8)
    cpu = run_oracle(oracle, w, us, kept_cap=8)
    log(f"min_p > 1, B={B}: {compare(w, gpu, cpu, f'minp-above-one-{B}')}")
    big = w.params["min_p"] > 1.0
    assert np.array_equal(gpu[0][big], cpu[0][big])
    assert not np.any(gpu[2][big] & np.uint32(0x4)), "a row without survivors consumed a uniform"


@pytest.mark.parametrize("B", [256, 16])
def test_capture_pool_overflow(sampler, oracle, B):
    """A repetition penalty below 1 can raise a logit, so every vector is
    looked at and every special element captured; windows of 3,000 distinct
    ids overflow the 2,048-entry capture pool (not the 4,096-slot hash), and
    those rows resolve their special ids from HBM.  Same result as the
    oracle."""
    w = make_c3(9, B=B, V=65536)
    rng = np.random.default_rng(99)
    lens = np.full(w.B, 64, dtype=np.int64)
    lens[: min(4, B)] = 3000
    w.hist = np.concatenate([rng.permutation(w.V)[:n].astype(np.uint32) if n > 64 else
                             rng.integers(0, w.V, n).astype(np.uint32) for n in lens])
    w.hist_off = np.zeros(w.B + 1, dtype=np.int64)
    w.hist_off[1:] = np.cumsum(lens)
    w.params["repetition_penalty"] = np.where(np.arange(w.B) % 2 == 0, 0.9, 1.2).astype(np.float32)
    w.params["repetition_context_size"] = 0xFFFFFFFF
    us = _uniforms(w.B, 909)
    gpu = run_gpu(sampler, w, us, kept_cap=16)
    cpu = run_oracle(oracle, w, us, kept_cap=16)
    log(f"capture pool overflow, B={B}: {compare(w, gpu, cpu, f'capture-overflow-{B}')}")


def test_bias_capacity_is_flagged_not_wrong(sampler, oracle):
    """A row with more bias entries than the kernel holds (1024 per row from
    2 rows on) comes back as token 0 with AXS_FLAG_ERROR | AXS_FLAG_CAPACITY;
    the other rows are sampled as usual, and the host entry point refuses
    the batch with AXS_E_CAPACITY."""
    from ax_sampler import _abi
    from ax_sampler.synth import make_mixed

    w = make_mixed(71, 4, 8192, DTYPE_F32, hist_len=64, mask=False, bias=True, ngram=False)
    rs = np.random.default_rng(72)
    rows = [(w.bias_ids[w.bias_off[r]:w.bias_off[r + 1]], w.bias_vals[w.bias_off[r]:w.bias_off[r + 1]])
            for r in range(w.B)]
    rows[1] = (rs.integers(0, 8192, 1025).astype(np.uint32), rs.uniform(-1, 1, 1025).astype(np.float32))
    us = _uniforms(w.B, 73)
    from gpu_common import hist_rows, to_device
    import torch

    res = sampler.sample(to_device(w), w.params, history=hist_rows(w), bias=rows, uniforms=us, logprobs=True)
    torch.cuda.synchronize()
    tid, _, fl, _, _ = res.numpy()
    assert fl[1] & np.uint32(_abi.FLAG_ERROR) and fl[1] & np.uint32(_abi.FLAG_CAPACITY) and tid[1] == 0
    ids = np.concatenate([r[0] for r in rows]).astype(np.uint32)
    vals = np.concatenate([r[1] for r in rows]).astype(np.float32)
    off = np.zeros(w.B + 1, np.int64)
    off[1:] = np.cumsum([len(r[0]) for r in rows])
    want, ex, _ = oracle.sample_batch(w.logits, w.dtype, w.B, w.V, w.V, w.params, w.hist, w.hist_off,
                                      None, 0, ids, vals, off, us)
    for r in (0, 2, 3):
        assert not fl[r] & np.uint32(_abi.FLAG_ERROR) and tid[r] == want[r], r
    with pytest.raises(_abi.SamplerError, match="1024 bias entries"):
        sampler.sample_host(w.logits, w.params, history=hist_rows(w), bias=rows, uniforms=us)
