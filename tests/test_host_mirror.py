"""CPU checks of the host-side mirror of the reference's sampler API
(ax-engine_amd/ax_sampler): routing predicates, repetition windows, the
numpy Philox, and the argument checks that run before any GPU call.  The
first three tests transcribe the reference's own unit tests."""
import numpy as np
import pytest

from ax_sampler import (BatchedSamplingClass, MlxSamplingParams, SamplingParams, batched_sampling_class,
                        recent_repetition_tokens, sample_batched,
                        sampling_params_allow_deterministic_argmax_fast_path)
from ax_sampler.philox import philox4x32_10, philox_uniforms


def test_classify_matches_single_decode_branches():
    """crates/ax-engine-mlx/src/batched_sampling.rs:267-311."""
    G, H = BatchedSamplingClass.GREEDY, BatchedSamplingClass.HOST_SAMPLED
    assert batched_sampling_class(MlxSamplingParams.greedy(), False) == G
    assert batched_sampling_class(MlxSamplingParams.new(0.7, 0.9, 40), True) == G
    assert batched_sampling_class(MlxSamplingParams.new(0.7, 0.9, 0), False) == H
    assert batched_sampling_class(MlxSamplingParams.new(0.7, 1.0, 40), False) == H
    assert batched_sampling_class(MlxSamplingParams.greedy().with_repetition_penalty(1.2, None), False) == H
    assert batched_sampling_class(MlxSamplingParams.new(0.8, 1.0, 0), False) is None
    assert batched_sampling_class(MlxSamplingParams.new(0.8, 1.0, 0).with_repetition_penalty(1.0, None),
                                  False) is None


def test_deterministic_argmax_fast_path_only_allows_default_greedy_sampling():
    """crates/ax-engine-core/src/sampling.rs:357-370, plus each field that
    closes the fast path (:43-52)."""
    assert sampling_params_allow_deterministic_argmax_fast_path(SamplingParams())
    assert not sampling_params_allow_deterministic_argmax_fast_path(SamplingParams(temperature=0.7))
    for kw in ({"top_k": 5}, {"top_p": 0.9}, {"repetition_penalty": 1.1},
               {"no_repeat_ngram_size": 3}, {"deterministic": False}):
        assert not sampling_params_allow_deterministic_argmax_fast_path(SamplingParams(**kw)), kw
    # min_p is inert for greedy argmax: the fast path ignores it
    assert sampling_params_allow_deterministic_argmax_fast_path(SamplingParams(min_p=0.2))


def test_recent_repetition_tokens_respects_context_size_across_prompt_and_generated():
    """crates/ax-engine-core/src/sampling.rs:441-451."""
    assert recent_repetition_tokens([1, 2, 3], [4, 5], 3) == [3, 4, 5]
    assert recent_repetition_tokens([1, 2, 3], [4, 5], 1) == [5]
    assert recent_repetition_tokens([1, 2, 3], [4, 5], None) == [1, 2, 3, 4, 5]
    assert recent_repetition_tokens([1, 2, 3], [4, 5], 0) == []
    assert recent_repetition_tokens([1, 2, 3], [], 2) == [2, 3]


def test_numpy_philox_matches_the_oracle_and_known_answers(oracle):
    # Random123 known answer (Salmon et al., SC'11)
    out = philox4x32_10(np.array([[0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344]], np.uint32),
                        np.array([[0xA4093822, 0x299F31D0]], np.uint32))
    assert out[0].tolist() == [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]
    rs = np.random.default_rng(3)
    seeds = [int(x) for x in rs.integers(0, 2**63, 64)] + [0, 2**64 - 1]
    rows = [int(x) for x in rs.integers(0, 2**32, 66)]
    steps = [int(x) for x in rs.integers(0, 2**63, 66)]
    for purpose, word in ((0, 0), (1, 2), (2, 3)):
        u = philox_uniforms(seeds, rows, steps, purpose, word)
        want = [oracle.philox_uniform(s, r, t, purpose, word) for s, r, t in zip(seeds, rows, steps)]
        assert u.tolist() == want
        assert np.all((u >= 0.0) & (u < 1.0))


def test_sample_batched_rejects_length_mismatches_like_the_reference():
    """sample_batched_host asserts one params / recent / rng entry per row
    (crates/ax-engine-mlx/src/batched_sampling.rs:129-141); the mirror raises
    before any GPU call."""
    class Logits:
        shape = (3, 5)

    p = [MlxSamplingParams.greedy()] * 3
    with pytest.raises(AssertionError):
        sample_batched(None, Logits(), p[:2], [[]] * 3, [1] * 3, [0] * 3)
    with pytest.raises(AssertionError):
        sample_batched(None, Logits(), p, [[]] * 2, [1] * 3, [0] * 3)
    with pytest.raises(AssertionError):
        sample_batched(None, Logits(), p, [[]] * 3, [1] * 2, [0] * 3)
