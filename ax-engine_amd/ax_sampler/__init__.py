"""MI355X per-step token sampler (gfx950 HIP kernels behind a C ABI).

Host-side mirror of AX Engine's sampler API; see sampler.py and params.py.
"""
from .params import (  # noqa: F401
    PARAMS_DTYPE,
    MlxSamplingParams,
    SampledToken,
    SamplerInput,
    SamplerRequest,
    SamplingParams,
    StopReason,
    pack_params,
    sampling_params_allow_deterministic_argmax_fast_path,
)
from .sampler import (  # noqa: F401
    BatchedSamplingClass,
    HipSampler,
    HipTokenSampler,
    argmax_batched,
    batched_sampling_class,
    recent_repetition_tokens,
    sample_batched,
)
