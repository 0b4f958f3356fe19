"""Sampling parameters and the engine-level sampler types.

Mirrors the reference's plug-in API so a caller of ax-engine-core finds the
same names and meanings:

* ``SamplingParams``  — crates/ax-engine-core/src/sampling.rs:7-41 (defaults
  :25-41), plus the two build extensions ``presence_penalty`` /
  ``frequency_penalty`` (absent in the reference, whose OpenAI route rejects
  them: crates/ax-engine-server/src/openai/requests.rs:1240-1281).
* ``StopReason``, ``SampledToken``, ``SamplerRequest``, ``SamplerInput`` —
  crates/ax-engine-core/src/sampling.rs:54-88.
* ``MlxSamplingParams`` — crates/ax-engine-mlx/src/sampling.rs:39-114 (the
  runner-level parameter set that ``sample_categorical_into`` consumes).

``PARAMS_DTYPE`` is the numpy layout of the C ``axs_sampling_params`` struct
(include/ax_hip_sampler.h), 64 bytes per row.
"""
from __future__ import annotations

import enum
import math
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np

AXS_NONE_U32 = 0xFFFFFFFF

PARAMS_DTYPE = np.dtype(
    [
        ("temperature", "<f4"),
        ("top_p", "<f4"),
        ("top_k", "<u4"),
        ("min_p", "<f4"),
        ("has_min_p", "<u4"),
        ("repetition_penalty", "<f4"),
        ("repetition_context_size", "<u4"),
        ("no_repeat_ngram_size", "<u4"),
        ("ngram_window", "<u4"),
        ("presence_penalty", "<f4"),
        ("frequency_penalty", "<f4"),
        ("reserved0", "<u4"),
        ("seed", "<u8"),
        ("step", "<u8"),
    ]
)
assert PARAMS_DTYPE.itemsize == 64


@dataclass
class MlxSamplingParams:
    """Runner-level knobs (crates/ax-engine-mlx/src/sampling.rs:39-114)."""

    temperature: float = 0.0
    top_p: float = 1.0
    top_k: int = 0
    min_p: Optional[float] = None
    repetition_penalty: float = 1.0
    repetition_context_size: Optional[int] = None
    no_repeat_ngram_size: int = 0
    ngram_window: int = 128
    # build extensions (not in the reference)
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0

    @staticmethod
    def new(temperature: float, top_p: float, top_k: int) -> "MlxSamplingParams":
        """``MlxSamplingParams::new`` (sampling.rs:53-64)."""
        return MlxSamplingParams(temperature=temperature, top_p=top_p, top_k=top_k)

    @staticmethod
    def greedy() -> "MlxSamplingParams":
        """``MlxSamplingParams::greedy`` (sampling.rs:66-68)."""
        return MlxSamplingParams.new(0.0, 1.0, 0)

    def with_repetition_penalty(self, penalty: float, context: Optional[int]) -> "MlxSamplingParams":
        self.repetition_penalty = penalty
        self.repetition_context_size = context
        return self

    def with_min_p(self, min_p: Optional[float]) -> "MlxSamplingParams":
        self.min_p = min_p
        return self

    def with_no_repeat_ngram(self, size: int, window: int) -> "MlxSamplingParams":
        self.no_repeat_ngram_size = size
        self.ngram_window = window
        return self

    def uses_min_p(self) -> bool:
        """sampling.rs:86-89: active iff finite and > 0."""
        return self.min_p is not None and math.isfinite(self.min_p) and self.min_p > 0.0

    def uses_repetition_penalty(self) -> bool:
        """sampling.rs:91-95: active iff finite, > 0 and != 1."""
        r = self.repetition_penalty
        return math.isfinite(r) and r > 0.0 and r != 1.0

    def uses_no_repeat_ngram(self) -> bool:
        return self.no_repeat_ngram_size > 0

    def uses_logits_processors(self) -> bool:
        return self.uses_repetition_penalty() or self.uses_no_repeat_ngram()


@dataclass
class SamplingParams:
    """Engine-level request parameters (crates/ax-engine-core/src/sampling.rs:7-41)."""

    temperature: float = 0.0
    top_p: float = 1.0
    top_k: int = 0
    min_p: Optional[float] = None
    repetition_penalty: float = 1.0
    repetition_context_size: Optional[int] = None
    no_repeat_ngram_size: int = 0
    ngram_window: int = 128
    seed: int = 0
    deterministic: bool = True
    ignore_eos: bool = False
    # build extensions (not in the reference)
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0

    def to_mlx(self) -> MlxSamplingParams:
        """``sampling_params_from_context`` (crates/ax-engine-mlx/src/runner/mod.rs:2063-2069)."""
        return MlxSamplingParams(
            temperature=self.temperature,
            top_p=self.top_p,
            top_k=self.top_k,
            min_p=self.min_p,
            repetition_penalty=self.repetition_penalty,
            repetition_context_size=self.repetition_context_size,
            no_repeat_ngram_size=self.no_repeat_ngram_size,
            ngram_window=self.ngram_window,
            presence_penalty=self.presence_penalty,
            frequency_penalty=self.frequency_penalty,
        )


def sampling_params_allow_deterministic_argmax_fast_path(p: SamplingParams) -> bool:
    """crates/ax-engine-core/src/sampling.rs:43-52."""
    return (
        p.deterministic
        and p.temperature <= 0.0
        and p.top_k == 0
        and p.top_p >= 1.0
        and p.repetition_penalty == 1.0
        and p.no_repeat_ngram_size == 0
    )


class StopReason(enum.Enum):
    """crates/ax-engine-core/src/sampling.rs:54-64."""

    EOS_TOKEN = "eos_token"
    MAX_OUTPUT_TOKENS = "max_output_tokens"
    CANCELLED = "cancelled"
    ERROR = "error"
    LOOP_DETECTED = "loop_detected"


@dataclass
class SampledToken:
    """crates/ax-engine-core/src/sampling.rs:66-72."""

    request_id: int
    token_id: int
    stop_reason: Optional[StopReason]
    logprob: Optional[float]


@dataclass
class SamplerRequest:
    """crates/ax-engine-core/src/sampling.rs:74-83."""

    request_id: int
    previous_token: int
    logits: Optional[Sequence[float]]
    recent_tokens: List[int] = field(default_factory=list)
    generated_len: int = 0
    max_output_tokens: int = 0
    sampling_params: SamplingParams = field(default_factory=SamplingParams)


@dataclass
class SamplerInput:
    """crates/ax-engine-core/src/sampling.rs:85-88."""

    requests: List[SamplerRequest]


def pack_params(
    params: Sequence[MlxSamplingParams],
    seeds: Optional[Sequence[int]] = None,
    steps: Optional[Sequence[int]] = None,
) -> np.ndarray:
    """Packs per-row parameters into the C ``axs_sampling_params`` layout."""
    out = np.zeros(len(params), dtype=PARAMS_DTYPE)
    for i, p in enumerate(params):
        out[i]["temperature"] = p.temperature
        out[i]["top_p"] = p.top_p
        out[i]["top_k"] = p.top_k
        out[i]["has_min_p"] = 0 if p.min_p is None else 1
        out[i]["min_p"] = 0.0 if p.min_p is None else p.min_p
        out[i]["repetition_penalty"] = p.repetition_penalty
        out[i]["repetition_context_size"] = (
            AXS_NONE_U32 if p.repetition_context_size is None else p.repetition_context_size
        )
        out[i]["no_repeat_ngram_size"] = p.no_repeat_ngram_size
        out[i]["ngram_window"] = p.ngram_window
        out[i]["presence_penalty"] = p.presence_penalty
        out[i]["frequency_penalty"] = p.frequency_penalty
        out[i]["seed"] = 0 if seeds is None else int(seeds[i]) & 0xFFFFFFFFFFFFFFFF
        out[i]["step"] = 0 if steps is None else int(steps[i]) & 0xFFFFFFFFFFFFFFFF
    return out
