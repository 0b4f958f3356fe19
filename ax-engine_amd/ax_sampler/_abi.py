"""ctypes binding of libax_hip_sampler.so (include/ax_hip_sampler.h) and its build.

The library is the product: every sampling call goes through it.  Loading it
fails loudly when it is missing — there is no CPU fallback in this package.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
import threading

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(PKG_DIR))
CSRC = os.path.join(os.path.dirname(PKG_DIR), "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB_PATH = os.path.join(PKG_DIR, "libax_hip_sampler.so")

ABI_VERSION = 2
AXS_OK = 0
AXS_DTYPE_F32 = 0
AXS_DTYPE_BF16 = 1

FLAG_GREEDY = 1 << 0
FLAG_ARGMAX_FALLBACK = 1 << 1
FLAG_DREW = 1 << 2
FLAG_EXACT_PATH = 1 << 3
FLAG_NEAR_DRAW = 1 << 4
FLAG_NEAR_NUCLEUS = 1 << 5
FLAG_NEAR_MINP = 1 << 6
FLAG_NEAR_TIE = 1 << 7
FLAG_NEAR_ANY = FLAG_NEAR_DRAW | FLAG_NEAR_NUCLEUS | FLAG_NEAR_MINP | FLAG_NEAR_TIE
FLAG_CAPACITY = 1 << 8
FLAG_ERROR = 1 << 31

MTP_FLAG_RESIDUAL = 1 << 0
MTP_FLAG_BONUS = 1 << 1
MTP_FLAG_NEAR_ACCEPT = 1 << 2
MTP_FLAG_NEAR = 1 << 3
MTP_FLAG_CORRECTION = 1 << 4
MTP_FLAG_TAIL_ROW = 1 << 5
MTP_FLAG_ERROR = 1 << 31

MTP_SRC_DEFAULT, MTP_SRC_MTP, MTP_SRC_GEMMA, MTP_SRC_NGRAM, MTP_SRC_HYBRID = range(5)
MTP_MODEL_GREEDY, MTP_MODEL_REJECTION = 0, 1
MTP_NGRAM_CONFIDENCE, MTP_NGRAM_DELTA, MTP_NGRAM_GREEDY = 0, 1, 2
MTP_LNQ_DISTRIBUTION, MTP_LNQ_FULL_SOFTMAX = 0, 1
MTP_DRAFT_SAMPLED, MTP_DRAFT_STOCHASTIC = 0, 1
MTP_TARGET_DISTRIBUTION, MTP_TARGET_FILTERED = 0, 1

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

EXPORTS = (
    "axs_abi_version",
    "axs_last_error",
    "axs_set_error_handler",
    "axs_context_create",
    "axs_context_destroy",
    "axs_sample_batch",
    "axs_sample_batch_host",
    "axs_argmax_batch",
    "axs_argmax_batch_noalloc",
    "axs_mtp_verify",
    "axs_mtp_verify_ex",
    "axs_token_logprob_batch",
    "axs_soft_close_probe",
    "axs_top_logprobs",
    "axs_lm_head",
    "axs_mtp_draft",
    "axs_timing_enable",
    "axs_timing_read",
)

KERNEL_STREAM, KERNEL_EXACT_MAT, KERNEL_EXACT_ROW, KERNEL_MTP, KERNEL_LM_HEAD = range(5)
KERNEL_NAMES = ("k_stream", "k_exact_mat", "k_exact_row", "k_mtp_verify", "k_lm_head")


def build_library(verbose: bool = False) -> str:
    """Compiles csrc/axs_sampler.hip for gfx950 into LIB_PATH (in-tree)."""
    src = os.path.join(CSRC, "axs_sampler.hip")
    tmp = LIB_PATH + ".tmp"
    cmd = ["hipcc", *HIPCC_FLAGS, f"-I{INCLUDE}", "-o", tmp, src]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + r.stderr[-4000:])
    if verbose and r.stderr:
        print(r.stderr[-2000:])
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


class BatchDesc(C.Structure):
    _fields_ = [
        ("logits", C.c_void_p),
        ("dtype", C.c_int32),
        ("batch", C.c_int32),
        ("vocab", C.c_int32),
        ("reserved0", C.c_int32),
        ("row_stride", C.c_int64),
        ("params", C.c_void_p),
        ("history", C.c_void_p),
        ("history_offsets", C.c_void_p),
        ("history_len", C.c_int64),
        ("mask_words", C.c_void_p),
        ("mask_stride", C.c_int64),
        ("bias_ids", C.c_void_p),
        ("bias_values", C.c_void_p),
        ("bias_offsets", C.c_void_p),
        ("bias_len", C.c_int64),
        ("uniforms", C.c_void_p),
    ]


class Outputs(C.Structure):
    _fields_ = [
        ("token_ids", C.c_void_p),
        ("logprobs", C.c_void_p),
        ("flags", C.c_void_p),
        ("kept_ids", C.c_void_p),
        ("kept_count", C.c_void_p),
        ("kept_cap", C.c_int32),
        ("reserved0", C.c_int32),
    ]


class MtpDesc(C.Structure):
    _fields_ = [
        ("target_logits", C.c_void_p),
        ("draft_logits", C.c_void_p),
        ("dtype", C.c_int32),
        ("batch", C.c_int32),
        ("depth", C.c_int32),
        ("vocab", C.c_int32),
        ("row_stride", C.c_int64),
        ("draft_ids", C.c_void_p),
        ("target_params", C.c_void_p),
        ("draft_params", C.c_void_p),
        ("uniforms", C.c_void_p),
    ]


class MtpOptions(C.Structure):
    _fields_ = [
        ("sources", C.c_void_p),
        ("pending_log_probs", C.c_void_p),
        ("predicted", C.c_void_p),
        ("model_mode", C.c_int32),
        ("ngram_mode", C.c_int32),
        ("lnq_mode", C.c_int32),
        ("delta_correction", C.c_int32),
        ("target_law", C.c_int32),
        ("target_topk", C.c_uint32),
    ]


class MtpOutputs(C.Structure):
    _fields_ = [
        ("out_ids", C.c_void_p),
        ("out_count", C.c_void_p),
        ("accept_count", C.c_void_p),
        ("flags", C.c_void_p),
    ]


_lib = None
_lock = threading.Lock()


class SamplerError(RuntimeError):
    pass


def lib():
    """Loads the HIP library (torch is imported first so that one HIP runtime
    serves both: the library's libamdhip64.so.7 resolves to torch's copy)."""
    global _lib
    with _lock:
        if _lib is None:
            import torch  # noqa: F401  (HIP runtime shared with torch)

            if not os.path.exists(LIB_PATH):
                raise SamplerError(
                    f"{LIB_PATH} is missing: build it first (__graft_entry__.build() or "
                    "ax_sampler._abi.build_library())"
                )
            L = C.CDLL(LIB_PATH)
            vp, i32, i64 = C.c_void_p, C.c_int, C.c_int64
            L.axs_abi_version.restype = i32
            L.axs_abi_version.argtypes = []
            L.axs_last_error.restype = C.c_char_p
            L.axs_last_error.argtypes = []
            L.axs_set_error_handler.restype = None
            L.axs_set_error_handler.argtypes = [vp, vp]
            L.axs_context_create.restype = i32
            L.axs_context_create.argtypes = [i32, i32, i32, C.POINTER(vp)]
            L.axs_context_destroy.restype = i32
            L.axs_context_destroy.argtypes = [vp]
            L.axs_sample_batch.restype = i32
            L.axs_sample_batch.argtypes = [vp, C.POINTER(BatchDesc), C.POINTER(Outputs), vp]
            L.axs_sample_batch_host.restype = i32
            L.axs_sample_batch_host.argtypes = [vp, C.POINTER(BatchDesc), C.POINTER(Outputs)]
            L.axs_argmax_batch.restype = i32
            L.axs_argmax_batch.argtypes = [vp, vp, i32, i32, i32, i64, vp, vp, vp]
            L.axs_argmax_batch_noalloc.restype = i32
            L.axs_argmax_batch_noalloc.argtypes = [i32, vp, i32, i32, i32, i64, vp, vp, vp]
            L.axs_token_logprob_batch.restype = i32
            L.axs_token_logprob_batch.argtypes = [vp, vp, i32, i32, i32, i64, vp, vp, vp, vp]
            L.axs_top_logprobs.restype = i32
            L.axs_top_logprobs.argtypes = [vp, vp, i32, i32, i32, i64, vp, i32, vp, vp, vp]
            L.axs_soft_close_probe.restype = i32
            L.axs_soft_close_probe.argtypes = [vp, vp, i32, i32, i32, i64, vp, vp, vp, vp]
            L.axs_mtp_draft.restype = i32
            L.axs_mtp_draft.argtypes = [vp, vp, i32, i32, i32, i64, vp, i32, vp, vp, vp, vp]
            L.axs_lm_head.restype = i32
            L.axs_lm_head.argtypes = [vp, vp, i64, vp, i64, i32, i32, i32, C.c_float, C.c_float, vp, i64, vp,
                                      vp]
            L.axs_mtp_verify_ex.restype = i32
            L.axs_mtp_verify_ex.argtypes = [vp, C.POINTER(MtpDesc), C.POINTER(MtpOptions), C.POINTER(MtpOutputs), vp]
            L.axs_mtp_verify.restype = i32
            L.axs_mtp_verify.argtypes = [vp, C.POINTER(MtpDesc), C.POINTER(MtpOutputs), vp]
            L.axs_timing_enable.restype = i32
            L.axs_timing_enable.argtypes = [vp, i32]
            L.axs_timing_read.restype = i32
            L.axs_timing_read.argtypes = [vp, i32, C.POINTER(C.c_double), C.POINTER(C.c_int)]
            if L.axs_abi_version() != ABI_VERSION:
                raise SamplerError("ABI version mismatch")
            _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != AXS_OK:
        msg = lib().axs_last_error().decode(errors="replace")
        raise SamplerError(f"ax_hip_sampler error {rc}: {msg}")
