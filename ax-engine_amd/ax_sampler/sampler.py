"""Host-side mirror of the reference's sampler API over the HIP C ABI.

Runner level (crates/ax-engine-mlx):
  * ``HipSampler.sample``      — batched ``sample_categorical_into`` over a
    device [B, V] logits tensor (replaces ``sample_batched_host``,
    crates/ax-engine-mlx/src/batched_sampling.rs:123-149, and the serial loop of
    ``resolve_batched_group_tokens``, runner/mod.rs:3132-3210).
  * ``HipSampler.argmax``      — ``argmax_batched`` (batched_sampling.rs:102-111).
  * ``HipSampler.mtp_verify``  — the MTP accept / residual / bonus step
    (runner/mod.rs:12333-12462, 9732-9775).
  * ``sample_batched`` / ``argmax_batched`` — the reference's function names
    and argument meaning (per-row params, recent tokens, RNG per row; length
    mismatches raise like the reference's asserts).
  * ``batched_sampling_class`` — batched_sampling.rs:63-83.

Engine level (crates/ax-engine-core):
  * ``HipTokenSampler.sample(SamplerInput) -> list[SampledToken]`` — the
    ``TokenSampler`` plug-in (core sampling.rs:90-92) with its contract:
    one token per request in order, invalid logits → token 0 + Error,
    MaxOutputTokens at the budget (core sampling.rs:97-136).

Every call runs on the HIP library; nothing here computes a token on the CPU.
"""
from __future__ import annotations

import ctypes as C
import enum
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple, Union

import numpy as np

from . import _abi
from .params import (
    PARAMS_DTYPE,
    MlxSamplingParams,
    SampledToken,
    SamplerInput,
    SamplingParams,
    StopReason,
    pack_params,
)
from .philox import philox_uniforms


def _torch():
    import torch

    return torch


def _dev_bytes(arr: np.ndarray, device):
    """Uploads a numpy array as raw bytes; returns the device tensor."""
    torch = _torch()
    a = np.ascontiguousarray(arr)
    return torch.from_numpy(a.view(np.uint8).reshape(-1)).to(device, non_blocking=False)


def _ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


@dataclass
class SampleResult:
    token_ids: "object"   # torch.int32 [B] (u32 bits)
    logprobs: "object"    # torch.float32 [B] or None
    flags: "object"       # torch.int32 [B] (u32 bits)
    kept_ids: "object"    # torch.int32 [B, kept_cap] or None
    kept_count: "object"  # torch.int32 [B] or None
    _keep: tuple = ()

    def numpy(self):
        tid = self.token_ids.cpu().numpy().view(np.uint32)
        fl = self.flags.cpu().numpy().view(np.uint32)
        lp = None if self.logprobs is None else self.logprobs.cpu().numpy()
        kid = None if self.kept_ids is None else self.kept_ids.cpu().numpy().view(np.uint32)
        kc = None if self.kept_count is None else self.kept_count.cpu().numpy().view(np.uint32)
        return tid, lp, fl, kid, kc


@dataclass
class MtpResult:
    out_ids: "object"      # torch.int32 [B, depth + 1]
    out_count: "object"    # torch.int32 [B]
    accept_count: "object"
    flags: "object"
    _keep: tuple = ()

    def numpy(self):
        return (
            self.out_ids.cpu().numpy().view(np.uint32),
            self.out_count.cpu().numpy().view(np.uint32),
            self.accept_count.cpu().numpy().view(np.uint32),
            self.flags.cpu().numpy().view(np.uint32),
        )


def _dtype_code(t) -> int:
    torch = _torch()
    if t.dtype == torch.float32:
        return _abi.AXS_DTYPE_F32
    if t.dtype == torch.bfloat16:
        return _abi.AXS_DTYPE_BF16
    raise TypeError(f"logits must be float32 or bfloat16, got {t.dtype}")


def _csr(rows: Sequence[Sequence[int]]) -> Tuple[np.ndarray, np.ndarray]:
    off = np.zeros(len(rows) + 1, dtype=np.int64)
    for i, r in enumerate(rows):
        off[i + 1] = off[i] + len(r)
    flat = np.zeros(max(int(off[-1]), 1), dtype=np.uint32)
    for i, r in enumerate(rows):
        if len(r):
            flat[off[i] : off[i + 1]] = np.asarray(r, dtype=np.uint32)
    return flat, off


class PreparedSample:
    """One sampling step's descriptor and outputs (HipSampler.prepare_sample)."""

    def __init__(self, sampler: "HipSampler", desc, outputs, result: SampleResult):
        self.sampler, self.desc, self.outputs, self.result = sampler, desc, outputs, result
        self._dp, self._op = C.byref(desc), C.byref(outputs)

    def run(self, stream=None) -> SampleResult:
        s = self.sampler
        _abi.check(s.L.axs_sample_batch(s.ctx, self._dp, self._op, s._stream(stream)))
        return self.result


class HipSampler:
    """A sampler context on one GPU (``axs_context``): device workspace for up
    to ``max_batch`` rows of ``max_vocab`` ids."""

    def __init__(self, device: int = 0, max_batch: int = 256, max_vocab: int = 262144):
        torch = _torch()
        self.L = _abi.lib()
        self.device = torch.device("cuda", device)
        self.max_batch = max_batch
        self.max_vocab = max_vocab
        h = C.c_void_p()
        _abi.check(self.L.axs_context_create(device, max_batch, max_vocab, C.byref(h)))
        self.ctx = h

    def close(self) -> None:
        if getattr(self, "ctx", None):
            _abi.check(self.L.axs_context_destroy(self.ctx))
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def timing(self, enable: bool) -> None:
        """Brackets every launch with hipEvents on its stream (clears records)."""
        _abi.check(self.L.axs_timing_enable(self.ctx, 1 if enable else 0))

    def timing_read(self, kernel: int):
        """(total ms, launches) of one kernel class since timing was enabled."""
        ms, n = C.c_double(), C.c_int()
        _abi.check(self.L.axs_timing_read(self.ctx, kernel, C.byref(ms), C.byref(n)))
        return ms.value, n.value

    def _stream(self, stream):
        torch = _torch()
        s = torch.cuda.current_stream(self.device) if stream is None else stream
        return C.c_void_p(s.cuda_stream)

    def _params_dev(self, params):
        torch = _torch()
        if isinstance(params, np.ndarray):
            assert params.dtype == PARAMS_DTYPE
            return _dev_bytes(params, self.device)
        if isinstance(params, torch.Tensor):
            return params
        return _dev_bytes(pack_params(list(params)), self.device)

    def sample(
        self,
        logits,
        params,
        *,
        history: Union[None, Sequence[Sequence[int]], Tuple[object, object]] = None,
        mask_words=None,
        bias: Union[None, Sequence[Tuple[Sequence[int], Sequence[float]]], Tuple[object, object, object]] = None,
        uniforms=None,
        logprobs: bool = False,
        kept_cap: int = 0,
        stream=None,
    ) -> SampleResult:
        """One batched sampling step over device logits [B, V] / [B, 1, V]."""
        prep = self.prepare_sample(logits, params, history=history, mask_words=mask_words, bias=bias,
                                   uniforms=uniforms, logprobs=logprobs, kept_cap=kept_cap)
        prep.run(stream)
        return prep.result

    def prepare_sample(self, logits, params, *, history=None, mask_words=None, bias=None, uniforms=None,
                       logprobs: bool = False, kept_cap: int = 0) -> "PreparedSample":
        """The descriptor and output buffers of one sampling step, built once:
        ``run()`` then enqueues the step with a single C-ABI call and no
        allocation (for loops that sample the same buffers every step)."""
        torch = _torch()
        if logits.dim() == 3:
            if logits.shape[1] != 1:
                raise ValueError(f"batched logits must be [B, V] or [B, 1, V], got {tuple(logits.shape)}")
            logits = logits[:, 0, :]
        if logits.dim() != 2:
            raise ValueError(f"batched logits must be [B, V] or [B, 1, V], got {tuple(logits.shape)}")
        if logits.stride(1) != 1:
            logits = logits.contiguous()
        B, V = logits.shape
        keep = [logits]
        d = _abi.BatchDesc()
        d.logits = logits.data_ptr()
        d.dtype = _dtype_code(logits)
        d.batch = B
        d.vocab = V
        d.row_stride = logits.stride(0)
        pd = self._params_dev(params)
        keep.append(pd)
        d.params = pd.data_ptr()
        if history is not None:
            if isinstance(history, tuple):
                ht, ho = history
            else:
                if len(history) != B:
                    raise ValueError("history must have one entry per row")
                flat, off = _csr(history)
                ht, ho = _dev_bytes(flat, self.device), _dev_bytes(off, self.device)
                d.history_len = int(off[-1])
            if isinstance(history, tuple):
                d.history_len = int(ht.numel() * ht.element_size() // 4)
            keep += [ht, ho]
            d.history = ht.data_ptr()
            d.history_offsets = ho.data_ptr()
        if mask_words is not None:
            mw = mask_words if isinstance(mask_words, torch.Tensor) else _dev_bytes(
                np.asarray(mask_words, dtype=np.uint32), self.device)
            words = np.asarray(mask_words).shape[-1] if not isinstance(mask_words, torch.Tensor) else mask_words.shape[-1]
            keep.append(mw)
            d.mask_words = mw.data_ptr()
            d.mask_stride = int(words)
        if bias is not None:
            if isinstance(bias, tuple) and len(bias) == 3:
                bi, bv, bo = bias
                d.bias_len = int(bi.numel())
            else:
                if len(bias) != B:
                    raise ValueError("bias must have one entry per row")
                ids, off = _csr([b[0] for b in bias])
                vals = np.zeros(max(int(off[-1]), 1), dtype=np.float32)
                for i, b in enumerate(bias):
                    if len(b[1]):
                        vals[off[i] : off[i + 1]] = np.asarray(b[1], dtype=np.float32)
                bi, bv, bo = (_dev_bytes(ids, self.device), _dev_bytes(vals, self.device),
                              _dev_bytes(off, self.device))
                d.bias_len = int(off[-1])
            keep += [bi, bv, bo]
            d.bias_ids, d.bias_values, d.bias_offsets = bi.data_ptr(), bv.data_ptr(), bo.data_ptr()
        if uniforms is not None:
            ut = uniforms if isinstance(uniforms, torch.Tensor) else torch.from_numpy(
                np.ascontiguousarray(np.asarray(uniforms, dtype=np.float32))).to(self.device)
            keep.append(ut)
            d.uniforms = ut.data_ptr()
        out_ids = torch.empty(B, dtype=torch.int32, device=self.device)
        out_flags = torch.empty(B, dtype=torch.int32, device=self.device)
        out_lp = torch.empty(B, dtype=torch.float32, device=self.device) if logprobs else None
        kept = torch.empty((B, kept_cap), dtype=torch.int32, device=self.device) if kept_cap else None
        kept_n = torch.empty(B, dtype=torch.int32, device=self.device) if kept_cap else None
        o = _abi.Outputs()
        o.token_ids = out_ids.data_ptr()
        o.flags = out_flags.data_ptr()
        o.logprobs = _ptr(out_lp)
        o.kept_ids = _ptr(kept)
        o.kept_count = _ptr(kept_n)
        o.kept_cap = kept_cap
        return PreparedSample(self, d, o, SampleResult(out_ids, out_lp, out_flags, kept, kept_n, tuple(keep)))

    def sample_host(
        self,
        logits: np.ndarray,
        params,
        *,
        history: Optional[Sequence[Sequence[int]]] = None,
        mask_words: Optional[np.ndarray] = None,
        bias: Optional[Sequence[Tuple[Sequence[int], Sequence[float]]]] = None,
        uniforms: Optional[np.ndarray] = None,
        logprobs: bool = False,
        kept_cap: int = 0,
        bf16: bool = False,
    ):
        """One batched sampling step over HOST logits (``axs_sample_batch_host``):
        the engine-level boundary, whose requests carry their logits as host
        vectors (crates/ax-engine-core/src/sampling.rs:78).  ``logits`` is a
        [B, V] float32 array (or uint16 bf16 bits with ``bf16=True``); every
        other argument is host data too.  Synchronous; returns numpy arrays
        (token ids, logprobs or None, flags, kept ids or None, kept counts or
        None)."""
        lg = np.ascontiguousarray(logits)
        if lg.ndim != 2:
            raise ValueError(f"logits must be [B, V], got {lg.shape}")
        if bf16 and lg.dtype != np.uint16:
            raise TypeError("bf16 logits are passed as uint16 bits")
        if not bf16 and lg.dtype != np.float32:
            raise TypeError("logits must be float32 (or uint16 bf16 bits with bf16=True)")
        B, V = lg.shape
        keep = [lg]
        d = _abi.BatchDesc()
        d.logits = lg.ctypes.data
        d.dtype = _abi.AXS_DTYPE_BF16 if bf16 else _abi.AXS_DTYPE_F32
        d.batch, d.vocab, d.row_stride = B, V, V
        pp = params if isinstance(params, np.ndarray) else pack_params(list(params))
        assert pp.dtype == PARAMS_DTYPE and pp.size == B
        pp = np.ascontiguousarray(pp)
        keep.append(pp)
        d.params = pp.ctypes.data
        if history is not None:
            if len(history) != B:
                raise ValueError("history must have one entry per row")
            flat, off = _csr(history)
            keep += [flat, off]
            d.history, d.history_offsets, d.history_len = flat.ctypes.data, off.ctypes.data, int(off[-1])
        if mask_words is not None:
            mw = np.ascontiguousarray(mask_words, dtype=np.uint32)
            keep.append(mw)
            d.mask_words, d.mask_stride = mw.ctypes.data, int(mw.shape[-1])
        if bias is not None:
            if len(bias) != B:
                raise ValueError("bias must have one entry per row")
            ids, off = _csr([b[0] for b in bias])
            vals = np.zeros(max(int(off[-1]), 1), dtype=np.float32)
            for i, b in enumerate(bias):
                if len(b[1]):
                    vals[off[i]: off[i + 1]] = np.asarray(b[1], dtype=np.float32)
            keep += [ids, vals, off]
            d.bias_ids, d.bias_values, d.bias_offsets = ids.ctypes.data, vals.ctypes.data, off.ctypes.data
            d.bias_len = int(off[-1])
        if uniforms is not None:
            un = np.ascontiguousarray(uniforms, dtype=np.float32)
            keep.append(un)
            d.uniforms = un.ctypes.data
        tid = np.zeros(B, dtype=np.uint32)
        fl = np.zeros(B, dtype=np.uint32)
        lp = np.zeros(B, dtype=np.float32) if logprobs else None
        kid = np.zeros((B, kept_cap), dtype=np.uint32) if kept_cap else None
        kc = np.zeros(B, dtype=np.uint32) if kept_cap else None
        o = _abi.Outputs()
        o.token_ids, o.flags = tid.ctypes.data, fl.ctypes.data
        o.logprobs = None if lp is None else lp.ctypes.data
        o.kept_ids = None if kid is None else kid.ctypes.data
        o.kept_count = None if kc is None else kc.ctypes.data
        o.kept_cap = kept_cap
        _abi.check(self.L.axs_sample_batch_host(self.ctx, C.byref(d), C.byref(o)))
        return tid, lp, fl, kid, kc

    def argmax(self, logits, logprobs: bool = True, stream=None):
        """Greedy ids (first maximum, NaN skipped) and -ln sum exp(l - max)."""
        torch = _torch()
        if logits.dim() == 3:
            logits = logits[:, 0, :]
        if logits.stride(1) != 1:
            logits = logits.contiguous()
        B, V = logits.shape
        ids = torch.empty(B, dtype=torch.int32, device=self.device)
        lp = torch.empty(B, dtype=torch.float32, device=self.device) if logprobs else None
        _abi.check(self.L.axs_argmax_batch(self.ctx, logits.data_ptr(), _dtype_code(logits), B, V,
                                           logits.stride(0), ids.data_ptr(), _ptr(lp),
                                           self._stream(stream)))
        return ids, lp

    def token_logprob(self, logits, tokens, temperatures, stream=None):
        """full_vocab_token_logprob per row (axs_token_logprob_batch):
        max(ln softmax(l / T)[t], -30) over device logits [B, V]."""
        torch = _torch()
        if logits.stride(1) != 1:
            logits = logits.contiguous()
        B, V = logits.shape
        tok = tokens if isinstance(tokens, torch.Tensor) else torch.from_numpy(
            np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32)).view(np.int32)).to(self.device)
        tem = temperatures if isinstance(temperatures, torch.Tensor) else torch.from_numpy(
            np.ascontiguousarray(np.asarray(temperatures, dtype=np.float32))).to(self.device)
        out = torch.empty(B, dtype=torch.float32, device=self.device)
        _abi.check(self.L.axs_token_logprob_batch(self.ctx, logits.data_ptr(), _dtype_code(logits), B, V,
                                                  logits.stride(0), tok.data_ptr(), tem.data_ptr(),
                                                  out.data_ptr(), self._stream(stream)))
        return out

    def top_logprobs(self, logits, temperatures, n: int, stream=None):
        """The n largest full-softmax probabilities per row with their
        full_vocab_token_logprob (axs_top_logprobs): (ids int32 [B, n] holding
        uint32 ids, logprobs f32 [B, n]) on the device."""
        torch = _torch()
        if logits.stride(1) != 1:
            logits = logits.contiguous()
        B, V = logits.shape
        tem = temperatures if isinstance(temperatures, torch.Tensor) else torch.from_numpy(
            np.ascontiguousarray(np.asarray(temperatures, dtype=np.float32))).to(self.device)
        ids = torch.empty((B, n), dtype=torch.int32, device=self.device)
        lp = torch.empty((B, n), dtype=torch.float32, device=self.device)
        _abi.check(self.L.axs_top_logprobs(self.ctx, logits.data_ptr(), _dtype_code(logits), B, V,
                                           logits.stride(0), tem.data_ptr(), n, ids.data_ptr(),
                                           lp.data_ptr(), self._stream(stream)))
        return ids, lp

    def mtp_draft(self, logits, params, mode: int, uniforms=None, stream=None):
        """One MTP draft depth (axs_mtp_draft): the draft token of every row
        (argmax, or a categorical draw at the row's temperature) and its
        full-softmax log-prob.  params: PARAMS_DTYPE [B] (numpy or a device
        uint8 tensor); returns (ids int32 [B] holding uint32 ids, lnq f32 [B])
        on the device."""
        torch = _torch()
        if logits.stride(1) != 1:
            logits = logits.contiguous()
        B, V = logits.shape
        pd = params if isinstance(params, torch.Tensor) else torch.from_numpy(
            np.ascontiguousarray(params).view(np.uint8)).to(self.device)
        ud = None
        if uniforms is not None:
            ud = uniforms if isinstance(uniforms, torch.Tensor) else torch.from_numpy(
                np.ascontiguousarray(np.asarray(uniforms, dtype=np.float32))).to(self.device)
        ids = torch.empty(B, dtype=torch.int32, device=self.device)
        lnq = torch.empty(B, dtype=torch.float32, device=self.device)
        _abi.check(self.L.axs_mtp_draft(self.ctx, logits.data_ptr(), _dtype_code(logits), B, V, logits.stride(0),
                                        pd.data_ptr(), int(mode), ud.data_ptr() if ud is not None else None,
                                        ids.data_ptr(), lnq.data_ptr(), self._stream(stream)))
        return ids, lnq

    def lm_head(self, hidden, weight, scale: float = 1.0, softcap: float = 0.0, want_logits: bool = True,
                want_argmax: bool = True, stream=None):
        """The LM-head projection with the greedy decision fused (axs_lm_head):
        hidden bf16 [B, H], weight bf16 [V, H] on the device.  Returns
        (logits f32 [B, V] or None, argmax int32 [B] holding uint32 ids or
        None)."""
        torch = _torch()
        if hidden.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
            raise ValueError("hidden and weight must be bfloat16")
        if hidden.stride(1) != 1:
            hidden = hidden.contiguous()
        if weight.stride(1) != 1:
            weight = weight.contiguous()
        B, H = hidden.shape
        V = weight.shape[0]
        logits = torch.empty((B, V), dtype=torch.float32, device=self.device) if want_logits else None
        ids = torch.empty(B, dtype=torch.int32, device=self.device) if want_argmax else None
        _abi.check(self.L.axs_lm_head(self.ctx, hidden.data_ptr(), hidden.stride(0), weight.data_ptr(),
                                      weight.stride(0), B, H, V, float(scale), float(softcap),
                                      logits.data_ptr() if logits is not None else None,
                                      logits.stride(0) if logits is not None else 0,
                                      ids.data_ptr() if ids is not None else None, self._stream(stream)))
        return logits, ids

    def soft_close_probe(self, logits, think_ids, ranks, stream=None):
        """think_soft_close_in_top_k per row (axs_soft_close_probe): 1 when
        think_ids[r] is within the top ranks[r] raw logits of row r, else 0
        (0xFFFFFFFF: declined, see the header).  Returns a device uint32 view
        (torch int32)."""
        torch = _torch()
        if logits.stride(1) != 1:
            logits = logits.contiguous()
        B, V = logits.shape
        tid = think_ids if isinstance(think_ids, torch.Tensor) else torch.from_numpy(
            np.ascontiguousarray(np.asarray(think_ids, dtype=np.uint32)).view(np.int32)).to(self.device)
        rk = ranks if isinstance(ranks, torch.Tensor) else torch.from_numpy(
            np.ascontiguousarray(np.asarray(ranks, dtype=np.uint32)).view(np.int32)).to(self.device)
        out = torch.empty(B, dtype=torch.int32, device=self.device)
        _abi.check(self.L.axs_soft_close_probe(self.ctx, logits.data_ptr(), _dtype_code(logits), B, V,
                                               logits.stride(0), tid.data_ptr(), rk.data_ptr(),
                                               out.data_ptr(), self._stream(stream)))
        return out

    def mtp_verify(self, target, draft, draft_ids, target_params, draft_params, uniforms=None,
                   stream=None, options: Optional[dict] = None) -> MtpResult:
        """target [B, D+1, V], draft [B, D, V] on device; draft_ids [B, D].
        ``options`` (dict) selects ``axs_mtp_verify_ex``: ``sources`` /
        ``pending_log_probs`` / ``predicted`` ([B, D] arrays or None),
        ``model_mode``, ``ngram_mode``, ``lnq_mode``, ``delta_correction``,
        ``target_law``, ``target_topk``;
        its uniforms are taken in the reference's stream order."""
        torch = _torch()
        B, D1, V = target.shape
        D = D1 - 1
        if tuple(draft.shape) != (B, D, V):
            raise ValueError("draft must be [B, depth, V] with target [B, depth + 1, V]")
        if target.stride(2) != 1 or not target.is_contiguous():
            target = target.contiguous()
        if not draft.is_contiguous():
            draft = draft.contiguous()
        if draft.dtype != target.dtype:
            raise TypeError("target and draft must share a dtype")
        keep = [target, draft]
        d = _abi.MtpDesc()
        d.target_logits = target.data_ptr()
        d.draft_logits = draft.data_ptr()
        d.dtype = _dtype_code(target)
        d.batch, d.depth, d.vocab = B, D, V
        d.row_stride = V
        di = draft_ids if isinstance(draft_ids, torch.Tensor) else _dev_bytes(
            np.asarray(draft_ids, dtype=np.uint32), self.device)
        tp, dp = self._params_dev(target_params), self._params_dev(draft_params)
        keep += [di, tp, dp]
        d.draft_ids, d.target_params, d.draft_params = di.data_ptr(), tp.data_ptr(), dp.data_ptr()
        if uniforms is not None:
            ut = uniforms if isinstance(uniforms, torch.Tensor) else torch.from_numpy(
                np.ascontiguousarray(np.asarray(uniforms, dtype=np.float32))).to(self.device)
            keep.append(ut)
            d.uniforms = ut.data_ptr()
        out_ids = torch.empty((B, D + 1), dtype=torch.int32, device=self.device)
        out_n = torch.empty(B, dtype=torch.int32, device=self.device)
        acc = torch.empty(B, dtype=torch.int32, device=self.device)
        fl = torch.empty(B, dtype=torch.int32, device=self.device)
        o = _abi.MtpOutputs()
        o.out_ids, o.out_count, o.accept_count, o.flags = (out_ids.data_ptr(), out_n.data_ptr(),
                                                          acc.data_ptr(), fl.data_ptr())
        if options is None:
            _abi.check(self.L.axs_mtp_verify(self.ctx, C.byref(d), C.byref(o), self._stream(stream)))
            return MtpResult(out_ids, out_n, acc, fl, tuple(keep))
        op = _abi.MtpOptions()
        for name, dt in (("sources", np.uint32), ("pending_log_probs", np.float32), ("predicted", np.uint32)):
            v = options.get(name)
            if v is not None:
                t = v if isinstance(v, torch.Tensor) else _dev_bytes(np.asarray(v, dtype=dt), self.device)
                keep.append(t)
                setattr(op, name, t.data_ptr())
        op.model_mode = int(options.get("model_mode", _abi.MTP_MODEL_REJECTION))
        op.ngram_mode = int(options.get("ngram_mode", _abi.MTP_NGRAM_CONFIDENCE))
        op.lnq_mode = int(options.get("lnq_mode", _abi.MTP_LNQ_DISTRIBUTION))
        op.delta_correction = int(bool(options.get("delta_correction", False)))
        op.target_law = int(options.get("target_law", _abi.MTP_TARGET_DISTRIBUTION))
        op.target_topk = int(options.get("target_topk", 0))
        _abi.check(self.L.axs_mtp_verify_ex(self.ctx, C.byref(d), C.byref(op), C.byref(o), self._stream(stream)))
        return MtpResult(out_ids, out_n, acc, fl, tuple(keep))


# ---------------------------------------------------------------------------
# reference-named helpers
# ---------------------------------------------------------------------------


class BatchedSamplingClass(enum.Enum):
    """batched_sampling.rs:40-50."""

    GREEDY = "greedy"
    HOST_SAMPLED = "host_sampled"


def batched_sampling_class(sampling: MlxSamplingParams, deterministic_argmax_sampling: bool):
    """batched_sampling.rs:63-83: Greedy / HostSampled / None (pure temperature,
    which the reference sends to MLX's global-RNG categorical).  On this GPU path
    every class is served by ``HipSampler.sample``; the classifier is kept so a
    caller's routing logic ports unchanged."""
    if deterministic_argmax_sampling:
        return BatchedSamplingClass.GREEDY
    temp_positive = sampling.temperature > 0.0
    uses_processors = sampling.uses_logits_processors()
    if temp_positive and not uses_processors and sampling.top_k == 0 and sampling.top_p >= 1.0:
        return None
    if temp_positive or uses_processors:
        return BatchedSamplingClass.HOST_SAMPLED
    return BatchedSamplingClass.GREEDY


def argmax_batched(sampler: HipSampler, logits) -> List[int]:
    """argmax_batched (batched_sampling.rs:102-111) on the GPU."""
    ids, _ = sampler.argmax(logits, logprobs=False)
    return ids.cpu().numpy().view(np.uint32).tolist()


def sample_batched(
    sampler: HipSampler,
    logits,
    params: Sequence[MlxSamplingParams],
    recent: Sequence[Sequence[int]],
    seeds: Sequence[int],
    steps: Sequence[int],
    uniforms=None,
) -> List[int]:
    """sample_batched_host (batched_sampling.rs:123-149) on the GPU: row r is
    sample_categorical_into(row r, params[r], recent[r]) with the row's draw
    taken from Philox(seeds[r], r, steps[r]) (or ``uniforms[r]``)."""
    B = logits.shape[0]
    if len(params) != B:
        raise AssertionError("params must have one entry per row")
    if len(recent) != B:
        raise AssertionError("recent must have one entry per row")
    if len(seeds) != B or len(steps) != B:
        raise AssertionError("rngs must have one entry per row")
    packed = pack_params(list(params), seeds, steps)
    res = sampler.sample(logits, packed, history=list(recent), uniforms=uniforms)
    return res.token_ids.cpu().numpy().view(np.uint32).tolist()


def recent_repetition_tokens(prompt: Sequence[int], generated: Sequence[int],
                             context_size: Optional[int]) -> List[int]:
    """crates/ax-engine-core/src/sampling.rs:193-216."""
    total = len(prompt) + len(generated)
    keep = total if context_size is None else min(context_size, total)
    if keep == 0:
        return []
    start = total - keep
    if start < len(prompt):
        return list(prompt[start:]) + list(generated)
    return list(generated[start - len(prompt):])


class HipTokenSampler:
    """``TokenSampler`` (crates/ax-engine-core/src/sampling.rs:90-92) on the GPU.

    The requests that carry logits are sampled in one call of the host-pointer
    entry point (``axs_sample_batch_host``: the logits are host vectors at this
    level, core sampling.rs:78), each with its own ``SamplingParams`` under
    the MLX law (greedy rows: first-maximum argmax with the core sampler's
    logprob -ln sum exp(l - max), reproduced from its sequential f32 sum;
    sampled rows: the full filter chain, drawn from Philox(seed, request_id,
    generated_len)).  The core ``DeterministicSampler``'s contract otherwise
    (core sampling.rs:97-136):
      * one ``SampledToken`` per request, in order;
      * invalid logits — empty, or a maximum under ``f32::total_cmp`` that is
        not finite (a +NaN ranks above +inf there, a -NaN below -inf; core
        sampling.rs:172-178) — give token 0, ``StopReason.ERROR``, no logprob;
      * ``MaxOutputTokens`` when ``generated_len + 1 >= max_output_tokens``
        (saturating);
      * requests without logits keep the core stub: ``previous_token + 1``
        (saturating at 0xFFFFFFFF), logprob 0.
    Ties: this sampler keeps the MLX sampler's first maximum, where the core
    DeterministicSampler keeps the last one.  Rows of different widths are
    sampled in separate calls.
    """

    def __init__(self, sampler: HipSampler):
        self.sampler = sampler

    @staticmethod
    def _valid(arr: np.ndarray) -> bool:
        if arr.size == 0:
            return False
        bits = arr.view(np.uint32)
        nan = np.isnan(arr)
        if np.any(nan & ((bits >> np.uint32(31)) == 0)):
            return False  # a +NaN is the total_cmp maximum
        rest = arr[~nan]
        return rest.size > 0 and bool(np.isfinite(rest.max()))

    def sample(self, inp: SamplerInput) -> List[SampledToken]:
        reqs = inp.requests
        rows, idx = [], []
        for i, rq in enumerate(reqs):
            if rq.logits is None:
                continue
            arr = np.ascontiguousarray(rq.logits, dtype=np.float32)
            if not self._valid(arr):
                continue  # invalid: token 0 + Error below
            rows.append(arr)
            idx.append(i)
        tokens, lps = {}, {}
        groups = {}
        for r, i in zip(rows, idx):
            groups.setdefault(r.size, []).append((r, i))
        for V, items in groups.items():
            mat = np.stack([r for r, _ in items])
            ids = [i for _, i in items]
            # the core sampler penalises every recent token it is given (the
            # engine has already cut them to the window,
            # crates/ax-engine-core/src/engine.rs:1180-1197)
            mps = [reqs[i].sampling_params.to_mlx() for i in ids]
            for mp in mps:
                mp.repetition_context_size = None
            hist = [list(reqs[i].recent_tokens) for i in ids]
            seeds = [reqs[i].sampling_params.seed for i in ids]
            us = philox_uniforms(seeds, [reqs[i].request_id for i in ids],
                                 [reqs[i].generated_len for i in ids])
            tid, lp, fl, _, _ = self.sampler.sample_host(mat, pack_params(mps, seeds), history=hist,
                                                         uniforms=us, logprobs=True)
            for k, i in enumerate(ids):
                if fl[k] & _abi.FLAG_ERROR:
                    continue
                tokens[i] = int(tid[k])
                lps[i] = float(lp[k])
        out: List[SampledToken] = []
        for i, rq in enumerate(reqs):
            invalid = rq.logits is not None and i not in tokens
            if invalid:
                tok, lp, stop = 0, None, StopReason.ERROR
            else:
                tok = tokens.get(i, min(rq.previous_token + 1, 0xFFFFFFFF))
                lp = lps.get(i, 0.0)
                stop = (StopReason.MAX_OUTPUT_TOKENS
                        if min(rq.generated_len + 1, 0xFFFFFFFF) >= rq.max_output_tokens else None)
            out.append(SampledToken(rq.request_id, tok, stop, lp))
        return out
