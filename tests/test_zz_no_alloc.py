"""GPU check of axs_argmax_batch_noalloc (no context, static device scratch)
against axs_argmax_batch, called through the C ABI.

Two calls in a row on the one-row (segmented) shape, which is the shape that
uses the scratch, the second on a smaller row so that it reads scratch the
first call left behind; then a multi-row batch and a call beyond the scratch
limit, which must be refused.  Ids and logprobs must be bit-identical to the
context entry point's (same kernels, same inputs).
"""
import ctypes as C

import numpy as np
import pytest

from ax_sampler import _abi

pytestmark = pytest.mark.gpu


def _ctx_argmax(L, ctx, t, B, V, dtype):
    import torch

    ids = torch.empty(B, dtype=torch.int32, device="cuda:0")
    lp = torch.empty(B, dtype=torch.float32, device="cuda:0")
    _abi.check(L.axs_argmax_batch(ctx, t.data_ptr(), dtype, B, V, V, ids.data_ptr(), lp.data_ptr(), None))
    torch.cuda.synchronize()
    return ids.cpu().numpy().view(np.uint32), lp.cpu().numpy()


def _noalloc_argmax(L, t, B, V, dtype):
    import torch

    ids = torch.full((B,), -1, dtype=torch.int32, device="cuda:0")
    lp = torch.full((B,), float("nan"), dtype=torch.float32, device="cuda:0")
    _abi.check(L.axs_argmax_batch_noalloc(0, t.data_ptr(), dtype, B, V, V, ids.data_ptr(),
                                          lp.data_ptr(), None))
    torch.cuda.synchronize()
    return ids.cpu().numpy().view(np.uint32), lp.cpu().numpy()


def _logits(seed, B, V, dtype):
    import torch

    rs = np.random.default_rng(seed)
    x = (rs.standard_normal((B, V), dtype=np.float32) * np.float32(3.0))
    x[:, rs.integers(0, V)] = 30.0  # a clear maximum per row, at a seeded id
    t = torch.from_numpy(x).cuda()
    if dtype == _abi.AXS_DTYPE_BF16:
        t = t.to(torch.bfloat16)
    return t


def test_noalloc_argmax_matches_the_context_entry_point():
    L = _abi.lib()
    ctx = C.c_void_p()
    _abi.check(L.axs_context_create(0, 64, 262144, C.byref(ctx)))
    try:
        cases = [(1, 262144, _abi.AXS_DTYPE_BF16, 1),   # 128 scratch segments
                 (1, 151936, _abi.AXS_DTYPE_F32, 2),    # smaller: reuses the scratch
                 (1, 4099, _abi.AXS_DTYPE_F32, 3),
                 (24, 151936, _abi.AXS_DTYPE_BF16, 4)]  # k_row: no scratch
        for B, V, dt, seed in cases:
            print(f"noalloc argmax B={B} V={V} dtype={dt}", flush=True)
            t = _logits(seed, B, V, dt)
            want_ids, want_lp = _ctx_argmax(L, ctx, t, B, V, dt)
            got_ids, got_lp = _noalloc_argmax(L, t, B, V, dt)
            assert np.array_equal(got_ids, want_ids), (B, V, got_ids, want_ids)
            assert np.array_equal(got_lp.view(np.uint32), want_lp.view(np.uint32)), (B, V)
        # beyond the scratch limit: refused before any launch
        t = _logits(5, 1, 300000, _abi.AXS_DTYPE_F32)
        ids = C.c_void_p(t.data_ptr())  # any valid device pointer
        rc = L.axs_argmax_batch_noalloc(0, t.data_ptr(), _abi.AXS_DTYPE_F32, 1, 300000, 300000,
                                        ids, None, None)
        assert rc == 3, rc  # AXS_E_CAPACITY
        assert b"262144" in L.axs_last_error()
    finally:
        L.axs_context_destroy(ctx)
