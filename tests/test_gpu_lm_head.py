"""GPU parity of the fused LM head (axs_lm_head) through the C ABI.

The projection is floating point, so its reference is the exact product,
formed in float64 by torch on the device (every bf16 product and every sum of
4,096 of them is exact or within 2^-40 relative there):

  * each logit must be the bf16 value nearest the exact dot product x (ties
    to even), as a bf16 matmul's output is, except where the f32 sum the
    kernel rounds may lie on the other side of a rounding midpoint: a logit
    must always be the bf16 rounding of some value within the f32
    accumulation bound d of x (between round(x - d) and round(x + d)).  d is
    the two-level sum's bound (each matrix-core step sums 32 exact products,
    then H/32 such partials are accumulated): (H/32 + 32) * 2^-24 *
    sum_k |h_k w_k|, which also covers the vector path of B <= 2 (per lane
    H/64 products in order, then a 64-lane tree).  Fewer than 1% of the logits may take that allowance
    (mostly logits near 0, where cancellation leaves the bound wider than a
    bf16 step);
  * scale and softcap follow the reference's f32 operations
    (crates/ax-engine-mlx/src/model/shared/utils.rs:1826-1845), checked
    within 4 f32 ulps of the same operations with a float64 tanh;
  * the argmax must equal the CPU oracle's argmax_f32 over the logits the
    kernel wrote (bit-exact), with the logits written or not, including rows
    where the softcap saturates many logits to the same value (ties to the
    lowest id) and a row of NaN (id 0).
"""
import numpy as np
import pytest

from gpu_common import log

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sampler():
    from ax_sampler import HipSampler

    s = HipSampler(0, max_batch=256, max_vocab=262144)
    yield s
    s.close()


def _inputs(B, H, V, seed, wscale=0.02):
    import torch

    g = torch.Generator(device="cpu").manual_seed(seed)
    hidden = torch.randn(B, H, generator=g).to(torch.bfloat16).to("cuda:0")
    weight = (torch.randn(V, H, generator=g) * wscale).to(torch.bfloat16).to("cuda:0")
    return hidden, weight


def _exact(hidden, weight):
    """(exact dot products, sum |h w|) in float64, computed on the device."""
    import torch

    h = hidden.double()
    out = torch.empty((hidden.shape[0], weight.shape[0]), dtype=torch.float64, device=hidden.device)
    ab = torch.empty_like(out)
    step = 32768  # bounded float64 copies of the weight
    for v0 in range(0, weight.shape[0], step):
        w = weight[v0:v0 + step].double()
        out[:, v0:v0 + step] = h @ w.T
        ab[:, v0:v0 + step] = h.abs() @ w.abs().T
        del w
    return out.cpu().numpy(), ab.cpu().numpy()


def _bf16_neighbours(x: np.ndarray):
    """For float64 x (finite, inside the bf16 normal range): the bf16 values
    below and above it, their midpoint, and the nearest (ties to even), from
    float64 bit arithmetic (a bf16 value is a float64 whose 45 low
    significand bits are zero)."""
    M = np.uint64((1 << 45) - 1)
    bits = x.view(np.uint64)
    tb = bits & ~M                                    # toward zero
    ob = np.where(bits & M, tb + np.uint64(1 << 45), tb)  # away from zero
    t, o = tb.view(np.float64), ob.view(np.float64)
    lo, hi = np.minimum(t, o), np.maximum(t, o)
    lsb = (bits >> np.uint64(45)) & np.uint64(1)
    nb = (bits + np.uint64((1 << 44) - 1) + lsb) & ~M
    return lo, hi, (lo + hi) / 2, nb.view(np.float64)


def _check_logits(got, exact, ab, H, tag):
    lo, hi, mid, nearest = _bf16_neighbours(exact)
    g = got.astype(np.float64)
    delta = (H / 32 + 32) * 2.0 ** -24 * ab
    ok_exact = g == nearest
    ok_near = (g >= _bf16_neighbours(exact - delta)[3]) & (g <= _bf16_neighbours(exact + delta)[3]) & \
        (g.view(np.uint64) & np.uint64((1 << 45) - 1) == 0)
    bad = ~(ok_exact | ok_near)
    n_flip = int(np.count_nonzero(~ok_exact & ok_near))
    log(f"lm_head {tag}: {got.size} logits, {n_flip} not the nearest bf16 value but within the bound")
    if bad.any():
        at = [tuple(ix) for ix in np.argwhere(bad)[:4].tolist()]
        detail = [(ix, float(g[ix]), float(exact[ix]), float(lo[ix]), float(hi[ix]), float(delta[ix])) for ix in at]
        raise AssertionError(f"{tag}: {int(bad.sum())} logits off: (index, got, exact, lo, hi, d) {detail}")
    assert n_flip <= 0.01 * got.size
    return nearest


def _argmax_rows(oracle, logits):
    return np.array([oracle.argmax_f32(np.ascontiguousarray(r)) for r in logits], dtype=np.uint32)


# B = 1 walks K in groups of two 512-wide pieces, then single pieces, then a
# tail of H % 512: H = 4096 is whole groups, 2592 a group, one piece and a
# 32-wide tail, 544 no group; V is odd so the last workgroup's rows pass V.
@pytest.mark.parametrize("B,H,V,seed", [(1, 4096, 151936, 1), (2, 1056, 7777, 5), (13, 2080, 50021, 2),
                                        (40, 1056, 9001, 6), (64, 4096, 151936, 3), (80, 1024, 32003, 4),
                                        (200, 512, 20011, 7), (1, 2592, 30011, 8), (1, 544, 1001, 9)])
def test_lm_head_matches_exact_product(sampler, oracle, B, H, V, seed):
    import torch

    log(f"lm_head case B={B} H={H} V={V} seed={seed}")
    hidden, weight = _inputs(B, H, V, seed)
    logits, ids = sampler.lm_head(hidden, weight)
    _, ids_only = sampler.lm_head(hidden, weight, want_logits=False)
    torch.cuda.synchronize()
    got = logits.cpu().numpy()
    exact, ab = _exact(hidden, weight)
    _check_logits(got, exact, ab, H, f"B={B} H={H} V={V}")
    want = _argmax_rows(oracle, got)
    assert np.array_equal(ids.cpu().numpy().view(np.uint32), want)
    assert np.array_equal(ids_only.cpu().numpy().view(np.uint32), want)


@pytest.mark.parametrize("B", [1, 5])
def test_lm_head_strided_operands(sampler, oracle, B):
    """hidden and weight as views into padded buffers (row strides above H,
    hidden offset by 16 bytes) and an output row stride that is not a
    multiple of 4 (so no 16-byte stores): the logits are bit-identical to
    the contiguous call's (the same kernel sums in the same order), within
    the exact product's bound, and the output's padding columns are not
    written."""
    import torch

    from ax_sampler import _abi

    H, V = 1056, 3001
    log(f"lm_head strided case B={B} H={H} V={V}")
    hidden, weight = _inputs(B, H, V, 31 + B)
    hp = torch.zeros((B, H + 40), dtype=torch.bfloat16, device="cuda:0")
    hp[:, 8:8 + H] = hidden
    wp = torch.zeros((V, H + 24), dtype=torch.bfloat16, device="cuda:0")
    wp[:, :H] = weight
    hv, wv = hp[:, 8:8 + H], wp[:, :H]
    assert hv.stride(0) == H + 40 and wv.stride(0) == H + 24
    ref_logits, ref_ids = sampler.lm_head(hidden, weight)
    os_ = V + 3
    out = torch.full((B, os_), float("nan"), dtype=torch.float32, device="cuda:0")
    ids = torch.empty(B, dtype=torch.int32, device="cuda:0")
    _abi.check(sampler.L.axs_lm_head(sampler.ctx, hv.data_ptr(), hv.stride(0), wv.data_ptr(), wv.stride(0),
                                     B, H, V, 1.0, 0.0, out.data_ptr(), os_, ids.data_ptr(),
                                     sampler._stream(None)))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isnan(got[:, V:]).all()
    assert np.array_equal(got[:, :V].view(np.uint32), ref_logits.cpu().numpy().view(np.uint32))
    exact, ab = _exact(hidden, weight)
    _check_logits(np.ascontiguousarray(got[:, :V]), exact, ab, H, f"strided B={B}")
    want = _argmax_rows(oracle, np.ascontiguousarray(got[:, :V]))
    assert np.array_equal(ids.cpu().numpy().view(np.uint32), want)
    assert np.array_equal(ref_ids.cpu().numpy().view(np.uint32), want)


def test_lm_head_scale_and_softcap(sampler, oracle):
    import torch

    B, H, V = 7, 512, 262144
    hidden, weight = _inputs(B, H, V, 11, wscale=0.2)
    scale, cap = np.float32(0.75), np.float32(30.0)
    logits, ids = sampler.lm_head(hidden, weight, scale=float(scale), softcap=float(cap))
    torch.cuda.synchronize()
    got = logits.cpu().numpy()
    exact, ab = _exact(hidden, weight)
    d = (H / 32 + 32) * 2.0 ** -24 * ab

    def capped(b):  # the reference's f32 steps on a bf16 logit b, tanh in float64
        t = (b.astype(np.float32) * scale) * (np.float32(1.0) / cap)
        return (np.tanh(t.astype(np.float64)).astype(np.float32) * cap).astype(np.float32)

    # softcap is monotone: a logit lies between the images of the bf16
    # roundings of x - d and x + d, within 4 f32 ulps
    w_lo = capped(_bf16_neighbours(exact - d)[3]).astype(np.float64)
    w_hi = capped(_bf16_neighbours(exact + d)[3]).astype(np.float64)
    tol = 4 * np.spacing(np.maximum(np.abs(w_lo), np.abs(w_hi)).astype(np.float32)).astype(np.float64)
    g = got.astype(np.float64)
    bad = (g < w_lo - tol) | (g > w_hi + tol)
    assert not bad.any(), [(tuple(ix), float(g[tuple(ix)]), float(w_lo[tuple(ix)]), float(w_hi[tuple(ix)]))
                           for ix in np.argwhere(bad)[:4].tolist()]
    single = w_lo == w_hi  # no rounding allowance: the 4-ulp bound alone
    log(f"lm_head softcap: {int(single.sum())} of {single.size} logits with one admissible bf16 value")
    assert np.count_nonzero(single) > 0.9 * single.size
    assert np.array_equal(ids.cpu().numpy().view(np.uint32), _argmax_rows(oracle, got))


def test_lm_head_ties_and_nan_rows(sampler, oracle):
    """A large scale and a small cap saturate many logits to exactly the cap:
    the argmax is the lowest saturated id.  A NaN in a row's hidden state
    makes every logit of the row NaN: id 0."""
    import torch

    B, H, V = 5, 256, 70001
    hidden, weight = _inputs(B, H, V, 21, wscale=0.3)
    hidden[3, 17] = float("nan")
    logits, ids = sampler.lm_head(hidden, weight, scale=40.0, softcap=1.0)
    _, ids_only = sampler.lm_head(hidden, weight, scale=40.0, softcap=1.0, want_logits=False)
    torch.cuda.synchronize()
    got = logits.cpu().numpy()
    n_top = [(np.count_nonzero(got[r] == np.nanmax(got[r])) if r != 3 else 0) for r in range(B)]
    log(f"lm_head ties: saturated logits per row {n_top}")
    assert min(n for r, n in enumerate(n_top) if r != 3) > 1
    assert np.isnan(got[3]).all()
    want = _argmax_rows(oracle, got)
    assert want[3] == 0
    assert np.array_equal(ids.cpu().numpy().view(np.uint32), want)
    assert np.array_equal(ids_only.cpu().numpy().view(np.uint32), want)


def test_lm_head_rejects_bad_shapes(sampler):
    import torch

    from ax_sampler._abi import SamplerError

    hidden = torch.zeros((2, 100), dtype=torch.bfloat16, device="cuda:0")
    weight = torch.zeros((10, 100), dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(SamplerError):
        sampler.lm_head(hidden, weight)  # H % 32 != 0
    hidden = torch.zeros((257, 64), dtype=torch.bfloat16, device="cuda:0")
    weight = torch.zeros((10, 64), dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(SamplerError, match="larger than the context"):
        sampler.lm_head(hidden, weight)  # more rows than the context's max_batch (256)
