"""Seeded synthetic sampling workloads (the five shapes of the benchmark configs).

Every array is a deterministic function of (config, seed), so the GPU path and
the CPU checker see identical inputs.  Logits are generated in f32 and, for bf16
configs, rounded to bf16 (round to nearest even); bf16 logits are stored as
their uint16 bit patterns.

  C1  B=1,   V=151,936 f32  N(0, 2.5^2) + 16 spikes +8..+14; 256-token history;
      rep 1.1, T 0.7, top_k 40, top_p 0.95 (and a greedy variant)
  C2  B=64,  V=151,936 bf16 N(0, 3^2) - 1.1 ln(rank) over a per-row permutation;
      T ~ U[0.3, 1.2], top_k in {0, 20, 50}, top_p ~ U[0.8, 1.0], min_p 0.05;
      1,024-token histories, presence 0.5, frequency 0.3
  C3  B=256, V=262,144 bf16 N(0, 4^2) + the same Zipf head; 2,048-token
      histories; rep 1.05, presence 0.5, frequency 0.3, T 1.0, top_k 64,
      top_p 0.95, min_p 0.02; Philox seed per row
  C4  B=128, V=151,936 f32  N(0, 3^2); allowed-token bitmask with density
      ~ U[5%, 60%]; 32 bias entries in U[-5, 5]; T 1.0, top_p 0.9
  C5  B=32, depth 3, V=151,936 bf16: target [B, 4, V] ~ N(0, 3^2), draft =
      target[:, :3] + N(0, 0.5^2); T 0.6, top_p 0.95 (draft ids are drawn from
      the draft law by the caller)

Histories mix uniform ids with ids drawn from the row's 64 highest-ranked ids
(one in four), so repeated and high-probability tokens are penalised.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from .params import PARAMS_DTYPE, AXS_NONE_U32

DTYPE_F32 = 0
DTYPE_BF16 = 1


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 → bf16, returned as uint16 bits."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


@dataclass
class Workload:
    name: str
    dtype: int
    B: int
    V: int
    logits: np.ndarray                 # [B, V] f32, or uint16 bf16 bits
    params: np.ndarray                 # PARAMS_DTYPE [B]
    hist: Optional[np.ndarray] = None  # uint32 flat
    hist_off: Optional[np.ndarray] = None  # int64 [B + 1]
    mask: Optional[np.ndarray] = None  # uint32 [B, ceil(V/32)]
    bias_ids: Optional[np.ndarray] = None
    bias_vals: Optional[np.ndarray] = None
    bias_off: Optional[np.ndarray] = None
    extra: dict = field(default_factory=dict)

    @property
    def esize(self) -> int:
        return 2 if self.dtype == DTYPE_BF16 else 4

    def logits_f32(self) -> np.ndarray:
        if self.dtype == DTYPE_BF16:
            return bf16_bits_to_f32(self.logits)
        return self.logits

    def algorithmic_bytes(self) -> int:
        """Each input read once: logits, histories, mask words, bias entries,
        plus the per-row params and the token ids written."""
        b = self.B * self.V * self.esize
        if self.hist is not None:
            b += int(self.hist_off[-1]) * 4
        if self.mask is not None:
            b += self.mask.size * 4
        if self.bias_ids is not None:
            b += int(self.bias_off[-1]) * 8
        b += self.B * (PARAMS_DTYPE.itemsize + 4)
        return b


def _zipf_head(rng: np.random.Generator, B: int, V: int, s: float = 1.1):
    """-s ln(rank) over a per-row random permutation of the ids; also returns
    the ids of the 64 highest ranks per row.  The permutation of row r is the
    affine bijection id -> (a_r * id + b_r) mod V with a_r coprime to V."""
    a = rng.integers(1, V, size=B, dtype=np.int64)
    for r in range(B):
        while np.gcd(int(a[r]), V) != 1:
            a[r] = (a[r] + 1) % V or 1
    b = rng.integers(0, V, size=B, dtype=np.int64)
    ids = np.arange(V, dtype=np.int64)
    rank0 = (a[:, None] * ids[None, :] + b[:, None]) % V  # 0-based rank of each id
    head = (-s * np.log((rank0 + 1).astype(np.float32))).astype(np.float32)
    # ids of ranks 0..63: invert the affine map with a_r^-1 mod V
    top = np.empty((B, 64), dtype=np.uint32)
    ks = np.arange(64, dtype=np.int64)
    for r in range(B):
        ainv = pow(int(a[r]), -1, V)
        top[r] = ((ks - b[r]) % V * ainv % V).astype(np.uint32)
    return head, top


def _histories(rng, B, V, H, hot):
    hist = rng.integers(0, V, size=(B, H), dtype=np.int64).astype(np.uint32)
    if hot is not None:
        pick = rng.random((B, H)) < 0.25
        hv = hot[np.arange(B)[:, None], rng.integers(0, hot.shape[1], size=(B, H))]
        hist = np.where(pick, hv, hist).astype(np.uint32)
    off = (np.arange(B + 1, dtype=np.int64) * H).astype(np.int64)
    return hist.reshape(-1), off


def _params(B, **kw):
    p = np.zeros(B, dtype=PARAMS_DTYPE)
    p["top_p"] = 1.0
    p["repetition_penalty"] = 1.0
    p["repetition_context_size"] = AXS_NONE_U32
    p["ngram_window"] = 128
    for k, v in kw.items():
        p[k] = v
    return p


def make_c1(seed: int = 1, greedy: bool = False) -> Workload:
    rng = np.random.default_rng([seed, 1])
    B, V = 1, 151936
    x = (rng.standard_normal((B, V), dtype=np.float32) * np.float32(2.5)).astype(np.float32)
    spikes = rng.choice(V, size=16, replace=False)
    x[0, spikes] += np.linspace(8.0, 14.0, 16, dtype=np.float32)
    hist, off = _histories(rng, B, V, 256, spikes[None, :].astype(np.uint32))
    p = _params(B, temperature=0.0 if greedy else 0.7, top_k=0 if greedy else 40,
                top_p=1.0 if greedy else 0.95, repetition_penalty=1.1,
                seed=seed * 1000003, step=7)
    return Workload("C1-greedy" if greedy else "C1", DTYPE_F32, B, V, x, p, hist, off)


def make_c2(seed: int = 2, B: int = 64, V: int = 151936) -> Workload:
    rng = np.random.default_rng([seed, 2])
    noise = rng.standard_normal((B, V), dtype=np.float32) * np.float32(3.0)
    head, top = _zipf_head(rng, B, V)
    x = f32_to_bf16_bits(noise + head)
    hist, off = _histories(rng, B, V, 1024, top)
    p = _params(B)
    p["temperature"] = rng.uniform(0.3, 1.2, B).astype(np.float32)
    p["top_k"] = rng.choice(np.array([0, 20, 50], dtype=np.uint32), B)
    p["top_p"] = rng.uniform(0.8, 1.0, B).astype(np.float32)
    p["has_min_p"] = 1
    p["min_p"] = 0.05
    p["presence_penalty"] = 0.5
    p["frequency_penalty"] = 0.3
    p["seed"] = seed * 7919 + np.arange(B, dtype=np.uint64)
    p["step"] = 11
    return Workload("C2", DTYPE_BF16, B, V, x, p, hist, off)


def make_c3(seed: int = 3, B: int = 256, V: int = 262144) -> Workload:
    rng = np.random.default_rng([seed, 3])
    noise = rng.standard_normal((B, V), dtype=np.float32) * np.float32(4.0)
    head, top = _zipf_head(rng, B, V)
    x = f32_to_bf16_bits(noise + head)
    del noise, head
    hist, off = _histories(rng, B, V, 2048, top)
    p = _params(B, temperature=1.0, top_k=64, top_p=0.95, has_min_p=1, min_p=0.02,
                repetition_penalty=1.05, presence_penalty=0.5, frequency_penalty=0.3, step=5)
    p["seed"] = seed * 104729 + np.arange(B, dtype=np.uint64)
    return Workload("C3", DTYPE_BF16, B, V, x, p, hist, off)


def make_c4(seed: int = 4, B: int = 128, V: int = 151936) -> Workload:
    rng = np.random.default_rng([seed, 4])
    x = (rng.standard_normal((B, V), dtype=np.float32) * np.float32(3.0)).astype(np.float32)
    W = (V + 31) // 32
    dens = rng.uniform(0.05, 0.60, B)
    allowed = rng.random((B, V)) < dens[:, None]
    bits = np.zeros((B, W * 32), dtype=bool)
    bits[:, :V] = allowed
    # bit (t & 31) of word t >> 5, least significant bit = lowest id
    words = np.ascontiguousarray(np.packbits(bits, axis=1, bitorder="little").view("<u4"))
    bias_ids = np.stack([rng.choice(V, 32, replace=False) for _ in range(B)]).astype(np.uint32)
    bias_vals = rng.uniform(-5.0, 5.0, (B, 32)).astype(np.float32)
    boff = (np.arange(B + 1, dtype=np.int64) * 32).astype(np.int64)
    p = _params(B, temperature=1.0, top_p=0.9, step=3)
    p["seed"] = seed * 15485863 + np.arange(B, dtype=np.uint64)
    w = Workload("C4", DTYPE_F32, B, V, x, p, mask=words, bias_ids=bias_ids.reshape(-1),
                 bias_vals=bias_vals.reshape(-1), bias_off=boff)
    w.extra["allowed"] = allowed
    return w


def make_c5(seed: int = 5, B: int = 32, depth: int = 3, V: int = 151936):
    """Returns (target bf16 bits [B, D+1, V], draft bf16 bits [B, D, V],
    target params, draft params)."""
    rng = np.random.default_rng([seed, 5])
    t = rng.standard_normal((B, depth + 1, V), dtype=np.float32) * np.float32(3.0)
    d = t[:, :depth, :] + rng.standard_normal((B, depth, V), dtype=np.float32) * np.float32(0.5)
    tp = _params(B, temperature=0.6, top_p=0.95, step=9)
    tp["seed"] = seed * 32452843 + np.arange(B, dtype=np.uint64)
    dp = _params(B, temperature=0.6, top_p=0.95, step=9)
    dp["seed"] = seed * 49979687 + np.arange(B, dtype=np.uint64)
    return f32_to_bf16_bits(t), f32_to_bf16_bits(d), tp, dp


def make_mixed(seed: int, B: int, V: int, dtype: int = DTYPE_BF16, hist_len: int = 512,
               mask: bool = False, bias: bool = False, ngram: bool = False,
               edge_rows: bool = True) -> Workload:
    """Every row law at once, for parity tests of the routing and the edge cases.

    Rows cycle through greedy, index-order (no filter), min-p only, min-p +
    top-k + top-p, top-k, top-p, top_p <= 0 (sorted, untruncated) and a near-zero
    temperature; penalties, window sizes and history lengths vary per row.
    Optional: an allowed-token mask (densities 1%..100%, some rows all-allowed),
    bias lists with duplicate ids and ids outside the vocabulary, and the
    no-repeat n-gram ban.  With edge_rows, a few rows are all-equal, hold NaNs,
    are all -inf but one id, or are all NaN."""
    rng = np.random.default_rng([seed, 77, B, V])
    noise = rng.standard_normal((B, V), dtype=np.float32) * np.float32(3.0)
    if V >= 2:
        head, top = _zipf_head(rng, B, V)
    else:
        head, top = np.zeros((B, V), np.float32), np.zeros((B, 64), np.uint32)
    x = (noise + head).astype(np.float32)
    if edge_rows and B >= 8:
        x[1, :] = 1.5                       # all equal: every tie goes to the lowest id
        x[2, rng.choice(V, max(1, V // 7), replace=False)] = np.nan
        x[3, :] = -np.inf
        x[3, V // 3] = 0.25
        x[4, :] = np.nan
        x[5, V - 1] = 60.0                  # maximum at the last id
        x[6, 0] = 60.0                      # and at the first
    logits = f32_to_bf16_bits(x) if dtype == DTYPE_BF16 else x
    # histories of varied length (some empty), a quarter of the tokens hot
    lens = rng.integers(0, hist_len + 1, size=B)
    lens[::9] = 0
    hs = []
    for r in range(B):
        h = rng.integers(0, V, size=lens[r], dtype=np.int64).astype(np.uint32)
        pick = rng.random(lens[r]) < 0.25
        h[pick] = top[r, rng.integers(0, 64, size=int(pick.sum()))]
        hs.append(h)
    off = np.zeros(B + 1, dtype=np.int64)
    off[1:] = np.cumsum(lens)
    hist = np.concatenate(hs).astype(np.uint32) if off[-1] else np.zeros(1, np.uint32)
    p = _params(B)
    laws = [
        dict(temperature=0.0),
        dict(temperature=0.8),
        dict(temperature=0.9, has_min_p=1, min_p=0.05),
        dict(temperature=1.0, has_min_p=1, min_p=0.02, top_k=64, top_p=0.95),
        dict(temperature=0.7, top_k=40),
        dict(temperature=1.1, top_p=0.9),
        dict(temperature=0.6, top_p=0.0),
        dict(temperature=1e-3, top_k=5, top_p=0.9),
        dict(temperature=1.3, has_min_p=1, min_p=0.1, top_p=0.8),
    ]
    for r in range(B):
        for k, v in laws[r % len(laws)].items():
            p[r][k] = v
    p["repetition_penalty"] = rng.choice(np.array([1.0, 1.05, 1.3, 0.8], np.float32), B)
    p["presence_penalty"] = rng.choice(np.array([0.0, 0.5, -0.25], np.float32), B)
    p["frequency_penalty"] = rng.choice(np.array([0.0, 0.3], np.float32), B)
    ctx = rng.choice(np.array([AXS_NONE_U32, 16, 64, 0], np.uint32), B)
    p["repetition_context_size"] = ctx
    if ngram:
        p["no_repeat_ngram_size"] = rng.choice(np.array([0, 2, 3], np.uint32), B)
        p["ngram_window"] = rng.choice(np.array([32, 128, 1000], np.uint32), B)
    p["seed"] = seed * 2654435761 + np.arange(B, dtype=np.uint64)
    p["step"] = 13
    w = Workload(f"mixed{B}x{V}", dtype, B, V, logits, p, hist, off)
    if mask:
        W = (V + 31) // 32
        dens = rng.choice(np.array([0.01, 0.05, 0.3, 0.6, 1.0]), B)
        allowed = rng.random((B, V)) < dens[:, None]
        allowed[:, top[:, 0] % V] |= False
        bits = np.zeros((B, W * 32), dtype=bool)
        bits[:, :V] = allowed
        w.mask = np.ascontiguousarray(np.packbits(bits, axis=1, bitorder="little").view("<u4"))
        w.extra["allowed"] = allowed
    if bias:
        nb = rng.integers(0, 41, size=B)
        ids, vals = [], []
        for r in range(B):
            t = rng.choice(top[r], size=nb[r] // 2).astype(np.int64)       # hot ids
            u = rng.integers(0, V, size=nb[r] - nb[r] // 2, dtype=np.int64)
            e = np.concatenate([t, u])
            if nb[r] >= 4:
                e[-1] = e[0]                      # a duplicate (applied twice, in order)
                e[-2] = V + 5                     # outside the vocabulary (ignored)
            ids.append(e.astype(np.uint32))
            vals.append(rng.uniform(-6.0, 6.0, size=nb[r]).astype(np.float32))
        boff = np.zeros(B + 1, dtype=np.int64)
        boff[1:] = np.cumsum(nb)
        w.bias_ids = np.concatenate(ids).astype(np.uint32) if boff[-1] else np.zeros(1, np.uint32)
        w.bias_vals = np.concatenate(vals).astype(np.float32) if boff[-1] else np.zeros(1, np.float32)
        w.bias_off = boff
    return w


MAKERS = {"C1": make_c1, "C2": make_c2, "C3": make_c3, "C4": make_c4}
