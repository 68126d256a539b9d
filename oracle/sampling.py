"""numpy restatement of the device sampler (test infrastructure; see oracle/__init__.py).

Philox4x32-10 is the counter-based generator of Salmon, Moraes, Dror and Shaw ("Parallel random
numbers: as easy as 1, 2, 3", SC 2011), restated from the paper; `philox4x32_10` is pinned by the
known-answer vectors published with that paper's Random123 library (tests/test_sampling_host.py).
`sample` restates the Gumbel-max draw the device kernel makes: row b, offset o, token i takes
word i % 4 of Philox(counter = (i // 4, o low, o high, 0), key = seed_b low/high), uniform
u = ((x >> 9) + 1/2) / 2^23, score = logit / T - log(-log(u)); the draw is the first index of the
maximum. It is the reference's softmax(logits / T) sampling (modelcore/generate.py:18-34) in
Gumbel-max form, with a per-row counter-based stream in place of torch.multinomial's generator.
With top_k, only the k largest logits take part (`top_k_mask`: ties at the k-th value kept lowest
index first), the reference's top_k branch (generate.py:23-29: torch.topk, then the draw over the
kept values).
"""
from __future__ import annotations

import numpy as np

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = 0x9E3779B9, 0xBB67AE85
MASK = np.uint64(0xFFFFFFFF)


def philox4x32_10(ctr, key):
    """ctr: (..., 4) uint32, key: (..., 2) uint32 -> (..., 4) uint32."""
    c = [np.asarray(ctr[..., j], dtype=np.uint64) for j in range(4)]
    k0 = np.asarray(key[..., 0], dtype=np.uint64)
    k1 = np.asarray(key[..., 1], dtype=np.uint64)
    for _ in range(10):
        p0 = M0 * c[0]
        p1 = M1 * c[2]
        hi0, lo0 = p0 >> np.uint64(32), p0 & MASK
        hi1, lo1 = p1 >> np.uint64(32), p1 & MASK
        c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
        k0 = (k0 + np.uint64(W0)) & MASK
        k1 = (k1 + np.uint64(W1)) & MASK
    return np.stack(c, axis=-1).astype(np.uint32)


def uniforms(seed, offset, vocab):
    """The (vocab,) float64 uniforms row `seed` uses at `offset` (each is exactly a float32)."""
    g = np.arange((vocab + 3) // 4, dtype=np.uint64)
    ctr = np.zeros((g.size, 4), dtype=np.uint64)
    ctr[:, 0] = g
    ctr[:, 1] = np.uint64(offset) & MASK
    ctr[:, 2] = np.uint64(offset) >> np.uint64(32)
    key = np.zeros((g.size, 2), dtype=np.uint64)
    key[:, 0] = np.uint64(seed) & MASK
    key[:, 1] = np.uint64(seed) >> np.uint64(32)
    words = philox4x32_10(ctr, key).reshape(-1)[:vocab].astype(np.uint64)
    return ((words >> np.uint64(9)).astype(np.float64) + 0.5) / 8388608.0


def top_k_mask(logits, top_k):
    """(V,) bool: the top_k largest logits of the row, ordered by value then by lowest index (NaN
    after -inf, -0 equal to +0); all of them when top_k is None, <= 0 or >= V."""
    logits = np.asarray(logits, dtype=np.float64)
    V = logits.size
    keep = np.zeros(V, dtype=bool)
    if top_k is None or top_k <= 0 or top_k >= V:
        keep[:] = True
        return keep
    key = np.where(np.isnan(logits), -np.inf, logits)
    nan = np.isnan(logits)
    order = np.lexsort((np.arange(V), nan, -key))  # value descending, NaN last, then index
    keep[order[:top_k]] = True
    return keep


def scores(logits, seed, offset, temperature, top_k=None):
    """Gumbel-perturbed scores of one row, float64 (-inf outside the top_k set)."""
    logits = np.asarray(logits, dtype=np.float64)
    if temperature == 0:
        return logits
    u = uniforms(seed, offset, logits.size)
    s = logits / temperature - np.log(-np.log(u))
    return np.where(top_k_mask(logits, top_k), s, -np.inf)


def sample(logits, seeds, offsets, temperature, top_k=None):
    """(B,) token ids for (B, V) logits; returns (ids, margins) where a margin is the gap between
    the best and second-best score of the row (a device float32 evaluation can only differ from
    this float64 one when the gap is within rounding)."""
    logits = np.asarray(logits, dtype=np.float64)
    ids, margins = [], []
    for b in range(logits.shape[0]):
        s = scores(logits[b], int(seeds[b]), int(offsets[b]), temperature, top_k)
        order = np.argsort(-s, kind="stable")
        ids.append(int(order[0]))
        margins.append(float(s[order[0]] - s[order[1]]) if s.size > 1 else np.inf)
    return np.array(ids), np.array(margins)
