"""numpy restatement of the reference KV path (test infrastructure; see oracle/__init__.py).

Arrays follow the reference layouts: caches (B, T_max, H_kv, D) per slot, q/out (B, T_new, H, D),
new k/v (B, T_new, H_kv, D), seqlens (B,) = each row's position before the new tokens.
The copy functions work on any dtype, including raw bit patterns (bf16 viewed as uint16), so
"bit-exact" is literal. Attention computes in float64 from float inputs (bf16 values widen to
float32 exactly before they get here).
"""
from __future__ import annotations

import numpy as np


def append(k_cache, v_cache, k, v, seqlens):
    """KV append at per-row positions; returns updated copies of the caches.

    modelcore/kernels/flash_attn.py:336-346: uniform rows take a slice assignment, ragged rows an
    index_put; both write k[b, t] to k_cache[b, seqlens[b] + t] and nothing else. A position past
    the cache raises, as the reference's indexing does.
    """
    kc, vc = np.array(k_cache, copy=True), np.array(v_cache, copy=True)
    B, T_new = k.shape[:2]
    T_max = kc.shape[1]
    for b in range(B):
        p = int(seqlens[b])
        if p < 0 or p + T_new > T_max:
            raise IndexError(f"row {b}: positions [{p}, {p + T_new}) outside cache of {T_max}")
        kc[b, p:p + T_new] = k[b]
        vc[b, p:p + T_new] = v[b]
    return kc, vc


def replicate(dst_k, dst_v, src_k, src_v, n_tokens, rows):
    """dst[s, r, :n_tokens] = src[s, 0, :n_tokens] for every slot s and r in rows.

    modelcore/cache.py:84-85 (prefill: all rows, a broadcast) and :106-107 (prefill_row: one row).
    Caches here carry the slot axis: (S, B, T, H_kv, D).
    """
    dk, dv = np.array(dst_k, copy=True), np.array(dst_v, copy=True)
    for r in rows:
        dk[:, r, :n_tokens] = src_k[:, 0, :n_tokens]
        dv[:, r, :n_tokens] = src_v[:, 0, :n_tokens]
    return dk, dv


def visible(seqlens, T_new, Tk, window):
    """(B, T_new, Tk) bool: may query t of row b see key col?

    Query t of row b sits at p = seqlens[b] + t; it sees col <= p, and when window >= 0 only
    p - col <= window. This is the ragged mask of modelcore/kernels/flash_attn.py:246-264, and
    the key set of the uniform paths (:217-235) as well.
    """
    p = np.asarray(seqlens, dtype=np.int64)[:, None] + np.arange(T_new)[None, :]
    col = np.arange(Tk)[None, None, :]
    keep = col <= p[:, :, None]
    if window is not None and window >= 0:
        keep &= (p[:, :, None] - col) <= window
    return keep


def attention(q, k_cache, v_cache, seqlens, window=-1, head_map=None, scale=None):
    """Masked softmax attention of q over the cache, float64: (B, T_new, H, D).

    modelcore/kernels/flash_attn.py:348-366: keys up to the furthest row's last new token, SDPA
    with enable_gqa (query head h reads KV head h // (H // H_kv)), scale 1/sqrt(D), the mask of
    `visible`. `head_map` and `scale` exist so tests can plant mistakes; leave them None.
    """
    q = np.asarray(q, dtype=np.float64)
    B, T_new, H, D = q.shape
    H_kv = k_cache.shape[2]
    G = H // H_kv
    Tk = int(np.max(seqlens)) + T_new
    if Tk > k_cache.shape[1]:
        raise IndexError(f"positions up to {Tk} exceed cache length {k_cache.shape[1]}")
    kk = np.asarray(k_cache[:, :Tk], dtype=np.float64)
    vv = np.asarray(v_cache[:, :Tk], dtype=np.float64)
    hm = np.arange(H) // G if head_map is None else np.asarray(head_map)
    kh, vh = kk[:, :, hm], vv[:, :, hm]  # (B, Tk, H, D)
    sc = (1.0 / np.sqrt(D)) if scale is None else scale
    # (B, H, T_new, D) @ (B, H, D, Tk) -> scores (B, H, T_new, Tk)
    s = np.matmul(q.transpose(0, 2, 1, 3), kh.transpose(0, 2, 3, 1)) * sc
    keep = visible(seqlens, T_new, Tk, window)[:, None]  # (B, 1, T_new, Tk)
    s = np.where(keep, s, -np.inf)
    s -= s.max(axis=-1, keepdims=True)
    p = np.where(keep, np.exp(s), 0.0)
    p /= p.sum(axis=-1, keepdims=True)
    # (B, H, T_new, Tk) @ (B, H, Tk, D) -> (B, H, T_new, D) -> (B, T_new, H, D)
    return np.matmul(p, vh.transpose(0, 2, 1, 3)).transpose(0, 2, 1, 3)


def flash_attn_with_kvcache(q, k_cache, v_cache, k, v, seqlens, window=-1):
    """Append (when k, v are given), then attention: (out, k_cache', v_cache').

    modelcore/kernels/flash_attn.py:306-366 (the SDPA fallback): the caches are updated, the
    positions in seqlens are not.
    """
    if k is not None:
        k_cache, v_cache = append(k_cache, v_cache, k, v, seqlens)
    return attention(q, k_cache, v_cache, seqlens, window), k_cache, v_cache

