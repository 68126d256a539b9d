"""The reference's CPU fallback for the KV path, restated with the same torch operations
(test infrastructure and CPU baseline; see oracle/__init__.py).

* ``flash_attn_with_kvcache`` follows modelcore/kernels/flash_attn.py:330-366: one host read of
  cache_seqlens; append by slice assignment (uniform rows) or index_put (ragged rows); keys up to
  the furthest row; ``scaled_dot_product_attention`` with ``enable_gqa`` -- sliced and unmasked
  for a uniform single token (:217-224), causal for a uniform full prompt (:213-215), an explicit
  (Tq, Tk) mask for uniform chunks (:226-244), a (B, 1, T_new, Tk) mask when ragged (:246-264).
* ``flash_attn_func`` follows the no-cache fallback (modelcore/kernels/flash_attn.py:270-303
  without FA3 or document masks): transpose to (B, H, T, D), then the same uniform helper.
* ``flash_attn_varlen_with_kvcache`` is the varlen (packed prompts) form: the operator above run
  once per sequence on its own cache row, as the reference prefills each prompt alone
  (modelcore/generate.py:67-80).
* ``replicate`` follows KVCache.prefill's broadcast copy (modelcore/cache.py:84-85).
* ``flash_attn`` is the operator namespace of the two functions, for model code that takes one.
"""
from __future__ import annotations

from types import SimpleNamespace

import torch
import torch.nn.functional as F


def _uniform_attention(q, k, v, window, enable_gqa):
    """(B, H, Tq, D) x (B, H_kv, Tk, D), every row at the same position."""
    Tq, Tk = q.size(2), k.size(2)
    if (window < 0 or window >= Tq) and Tq == Tk:
        return F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=enable_gqa)
    if Tq == 1:
        if 0 <= window < Tk:
            first = max(0, Tk - (window + 1))  # the last window + 1 keys
            k, v = k[:, :, first:], v[:, :, first:]
        return F.scaled_dot_product_attention(q, k, v, is_causal=False, enable_gqa=enable_gqa)
    q_pos = (Tk - Tq) + torch.arange(Tq).unsqueeze(1)
    col = torch.arange(Tk).unsqueeze(0)
    keep = col <= q_pos
    if 0 <= window < Tk:
        keep &= (q_pos - col) <= window
    return F.scaled_dot_product_attention(q, k, v, attn_mask=keep, enable_gqa=enable_gqa)


def _ragged_mask(cache_seqlens, T_new, Tk, window):
    q_pos = cache_seqlens.to(torch.long).unsqueeze(1) + torch.arange(T_new)  # (B, T_new)
    col = torch.arange(Tk).view(1, 1, Tk)
    keep = col <= q_pos.unsqueeze(2)
    if 0 <= window < Tk:
        keep &= (q_pos.unsqueeze(2) - col) <= window
    return keep.unsqueeze(1)


def flash_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None, cache_seqlens=None,
                            window_size=(-1, -1), force_ragged=False, causal=True):
    """CPU fallback of the operator: in-place append into k_cache/v_cache, returns (B, T_new, H, D)."""
    B, T_new, H, D = q.shape
    positions = cache_seqlens.tolist()
    lo, hi = min(positions), max(positions)
    ragged = force_ragged or lo != hi
    if k is not None and v is not None:
        if ragged:
            rows = torch.arange(B).unsqueeze(1)
            cols = cache_seqlens.to(torch.long).unsqueeze(1) + torch.arange(T_new)
            k_cache[rows, cols] = k
            v_cache[rows, cols] = v
        else:
            k_cache[:, lo:lo + T_new] = k
            v_cache[:, lo:lo + T_new] = v
    Tk = hi + T_new
    qs = q.transpose(1, 2)
    ks = k_cache[:, :Tk].transpose(1, 2)
    vs = v_cache[:, :Tk].transpose(1, 2)
    gqa = qs.size(1) != ks.size(1)
    window = window_size[0]
    if ragged:
        keep = _ragged_mask(cache_seqlens, T_new, Tk, window)
        y = F.scaled_dot_product_attention(qs, ks, vs, attn_mask=keep, enable_gqa=gqa)
    else:
        y = _uniform_attention(qs, ks, vs, window, gqa)
    return y.transpose(1, 2)


def flash_attn_func(q, k, v, causal=True, window_size=(-1, -1), doc_args=None):
    """No-cache causal attention, (B, T, H, D) in and out."""
    assert doc_args is None
    qs, ks, vs = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    y = _uniform_attention(qs, ks, vs, window_size[0], qs.size(1) != ks.size(1))
    return y.transpose(1, 2)


def flash_attn_varlen_with_kvcache(q, k_cache, v_cache, k=None, v=None, cache_seqlens=None,
                                   cu_seqlens=None, max_seqlen=None, rows=None, causal=True,
                                   window_size=(-1, -1), advance=False):
    """Several sequences packed along one token axis, each appended and attended in its own
    cache row: sequence b is tokens [cu_seqlens[b], cu_seqlens[b + 1]) of q (total, H, D) and k/v
    (total, H_kv, D), in row rows[b] (b when None). The reference prefills each prompt alone and
    copies it into its row (modelcore/generate.py:67-80, modelcore/cache.py:92-119); this runs
    the fallback above once per sequence on that row, which is the same arithmetic. With
    `advance`, each row's position then moves on by its sequence's length."""
    cu = [int(x) for x in cu_seqlens.tolist()]
    n = len(cu) - 1
    rows = list(range(n)) if rows is None else [int(r) for r in rows.tolist()]
    outs = []
    for b in range(n):
        r, a, e = rows[b], cu[b], cu[b + 1]
        kb = None if k is None else k[a:e].unsqueeze(0)
        vb = None if v is None else v[a:e].unsqueeze(0)
        y = flash_attn_with_kvcache(q[a:e].unsqueeze(0), k_cache[r:r + 1], v_cache[r:r + 1], kb,
                                    vb, cache_seqlens[r:r + 1], window_size)
        outs.append(y[0])
    if advance:
        for b in range(n):
            cache_seqlens[rows[b]] += cu[b + 1] - cu[b]
    return torch.cat(outs, 0) if outs else q.new_empty((0,) + tuple(q.shape[1:]))


flash_attn = SimpleNamespace(flash_attn_func=flash_attn_func,
                             flash_attn_with_kvcache=flash_attn_with_kvcache,
                             flash_attn_varlen_with_kvcache=flash_attn_varlen_with_kvcache)


def replicate(dst_k, dst_v, src_k, src_v, n_tokens):
    """Broadcast row 0 of a (S, 1, T, H_kv, D) source into every row of (S, B, T', H_kv, D)."""
    dst_k[:, :, :n_tokens] = src_k[:, :, :n_tokens]
    dst_v[:, :, :n_tokens] = src_v[:, :, :n_tokens]


def replicate_rows(dst, src, row_begin, n_rows, n_tokens, src_row=0):
    """KVCache-level copy of row `src_row`, positions [0, n_tokens), of every slot of `src` into
    rows [row_begin, row_begin + n_rows) of `dst` (modelcore/cache.py:84-85 and :106-107); the
    same argument meaning as modelcore_amd.cache.KVCache._replicate_from, for CPU caches."""
    rows = slice(row_begin, row_begin + n_rows)
    dst.k_cache[:, rows, :n_tokens] = src.k_cache[:, src_row:src_row + 1, :n_tokens]
    dst.v_cache[:, rows, :n_tokens] = src.v_cache[:, src_row:src_row + 1, :n_tokens]
