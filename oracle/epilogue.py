"""The reference's pre-attention step, restated with the same torch operations on the CPU (test
infrastructure; see oracle/__init__.py).

For a producer attention layer with a cache (modelcore/components/attention.py:143-150):
  * RoPE at the rows' positions: the uniform window ``cos[:, T0:T0 + T]`` or, for a ragged
    cache, the per-row gather of positions ``cache_seqlens[b] + t``
    (modelcore/components/rotary.py:50-67), then ``apply_rotary_emb``
    (modelcore/components/rope.py:4-12): ``[x1 * cos + x2 * sin, x1 * (-sin) + x2 * cos]`` on
    the two halves of the head dim, each op a separate torch op in the storage dtype;
  * the QK norm ``F.rms_norm(x, (D,), eps=eps)`` (modelcore/components/norm.py:43-44);
  * ``x * 1.2`` (attention.py:149-150);
  * the append of k and v at the same positions (modelcore/kernels/flash_attn.py:336-346).
A KV-sharing consumer applies the first three to q only (attention.py:155-157).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _windows(cos, sin, seqlens, T):
    """(B, T, 1, D/2) cos/sin at positions seqlens[b] + t; ``cos``/``sin`` reshape to
    (n_pos, D/2)."""
    half = cos.shape[-1]
    c, s = cos.reshape(-1, half), sin.reshape(-1, half)
    pos = seqlens.to(torch.long)[:, None] + torch.arange(T)  # (B, T)
    assert int(pos.max()) < c.size(0), "position beyond the rotary table"
    B = pos.size(0)
    return (c.index_select(0, pos.reshape(-1)).view(B, T, 1, half),
            s.index_select(0, pos.reshape(-1)).view(B, T, 1, half))


def apply_rotary(x, cos, sin):
    """modelcore/components/rope.py:4-12."""
    d = x.shape[3] // 2
    x1, x2 = x[..., :d], x[..., d:]
    return torch.cat([x1 * cos + x2 * sin, x1 * (-sin) + x2 * cos], 3)


def rope_norm_scale(x, cos, sin, seqlens, eps=None, scale=1.2):
    """RoPE at positions seqlens[b] + t, then RMS-norm over D, then the scale."""
    c, s = _windows(cos, sin, seqlens, x.size(1))
    y = apply_rotary(x, c, s)
    y = F.rms_norm(y, (y.size(-1),), eps=eps)
    return y * scale


def rope_norm_scale_append(q, cos, sin, seqlens, k=None, v=None, k_cache=None, v_cache=None,
                           eps=None, scale=1.2):
    """The whole step: returns q's result and writes k's result and v into the caches (CPU
    tensors, updated in place) at seqlens[b] + t."""
    q_out = rope_norm_scale(q, cos, sin, seqlens, eps, scale)
    if k is not None:
        k_out = rope_norm_scale(k, cos, sin, seqlens, eps, scale)
        for b in range(q.size(0)):
            p = int(seqlens[b])
            k_cache[b, p:p + k.size(1)] = k_out[b]
            v_cache[b, p:p + v.size(1)] = v[b]
    return q_out
