"""The step before the cached-attention operator, fused into one HIP launch: RoPE at each token's
cache position, QK RMS-norm, the x1.2 scale, and the append of the new K/V.

It replaces, in an attention layer's forward (modelcore/components/attention.py:143-150 for
producer layers, :155-157 for KV-sharing consumers), the calls

    q, k = rope(q, k, kv_cache)          # modelcore/components/rotary.py:69-81, rope.py:4-12
    q, k = norm(q), norm(k)              # modelcore/components/norm.py:43-44 (F.rms_norm)
    q, k = q * 1.2, k * 1.2
    ... flash_attn_with_kvcache(..., k=k, v=v, ...)   # its append half, flash_attn.py:336-346

with ``q = rope_norm_scale_append(q, cos, sin, cache_seqlens, k, v, k_cache, v_cache)`` followed
by the operator with ``k = v = None``. Positions are read from ``cache_seqlens`` on the device
(p = cache_seqlens[b] + t), so the call never syncs the host and can sit in a captured graph.

Numerics: every rotation product and sum is rounded to the storage dtype as the separate torch
ops round them, the norm runs in fp32 like ``F.rms_norm`` (which upcasts reduced-precision
inputs and, for ``eps=None``, adds float32's epsilon), and the scale is one fp32 multiply
rounded to the storage dtype. The order of the fp32 sum of squares is the only difference from
the unfused ops: results agree within one unit in the last place of the storage dtype.
"""
from __future__ import annotations

import torch

from modelcore_amd import _ext

__all__ = ["rope_norm_scale_append", "rope_norm_scale_append_partials", "default_eps"]


def default_eps() -> float:
    """The epsilon ``F.rms_norm(x, eps=None)`` adds: float32's, for fp32 and reduced-precision
    inputs alike (the computation is upcast to fp32 before the epsilon is chosen)."""
    return float(torch.finfo(torch.float32).eps)


def _table(t: torch.Tensor, half: int, dt: torch.dtype, device) -> torch.Tensor:
    if t.dtype != dt:
        raise TypeError(f"rotary table is {t.dtype}, q is {dt}")
    if t.device != device:
        raise ValueError(f"rotary table is on {t.device}, q on {device}")
    if t.shape[-1] != half or t.numel() % half != 0:
        raise ValueError(f"rotary table must end in head_dim/2 = {half}; got {tuple(t.shape)}")
    return t.reshape(-1, half).contiguous()


def _token_rows(t: torch.Tensor) -> tuple[torch.Tensor, int]:
    """t (B, T, heads, D) with heads and D contiguous and tokens evenly strided (a view of a fused
    projection's output qualifies), and the token stride in elements; else a contiguous copy."""
    B, T, Hh, D = t.shape
    # With one token per row its stride is meaningless (torch's views give the size-1 dim any
    # stride): tokens are then rows, stride(0) apart.
    tok = t.stride(1) if T > 1 else t.stride(0)
    if t.stride(3) == 1 and t.stride(2) == D and (B == 1 or t.stride(0) == T * tok) \
            and tok >= Hh * D:
        return t, tok
    t = t.contiguous()
    return t, Hh * D


def rope_norm_scale_append(q, cos, sin, cache_seqlens, k=None, v=None, k_cache=None,
                           v_cache=None, eps=None, scale=1.2):
    """RoPE + RMS-norm + scale of q (returned) and, when given, of k, which is appended with v.

    Args:
        q: (B, T, H, D) queries, bf16 or fp32; q, k and v may be strided views of one fused
            projection (heads contiguous, tokens evenly strided), read in place.
        cos, sin: rotary tables that reshape to (n_pos, D/2) in q's dtype -- the
            (1, n_pos, 1, D/2) buffers of the rotary module.
        cache_seqlens: (B,) int32, each row's position before these tokens (read only).
        k, v: (B, T, H_kv, D) new keys/values, or both None (transform q only).
        k_cache, v_cache: (B, T_max, H_kv, D) caches (a slot view), updated in place at
            cache_seqlens[b] + t.
        eps: RMS-norm epsilon; None is ``F.rms_norm``'s default (see ``default_eps``).
        scale: multiplier after the norm (1.2 in the model).
    """
    _ext.require_rocm(q, k, v, k_cache, v_cache, cache_seqlens, what="rope_norm_scale_append")
    if q.dim() != 4:
        raise ValueError(f"q must be (B, T, H, D); got {tuple(q.shape)}")
    B, T, H, D = q.shape
    if D % 2:
        raise ValueError(f"head_dim must be even for RoPE; got {D}")
    dt = q.dtype
    code = _ext.dtype_code(dt)
    half = D // 2
    cos_t, sin_t = _table(cos, half, dt, q.device), _table(sin, half, dt, q.device)
    if cos_t.shape != sin_t.shape:
        raise ValueError(f"cos {tuple(cos_t.shape)} and sin {tuple(sin_t.shape)} differ")
    if (k is None) != (v is None):
        raise ValueError("pass both k and v, or neither")
    seqlens = cache_seqlens
    if seqlens.dtype != torch.int32 or seqlens.shape != (B,) or seqlens.device != q.device:
        raise ValueError(f"cache_seqlens must be ({B},) int32 on {q.device}")
    seqlens = seqlens.contiguous()
    H_kv, T_max, cb = 1, 0, 0
    if k is not None:
        if k.dim() != 4 or k.shape != v.shape or k.shape[0] != B or k.shape[1] != T \
                or k.shape[3] != D:
            raise ValueError(f"k/v must be (B, T, H_kv, D) = ({B}, {T}, H_kv, {D}); got "
                             f"{tuple(k.shape)} and {tuple(v.shape)}")
        H_kv = k.shape[2]
        if H % H_kv:
            raise ValueError(f"n_head {H} is not a multiple of n_kv_head {H_kv}")
        if k_cache is None or v_cache is None or k_cache.shape != v_cache.shape \
                or k_cache.dim() != 4 or k_cache.shape[0] != B or k_cache.shape[2:] != (H_kv, D):
            raise ValueError(f"k_cache/v_cache must be (B, T_max, H_kv, D) = ({B}, T_max, {H_kv}, "
                             f"{D})")
        for name, t in (("k", k), ("v", v), ("k_cache", k_cache), ("v_cache", v_cache)):
            if t.dtype != dt:
                raise TypeError(f"{name} is {t.dtype}, q is {dt}")
        if k_cache.stride() != v_cache.stride() or not k_cache[0].is_contiguous() \
                or not v_cache[0].is_contiguous():
            raise ValueError("each row of k_cache/v_cache must be contiguous (T_max, H_kv, D), "
                             "with equal strides")
        T_max, cb = k_cache.shape[1], k_cache.stride(0)
        (k, ks), (v, vs) = _token_rows(k), _token_rows(v)
    else:
        ks = vs = 0
    q, qs = _token_rows(q)
    out = torch.empty((B, T, H, D), dtype=dt, device=q.device)
    eps = default_eps() if eps is None else float(eps)
    st = _ext.lib().mcamd_qk_rope_norm_append(
        q.data_ptr(), qs, k.data_ptr() if k is not None else None, ks,
        v.data_ptr() if v is not None else None, vs, cos_t.data_ptr(), sin_t.data_ptr(),
        cos_t.shape[0], k_cache.data_ptr() if k is not None else None,
        v_cache.data_ptr() if k is not None else None, seqlens.data_ptr(), out.data_ptr(), B, T,
        H, H_kv, D, T_max, cb, eps, float(scale), code, _ext.stream_handle(q.device))
    _ext.check(st, "rope_norm_scale_append")
    return out


def rope_norm_scale_append_partials(qkv, n_head, n_kv_head, cos, sin, cache_seqlens,
                                    k_cache=None, v_cache=None, eps=None, scale=1.2):
    """rope_norm_scale_append for bf16, with q, k, v taken from the unsummed K-split partials of
    the stacked QKV projection (``qkv``: a ``linear.Partials`` of shape (B, T, (H + 2 H_kv) D),
    or (B, T, H D) with no caches: q only). Each value is the in-order sum of the partials rounded
    to bf16 -- the projection's own output -- so the result is that of rope_norm_scale_append on
    the summed projection, without its separate reduce pass. Returns q (B, T, H, D) bf16."""
    from modelcore_amd.kernels.linear import Partials
    if not isinstance(qkv, Partials):
        raise TypeError("qkv must be the Partials of the stacked QKV projection")
    part = qkv.part
    _ext.require_rocm(part, k_cache, v_cache, cache_seqlens, what="rope_norm_scale_append_partials")
    B, T, n = qkv.shape
    with_kv = k_cache is not None
    D = n // (n_head + (2 * n_kv_head if with_kv else 0))
    if D * (n_head + (2 * n_kv_head if with_kv else 0)) != n or D % 2:
        raise ValueError(f"a row of {n} is not (H + 2 H_kv) * D with even D for H={n_head}, "
                         f"H_kv={n_kv_head}")
    if part.dtype != torch.float32 or part.shape != (qkv.splits, B * T, n) \
            or not part.is_contiguous():
        raise ValueError("partials must be contiguous (splits, B*T, n) fp32")
    half = D // 2
    dt = torch.bfloat16
    cos_t, sin_t = _table(cos, half, dt, part.device), _table(sin, half, dt, part.device)
    if cache_seqlens.dtype != torch.int32 or cache_seqlens.shape != (B,):
        raise ValueError(f"cache_seqlens must be ({B},) int32")
    T_max, cb = 0, 0
    if with_kv:
        if k_cache.shape != v_cache.shape or k_cache.dim() != 4 or k_cache.shape[0] != B \
                or k_cache.shape[2:] != (n_kv_head, D) or k_cache.dtype != dt \
                or v_cache.dtype != dt:
            raise ValueError(f"k_cache/v_cache must be (B, T_max, H_kv, D) = ({B}, T_max, "
                             f"{n_kv_head}, {D}) bf16")
        if k_cache.stride() != v_cache.stride() or not k_cache[0].is_contiguous():
            raise ValueError("each row of k_cache/v_cache must be contiguous, with equal strides")
        T_max, cb = k_cache.shape[1], k_cache.stride(0)
    out = torch.empty((B, T, n_head, D), dtype=dt, device=part.device)
    st = _ext.lib().mcamd_qk_rope_norm_append_partials(
        part.data_ptr(), qkv.splits, n, cos_t.data_ptr(), sin_t.data_ptr(), cos_t.shape[0],
        k_cache.data_ptr() if with_kv else None, v_cache.data_ptr() if with_kv else None,
        cache_seqlens.contiguous().data_ptr(), out.data_ptr(), B, T, n_head, n_kv_head, D, T_max,
        cb, default_eps() if eps is None else float(eps), float(scale), int(with_kv),
        _ext.stream_handle(part.device))
    _ext.check(st, "rope_norm_scale_append_partials")
    return out
