"""Drop-in for ``modelcore.kernels.flash_attn``: the FA3-style operator namespace, backed by the
hand-written gfx950 HIP kernels of ``modelcore_amd`` (C ABI in ``include/modelcore_amd.h``).

Usage is the reference's (modelcore/kernels/flash_attn.py:7-14)::

    from modelcore_amd.kernels.flash_attn import flash_attn
    y = flash_attn.flash_attn_with_kvcache(q, k_cache, v_cache, k=k, v=v,
                                           cache_seqlens=cache.cache_seqlens,
                                           causal=True, window_size=(window, 0))

Semantics are the reference fallback's (modelcore/kernels/flash_attn.py:330-366): the new
tokens' K/V are written in place at ``cache_seqlens`` (which is read, and advanced only when the
call asks for it with ``advance``), and query
t of row b, at position p = cache_seqlens[b] + t, attends keys col <= p with p - col <=
window_size[0] when that is >= 0. GQA maps query head h to KV head h // (H // H_kv). The softmax
scale is 1/sqrt(D). Uniform and ragged ``cache_seqlens`` run the same kernels (the reference's
uniform slice and ragged mask select the same keys), so there is no host sync on cache_seqlens.

Tensors must be on a ROCm device; there is no CPU or SDPA path. The module keeps the reference's
switch names (``_override_impl``, ``USE_FA3``, ``HAS_FA3``, ``FA3_LOAD_ERROR``, ``_force_ragged``)
so code and tests that set them keep working; they select nothing here.
"""
from __future__ import annotations

import os
from types import SimpleNamespace

import torch

from modelcore_amd import _ext

# -----------------------------------------------------------------------------------------------
# Backend switch, kept for signature parity with modelcore/kernels/flash_attn.py:64-93.
# -----------------------------------------------------------------------------------------------
_fa3 = None
FA3_LOAD_ERROR = "FA3 is a CUDA binary; this build runs hand-written HIP kernels on gfx950"
HAS_FA3 = False
IMPL = "hip-gfx950"
_override_impl = None


def _resolve_use_fa3():
    """Mirror of the reference resolver (modelcore/kernels/flash_attn.py:71-84): FA3 is never
    available here, 'fa3' is refused with the reference's message, anything else is False."""
    if _override_impl == "fa3":
        assert HAS_FA3, "Cannot override to FA3: not available on this hardware"
        return True
    return False


USE_FA3 = _resolve_use_fa3()

# The reference's test hook that forces its ragged (masked) SDPA branch
# (modelcore/kernels/flash_attn.py:88-93). The HIP kernels have a single branch for uniform and
# ragged rows, so the flag changes nothing.
_force_ragged = False


# Checked mode (opt-in): read cache_seqlens back before launching and raise IndexError when a new
# token's position falls outside [0, T_max), as the reference's cache write does
# (modelcore/kernels/flash_attn.py:336-346: an index_put past the cache raises). It costs one host
# sync per call and cannot run under graph capture. Unchecked, such a row is neither appended nor
# attended: its output is NaN, and the callers in this package check positions on the host side
# (Model.check_cache_room). Enabled by set_checked(True) or MODELCORE_AMD_CHECK_POSITIONS=1.
CHECK_POSITIONS = os.environ.get("MODELCORE_AMD_CHECK_POSITIONS", "0") == "1"


def set_checked(enabled: bool):
    """Turn the operator's checked mode on or off (see CHECK_POSITIONS)."""
    global CHECK_POSITIONS
    CHECK_POSITIONS = bool(enabled)


def _check_positions(seqlens, T_new, T_max, shared_prefix=0):
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("flash_attn_with_kvcache: checked mode reads cache_seqlens on the host "
                           "and cannot run under graph capture; call set_checked(False) first")
    lo, hi = (int(x) for x in torch.aminmax(seqlens))
    if lo < 0 or hi + T_new > T_max:
        raise IndexError(f"flash_attn_with_kvcache: positions [{lo}, {hi + T_new}) of the new "
                         f"tokens fall outside the cache of {T_max} positions")
    # The shared-prefix statement includes that every new token lands at or past the prefix.
    if lo < shared_prefix:
        raise ValueError(f"flash_attn_with_kvcache: shared_prefix {shared_prefix} past the "
                         f"position {lo} of a row's new token")


def hip_load_error():
    """Why the HIP library is unavailable, or None when it loads."""
    try:
        _ext.lib()
        return None
    except RuntimeError:
        return _ext.LOAD_ERROR


# -----------------------------------------------------------------------------------------------
# Argument checks (the reference asserts shapes implicitly through torch ops; these raise first).
# -----------------------------------------------------------------------------------------------
def _check_cache(k_cache, v_cache, B, H_kv, D):
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
        raise ValueError(f"k_cache/v_cache must both be (B, T_max, H_kv, D); got "
                         f"{tuple(k_cache.shape)} and {tuple(v_cache.shape)}")
    Bc, T_max, Hc, Dc = k_cache.shape
    if Bc != B or Dc != D or (H_kv is not None and Hc != H_kv):
        raise ValueError(f"cache shape {tuple(k_cache.shape)} does not match q/k/v "
                         f"(B={B}, H_kv={H_kv}, D={D})")
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        s = c.stride()
        if s[3] != 1 or s[2] != D or s[1] != Hc * D:
            raise ValueError(f"{name} must have a contiguous (T_max, H_kv, D) block per row; "
                             f"strides {s}")
    if k_cache.stride(0) != v_cache.stride(0):
        raise ValueError("k_cache and v_cache must have the same batch stride")
    return T_max, Hc


def _check_seqlens(cache_seqlens, B, device):
    if cache_seqlens is None:
        raise ValueError("cache_seqlens is required: (B,) int32, each row's position before the "
                         "new tokens")
    if cache_seqlens.dtype != torch.int32 or cache_seqlens.shape != (B,):
        raise ValueError(f"cache_seqlens must be ({B},) int32; got {tuple(cache_seqlens.shape)} "
                         f"{cache_seqlens.dtype}")
    if cache_seqlens.device != device:
        raise ValueError(f"cache_seqlens is on {cache_seqlens.device}, q on {device}")
    return cache_seqlens.contiguous()


def _window(window_size):
    w = int(window_size[0])
    return -1 if w < 0 else w


# -----------------------------------------------------------------------------------------------
# Public API: same interface as the reference (modelcore/kernels/flash_attn.py:270-366).
# -----------------------------------------------------------------------------------------------
def flash_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None, cache_seqlens=None,
                            causal=False, window_size=(-1, -1), *, advance=0, shared_prefix=0):
    """Attention with KV cache for inference (modelcore/kernels/flash_attn.py:306-366).

    Args:
        q: queries (B, T_new, H, D)
        k_cache, v_cache: preallocated caches (B, T_max, H_kv, D), updated in place
        k, v: new keys/values (B, T_new, H_kv, D) written at cache_seqlens, or both None
        cache_seqlens: (B,) int32 position of each row before the new tokens
        causal: accepted for signature parity; attention is always causal, as in the reference
            fallback
        window_size: (left, right); left = -1 means unlimited
        advance: extension, no counterpart in the reference operator. Non-zero: once the call has
            read cache_seqlens, add this to every row's entry on the device -- the
            KVCache.advance(advance) that follows the last layer's call in a decode step
            (modelcore/model.py:99-100, modelcore/cache.py:62-73). The single-token bf16 /
            head_dim 128 path does it in its last kernel, so the step saves that launch. The host
            side of a KVCache then moves with KVCache.note_device_advance. 0 (default): the
            reference behaviour, cache_seqlens only read.
        shared_prefix: extension, no counterpart in the reference operator. The caller's
            statement that every row's K/V at positions [0, shared_prefix) equal row 0's (rows
            replicated from one prompt, KVCache.prefill; KVCache.shared_prefix tracks it) and that
            the new tokens land at or past it. The single-token bf16 / head_dim 128 path then
            takes those keys from row 0: on the matrix cores for all rows at once when there is
            no window, the prefix has >= 512 keys and rows x query heads per KV head >= 64
            (outputs within bf16 rounding of the call without it: the sums run in another
            order), else read by the decode pass from row 0 (bit-identical outputs, the rows'
            repeated reads served by the caches). 0 (default): each row's own keys.

    Returns:
        (B, T_new, H, D) tensor in q's dtype.
    """
    _ext.require_rocm(q, k_cache, v_cache, k, v, cache_seqlens, what="flash_attn_with_kvcache")
    if q.dim() != 4:
        raise ValueError(f"q must be (B, T_new, H, D); got {tuple(q.shape)}")
    B, T_new, H, D = q.shape
    if (k is None) != (v is None):
        raise ValueError("pass both k and v, or neither")
    H_kv = None
    if k is not None:
        if k.shape != v.shape or k.dim() != 4 or k.shape[0] != B or k.shape[1] != T_new \
                or k.shape[3] != D:
            raise ValueError(f"k/v must be (B, T_new, H_kv, D) = ({B}, {T_new}, H_kv, {D}); got "
                             f"{tuple(k.shape)} and {tuple(v.shape)}")
        H_kv = k.shape[2]
    T_max, H_kv = _check_cache(k_cache, v_cache, B, H_kv, D)
    dt = q.dtype
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache), ("k", k), ("v", v)):
        if t is not None and t.dtype != dt:
            raise TypeError(f"{name} is {t.dtype}, q is {dt}")
    code = _ext.dtype_code(dt)
    seqlens = _check_seqlens(cache_seqlens, B, q.device)
    advance = int(advance)
    shared_prefix = int(shared_prefix)
    if not 0 <= shared_prefix <= T_max:
        raise ValueError(f"shared_prefix {shared_prefix} outside [0, {T_max}]")
    if advance and seqlens.data_ptr() != cache_seqlens.data_ptr():
        raise ValueError("advance needs cache_seqlens itself to be contiguous (it is updated in "
                         "place)")
    if CHECK_POSITIONS and B > 0:
        _check_positions(seqlens, T_new, T_max, shared_prefix)
    q = q.contiguous()
    if k is not None:
        k, v = k.contiguous(), v.contiguous()
    out = torch.empty((B, T_new, H, D), dtype=dt, device=q.device)
    lib = _ext.lib()
    w = _window(window_size)
    ws_bytes = lib.mcamd_attn_workspace_bytes(B, T_new, H, H_kv, D, T_max, w)
    ws = _ext.workspace(q.device, ws_bytes)
    args = (q.data_ptr(), k.data_ptr() if k is not None else None,
            v.data_ptr() if v is not None else None, k_cache.data_ptr(), v_cache.data_ptr(),
            seqlens.data_ptr(), out.data_ptr(), B, T_new, H, H_kv, D, T_max, k_cache.stride(0), w,
            int(bool(causal)), code)
    ws_args = (ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
               _ext.stream_handle(q.device))
    if advance or shared_prefix:
        st = lib.mcamd_flash_attn_with_kvcache_ex(*args, advance, shared_prefix, *ws_args)
    else:
        st = lib.mcamd_flash_attn_with_kvcache(*args, *ws_args)
    _ext.check(st, "flash_attn_with_kvcache")
    return out


def flash_attn_varlen_with_kvcache(q, k_cache, v_cache, k=None, v=None, cache_seqlens=None,
                                   cu_seqlens=None, max_seqlen=None, rows=None, causal=False,
                                   window_size=(-1, -1), *, advance=False):
    """Varlen cached attention: several sequences of different lengths packed along one token
    axis, each appended and attended in its own cache row, with no padding. Extension with no
    single counterpart in the reference: it replaces the multi-prompt prefill's one prefill per
    prompt into a batch-1 cache followed by a copy into its row (modelcore/generate.py:67-80 ->
    KVCache.prefill_row, modelcore/cache.py:92-119) with one call per layer that writes every
    prompt's K/V in place.

    Args:
        q: (total, H, D) packed queries; sequence b is tokens [cu_seqlens[b], cu_seqlens[b + 1])
        k_cache, v_cache: (B_cache, T_max, H_kv, D) caches, updated in place
        k, v: (total, H_kv, D) new keys/values, or both None
        cache_seqlens: (B_cache,) int32 positions; sequence b starts at cache_seqlens[rows[b]]
        cu_seqlens: (n + 1,) int32 on the device, ascending from 0
        max_seqlen: the longest sequence's length (host int)
        rows: (n,) int32 distinct cache rows on the device, or None for rows 0..n-1
        window_size: (left, right); left = -1 means unlimited
        advance: after the call, every sequence's row moves on by its length (device side)

    Returns:
        (total, H, D) tensor in q's dtype.
    """
    _ext.require_rocm(q, k_cache, v_cache, k, v, cache_seqlens, cu_seqlens, rows,
                      what="flash_attn_varlen_with_kvcache")
    if q.dim() != 3:
        raise ValueError(f"q must be (total, H, D); got {tuple(q.shape)}")
    total, H, D = q.shape
    if (k is None) != (v is None):
        raise ValueError("pass both k and v, or neither")
    if cu_seqlens is None or cu_seqlens.dtype != torch.int32 or cu_seqlens.dim() != 1 \
            or cu_seqlens.numel() < 1:
        raise ValueError("cu_seqlens must be a (n + 1,) int32 tensor")
    n = cu_seqlens.numel() - 1
    if rows is not None and (rows.dtype != torch.int32 or rows.shape != (n,)):
        raise ValueError(f"rows must be ({n},) int32; got {tuple(rows.shape)} {rows.dtype}")
    if max_seqlen is None or int(max_seqlen) < 1:
        raise ValueError("max_seqlen (the longest sequence's length, >= 1) is required")
    H_kv = None
    if k is not None:
        if k.shape != v.shape or k.dim() != 3 or k.shape[0] != total or k.shape[2] != D:
            raise ValueError(f"k/v must be (total, H_kv, D) = ({total}, H_kv, {D}); got "
                             f"{tuple(k.shape)} and {tuple(v.shape)}")
        H_kv = k.shape[1]
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
        raise ValueError(f"k_cache/v_cache must both be (B, T_max, H_kv, D); got "
                         f"{tuple(k_cache.shape)} and {tuple(v_cache.shape)}")
    B_cache = k_cache.shape[0]
    T_max, H_kv = _check_cache(k_cache, v_cache, B_cache, H_kv, D)
    dt = q.dtype
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache), ("k", k), ("v", v)):
        if t is not None and t.dtype != dt:
            raise TypeError(f"{name} is {t.dtype}, q is {dt}")
    code = _ext.dtype_code(dt)
    seqlens = _check_seqlens(cache_seqlens, B_cache, q.device)
    if advance and seqlens.data_ptr() != cache_seqlens.data_ptr():
        raise ValueError("advance needs cache_seqlens itself to be contiguous (it is updated in "
                         "place)")
    if CHECK_POSITIONS and n > 0:
        lens = (cu_seqlens[1:] - cu_seqlens[:-1]).long()
        base = seqlens.long()[rows.long()] if rows is not None else seqlens.long()[:n]
        lo, hi = int(base.min()), int((base + lens).max())
        if lo < 0 or hi > T_max:
            raise IndexError(f"flash_attn_varlen_with_kvcache: positions [{lo}, {hi}) of the new "
                             f"tokens fall outside the cache of {T_max} positions")
    q = q.contiguous()
    if k is not None:
        k, v = k.contiguous(), v.contiguous()
    out = torch.empty_like(q)
    lib = _ext.lib()
    st = lib.mcamd_flash_attn_varlen_with_kvcache(
        q.data_ptr(), k.data_ptr() if k is not None else None,
        v.data_ptr() if v is not None else None, k_cache.data_ptr(), v_cache.data_ptr(),
        seqlens.data_ptr(), rows.data_ptr() if rows is not None else None,
        cu_seqlens.contiguous().data_ptr(), out.data_ptr(), n, int(max_seqlen), H, H_kv, D, T_max,
        k_cache.stride(0), _window(window_size), int(bool(causal)), code, int(bool(advance)),
        _ext.stream_handle(q.device))
    _ext.check(st, "flash_attn_varlen_with_kvcache")
    return out


def flash_attn_func(q, k, v, causal=False, window_size=(-1, -1), doc_args=None):
    """No-cache attention (modelcore/kernels/flash_attn.py:270-303), inference only.

    q (B, T, H, D), k/v (B, T, H_kv, D) form a cache of their own at position 0, so this runs
    the chunked-prefill kernel with cache_seqlens = 0 and the same causal/window rule as the
    reference fallback (which is causal whatever `causal` says). Training (autograd) and
    packed-document masking (doc_args) belong to the reference's training path, which this
    build does not cover; both raise.
    """
    _ext.require_rocm(q, k, v, what="flash_attn_func")
    if doc_args is not None:
        raise NotImplementedError("doc_args (packed-document training masks) is not supported")
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        raise NotImplementedError("flash_attn_func here is forward-only (no autograd)")
    if q.dim() != 4 or k.dim() != 4 or k.shape != v.shape:
        raise ValueError(f"q must be (B, T, H, D), k/v (B, T, H_kv, D); got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    B, T, H, D = q.shape
    if k.shape[0] != B or k.shape[1] != T or k.shape[3] != D:
        raise ValueError(f"k/v shape {tuple(k.shape)} does not match q {tuple(q.shape)}")
    for name, t in (("k", k), ("v", v)):
        if t.dtype != q.dtype:
            raise TypeError(f"{name} is {t.dtype}, q is {q.dtype}")
    code = _ext.dtype_code(q.dtype)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    H_kv = k.shape[2]
    out = torch.empty_like(q)
    seqlens = torch.zeros(B, dtype=torch.int32, device=q.device)
    lib = _ext.lib()
    st = lib.mcamd_prefill_attention(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), seqlens.data_ptr(), out.data_ptr(), B, T, H,
        H_kv, D, T, k.stride(0), _window(window_size), code, _ext.stream_handle(q.device))
    _ext.check(st, "flash_attn_func")
    return out


# Export: the operator namespace (modelcore/kernels/flash_attn.py:373-376).
flash_attn = SimpleNamespace(
    flash_attn_func=flash_attn_func,
    flash_attn_with_kvcache=flash_attn_with_kvcache,
    flash_attn_varlen_with_kvcache=flash_attn_varlen_with_kvcache,
    # Keyword arguments of flash_attn_with_kvcache beyond the reference's (callers check this
    # before passing them, so that an operator without them can stand in).
    EXTENSIONS=frozenset({"advance", "shared_prefix"}),
)
