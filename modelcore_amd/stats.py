"""Algorithmic byte and FLOP counts of the KV path: what a roofline divides by.

They count only what the mathematics needs -- every key a query may see read once, q read once,
the output written once, the new K/V written once -- and nothing a kernel adds (split partials,
re-reads, masked work). A decode call that appends reads the new token's K/V from the caller's
k/v (not from the cache) and writes them into the cache: the read is part of "every key read
once", the write is the append.

The reference prices the same work per layer (modelcore/stats.py:55-73, :98-107); its formulas are
restated below (``ref_*``) so that tests pin one against the other. They agree for full
attention. Under a sliding window of w keys back, a query here touches n = min(L, w) + 1 keys
(its own key included), while the reference's ``min(w, context)`` counts one fewer once the
context exceeds w; the counts here are the keys the kernels actually read.
"""
from __future__ import annotations

from typing import Iterable, Sequence


def keys_seen(L: int, t_new: int, window: int) -> int:
    """Distinct cache positions the queries of one row read: [lo, L + t_new - 1], where the
    first query sits at L and lo = max(0, L - window) (window < 0: lo = 0)."""
    last = L + t_new - 1
    lo = max(0, L - window) if window >= 0 else 0
    return last - lo + 1


def decode_kv_bytes(seqlens: Sequence[int], n_kv_head: int, head_dim: int, itemsize: int,
                    window: int = -1) -> int:
    """K and V bytes of every key the single-token queries of rows at positions `seqlens` see,
    each read once (the new token's key included)."""
    n = sum(keys_seen(int(L), 1, window) for L in seqlens)
    return 2 * n * n_kv_head * head_dim * itemsize


def decode_step_bytes(seqlens: Sequence[int], n_head: int, n_kv_head: int, head_dim: int,
                      itemsize: int, window: int = -1, append: bool = True) -> int:
    """One decode call: K/V of every visible key read once, q read, the output written, and with
    `append` the new K/V written into the cache (their read is one of the visible keys)."""
    B = len(seqlens)
    total = decode_kv_bytes(seqlens, n_kv_head, head_dim, itemsize, window)
    total += 2 * B * n_head * head_dim * itemsize
    if append:
        total += 2 * B * n_kv_head * head_dim * itemsize
    return total


def decode_flops(seqlens: Sequence[int], n_head: int, head_dim: int, window: int = -1) -> int:
    """4 * H * D FLOPs per visible key per row (QK^T and PV)."""
    return sum(4 * n_head * head_dim * keys_seen(int(L), 1, window) for L in seqlens)


def prefill_pairs(seqlens: Sequence[int], t_new: int, window: int = -1) -> int:
    """Attended (query, key) pairs of a chunk of t_new queries per row at positions `seqlens`:
    query p sees p + 1 keys, or min(p, window) + 1 under a window."""
    pairs = 0
    for L in seqlens:
        L = int(L)
        if window < 0:
            pairs += t_new * L + t_new * (t_new + 1) // 2  # sum over p in [L, L + t_new) of p + 1
        else:
            pairs += sum(min(p, window) + 1 for p in range(L, L + t_new))
    return pairs


def prefill_flops(seqlens: Sequence[int], t_new: int, n_head: int, head_dim: int,
                  window: int = -1) -> int:
    """4 * H * D FLOPs per attended (query, key) pair of a chunk at positions `seqlens`
    (modelcore/stats.py:66-73 counts the same pairs for a prompt from position 0)."""
    return 4 * n_head * head_dim * prefill_pairs(seqlens, t_new, window)


def append_bytes(batch: int, t_new: int, n_kv_head: int, head_dim: int, itemsize: int) -> int:
    """New K and V read once and written once."""
    return 2 * 2 * batch * t_new * n_kv_head * head_dim * itemsize


def replicate_bytes(n_slots: int, n_rows: int, n_tokens: int, n_kv_head: int, head_dim: int,
                    itemsize: int) -> int:
    """The source read once, every destination row written once, K and V."""
    per = n_slots * n_tokens * n_kv_head * head_dim * itemsize * 2
    return per * (n_rows + 1)


# -----------------------------------------------------------------------------------------------
# The reference's own per-layer model, restated (attention terms only; the matmul-parameter terms
# are outside the KV path). `windows` holds one window per attention layer (-1 = full context).
# -----------------------------------------------------------------------------------------------
def ref_effective_window(window: int, cap: int) -> int:
    """modelcore/stats.py:33-35: -1 means the whole context, capped at `cap`."""
    return cap if window < 0 else min(window, cap)


def ref_kv_read_bytes(windows: Iterable[int], n_kv_head: int, head_dim: int, itemsize: int,
                      context_len: int) -> int:
    """modelcore/stats.py:98-107: K/V bytes one decode step reads per row, summed per layer
    (a KV-sharing layer reads the shared slot itself)."""
    return sum(2 * n_kv_head * head_dim * itemsize * ref_effective_window(w, context_len)
               for w in windows)


def ref_decode_attn_flops(windows: Iterable[int], n_head: int, head_dim: int,
                          context_len: int) -> int:
    """The attention term of modelcore/stats.py:55-63 (one token at a context length)."""
    return sum(4 * n_head * head_dim * ref_effective_window(w, context_len) for w in windows)


def ref_prefill_attn_flops(windows: Iterable[int], n_head: int, head_dim: int,
                           num_tokens: int) -> int:
    """The attention term of modelcore/stats.py:66-73 (a causal prompt from position 0)."""
    total = 0
    for window in windows:
        w = ref_effective_window(window, num_tokens)
        attended = w * (w + 1) // 2 + (num_tokens - w) * w
        total += 4 * n_head * head_dim * attended
    return total
