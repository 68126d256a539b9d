"""Algorithmic byte and FLOP counts of the KV path: what a roofline divides by.

They count only what the mathematics needs -- every cache element a query may see read once,
q read once, the output written once, the new K/V read and appended once -- and nothing a kernel
adds (split partials, re-reads, masked work). The per-layer attention term follows the
reference's own model (modelcore/stats.py:55-73, :98-107) with one difference: a windowed query
here touches n = min(L + T_new, window + 1) keys (the query's own key included), where the
reference's kv_read_bytes counts min(window, ctx).
"""
from __future__ import annotations

from typing import Sequence


def keys_seen(L: int, t_new: int, window: int) -> int:
    """Distinct cache positions the queries of one row read: [lo, L + t_new - 1]."""
    last = L + t_new - 1
    lo = max(0, L - window) if window >= 0 else 0
    return last - lo + 1


def decode_kv_bytes(seqlens: Sequence[int], n_kv_head: int, head_dim: int, itemsize: int,
                    window: int = -1) -> int:
    """K and V bytes read by one single-token decode over rows at positions `seqlens`."""
    n = sum(keys_seen(int(L), 1, window) for L in seqlens)
    return 2 * n * n_kv_head * head_dim * itemsize


def decode_step_bytes(seqlens: Sequence[int], n_head: int, n_kv_head: int, head_dim: int,
                      itemsize: int, window: int = -1, append: bool = True) -> int:
    """One append + decode call: K/V read, q read, out written, new K/V read and written."""
    B = len(seqlens)
    total = decode_kv_bytes(seqlens, n_kv_head, head_dim, itemsize, window)
    total += 2 * B * n_head * head_dim * itemsize
    if append:
        total += 2 * 2 * B * n_kv_head * head_dim * itemsize
    return total


def decode_flops(seqlens: Sequence[int], n_head: int, head_dim: int, window: int = -1) -> int:
    """4 * H * D FLOPs per visible key per row (QK^T and PV)."""
    return sum(4 * n_head * head_dim * keys_seen(int(L), 1, window) for L in seqlens)


def prefill_flops(seqlens: Sequence[int], t_new: int, n_head: int, head_dim: int,
                  window: int = -1) -> int:
    """4 * H * D FLOPs per attended (query, key) pair of a chunk at positions `seqlens`
    (modelcore/stats.py:66-73 counts the same pairs for a prompt from position 0)."""
    pairs = 0
    for L in seqlens:
        for t in range(t_new):
            p = int(L) + t
            pairs += p + 1 if window < 0 else min(p, window) + 1
    return 4 * n_head * head_dim * pairs


def append_bytes(batch: int, t_new: int, n_kv_head: int, head_dim: int, itemsize: int) -> int:
    """New K and V read once and written once."""
    return 2 * 2 * batch * t_new * n_kv_head * head_dim * itemsize


def replicate_bytes(n_slots: int, n_rows: int, n_tokens: int, n_kv_head: int, head_dim: int,
                    itemsize: int) -> int:
    """The source read once, every destination row written once, K and V."""
    per = n_slots * n_tokens * n_kv_head * head_dim * itemsize * 2
    return per * (n_rows + 1)
