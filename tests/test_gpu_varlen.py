"""The varlen cached-attention operator (flash_attn_varlen_with_kvcache,
mcamd_flash_attn_varlen_with_kvcache) on the GPU against the float64 oracle: several sequences of
different lengths packed along one token axis, each appended and attended in its own cache row
(rows[b], at that row's position), as the reference's per-prompt prefill into a batch-1 cache and
copy into its row would leave them (modelcore/generate.py:67-80 -> modelcore/cache.py:92-119).

* Outputs within the attention tolerance of the oracle run once per sequence on its row.
* The appended K/V bit-exact at each row's own positions; rows not listed untouched.
* With advance, exactly the listed rows move on by their sequence's length.
* A sequence whose positions fall outside the cache: NaN output, the append drops the positions
  past it (as the operator's other paths do), the other sequences intact.
Both kernels are covered: the bf16 matrix-core kernel (head_dim 128, query tiles of 256 / G
positions, so sequences end inside, at and past tile boundaries) and the general kernel.
"""
import numpy as np
import pytest
import torch

from _util import ATOL, bits, gen, max_abs, randn, to_np
from oracle import kv_oracle as ko
from modelcore_amd.kernels.flash_attn import flash_attn

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _note(*a):
    print("case:", *a, flush=True)


CASES = [
    # dtype, H, H_kv, D, T_max, B_cache, rows, bases (positions before), lengths, window
    (torch.bfloat16, 32, 8, 128, 200, 8, [0, 2, 4, 6], [0, 0, 0, 0], [37, 150, 5, 88], -1),
    (torch.bfloat16, 16, 4, 128, 700, 4, [3, 0, 2, 1], [10, 0, 300, 3], [300, 1, 64, 257], 100),
    (torch.bfloat16, 12, 4, 128, 400, 5, [4, 1], [0, 77], [171, 85], -1),   # G = 3: 85 per tile
    (torch.bfloat16, 16, 1, 128, 300, 3, [2], [5], [40], 0),                # G = 16, window 0
    (torch.float32, 8, 2, 64, 128, 3, [1, 0, 2], [0, 4, 9], [5, 70, 1], -1),
    (torch.bfloat16, 12, 4, 64, 64, 2, [0, 1], [0, 20], [33, 2], 7),
    (torch.float32, 16, 4, 128, 96, 2, [1, 0], [3, 0], [40, 65], 31),
]


def _case(dtype, H, H_kv, D, T_max, B_cache, lengths, seed):
    g = gen(seed)
    total = sum(lengths)
    return dict(
        k_cache=randn(g, B_cache, T_max, H_kv, D, dtype=dtype),
        v_cache=randn(g, B_cache, T_max, H_kv, D, dtype=dtype),
        q=randn(g, total, H, D, dtype=dtype), k=randn(g, total, H_kv, D, dtype=dtype),
        v=randn(g, total, H_kv, D, dtype=dtype))


def _run(c, rows, bases, lengths, window, advance=False):
    B_cache = c["k_cache"].shape[0]
    seqlens = torch.zeros(B_cache, dtype=torch.int32)
    seqlens[rows] = torch.tensor(bases, dtype=torch.int32)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32)
    g = {n: t.to(DEV) for n, t in c.items()}
    sl = seqlens.to(DEV)
    out = flash_attn.flash_attn_varlen_with_kvcache(
        g["q"], g["k_cache"], g["v_cache"], k=g["k"], v=g["v"], cache_seqlens=sl,
        cu_seqlens=cu.to(DEV), max_seqlen=max(lengths),
        rows=torch.tensor(rows, dtype=torch.int32, device=DEV), causal=True,
        window_size=(window, 0), advance=advance)
    torch.cuda.synchronize()
    return out, g, sl.cpu(), seqlens


def _oracle(c, rows, bases, lengths, window):
    """Per sequence: the float64 oracle on its row (append, then attention)."""
    outs, kc, vc = [], bits(c["k_cache"]).copy(), bits(c["v_cache"]).copy()
    a = 0
    for r, s0, n in zip(rows, bases, lengths):
        q, k, v = (to_np(c[x][a:a + n])[None] for x in ("q", "k", "v"))
        y, k1, v1 = ko.flash_attn_with_kvcache(q, to_np(c["k_cache"][r:r + 1]),
                                               to_np(c["v_cache"][r:r + 1]), k, v, [s0], window)
        outs.append(y[0])
        kb, vb = ko.append(kc[r:r + 1], vc[r:r + 1], bits(c["k"][a:a + n])[None],
                           bits(c["v"][a:a + n])[None], [s0])
        kc[r:r + 1], vc[r:r + 1] = kb, vb
        a += n
    return np.concatenate(outs, 0), kc, vc


@pytest.mark.parametrize("dtype,H,H_kv,D,T_max,B_cache,rows,bases,lengths,window", CASES)
def test_varlen_matches_the_oracle_per_sequence(dtype, H, H_kv, D, T_max, B_cache, rows, bases,
                                                lengths, window):
    _note("varlen", dtype, H, H_kv, D, T_max, rows, bases, lengths, window)
    c = _case(dtype, H, H_kv, D, T_max, B_cache, lengths, seed=61)
    out, g, after, before = _run(c, rows, bases, lengths, window, advance=True)
    want, kc, vc = _oracle(c, rows, bases, lengths, window)
    err = max_abs(to_np(out), want)
    assert err <= ATOL[dtype], f"max-abs {err}"
    assert np.array_equal(bits(g["k_cache"]), kc) and np.array_equal(bits(g["v_cache"]), vc)
    moved = before.clone()
    moved[rows] += torch.tensor(lengths, dtype=torch.int32)
    assert torch.equal(after, moved), "advance moves exactly the listed rows by their lengths"


def test_varlen_without_rows_uses_rows_in_order_and_leaves_positions():
    c = _case(torch.bfloat16, 16, 4, 128, 160, 3, [60, 1, 99], seed=62)
    out, g, after, before = _run(c, [0, 1, 2], [0, 50, 7], [60, 1, 99], -1)
    want, kc, _ = _oracle(c, [0, 1, 2], [0, 50, 7], [60, 1, 99], -1)
    assert max_abs(to_np(out), want) <= ATOL[torch.bfloat16]
    assert np.array_equal(bits(g["k_cache"]), kc)
    assert torch.equal(after, before), "no advance requested"
    # the same call with rows=None: identical bits
    cu = torch.tensor([0, 60, 61, 160], dtype=torch.int32, device=DEV)
    g2 = {n: t.to(DEV) for n, t in c.items()}
    sl = torch.tensor([0, 50, 7], dtype=torch.int32, device=DEV)
    out2 = flash_attn.flash_attn_varlen_with_kvcache(g2["q"], g2["k_cache"], g2["v_cache"],
                                                     k=g2["k"], v=g2["v"], cache_seqlens=sl,
                                                     cu_seqlens=cu, max_seqlen=99)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out2), bits(out))


def test_a_sequence_past_the_cache_gets_nan_and_drops_the_positions_past_it():
    """Row 1's sequence would end past T_max: its attention output is NaN and the append drops
    the positions past the cache (as the operator's other paths do); the other sequence is
    unaffected."""
    c = _case(torch.bfloat16, 8, 2, 128, 64, 2, [30, 20], seed=63)
    out, g, _, _ = _run(c, [0, 1], [10, 50], [30, 20], -1)
    want, kc, _ = _oracle(c, [0], [10], [30], -1)
    y = to_np(out)
    assert max_abs(y[:30], want) <= ATOL[torch.bfloat16]
    assert np.isnan(y[30:]).all()
    got = bits(g["k_cache"])
    assert np.array_equal(got[0], kc[0])
    assert np.array_equal(got[1, :50], bits(c["k_cache"])[1, :50]), "row 1 before its position"
    assert np.array_equal(got[1, 50:], bits(c["k"])[30:44]), "row 1's tokens up to the end"
