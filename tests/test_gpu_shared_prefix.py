"""The decode operator's shared-prefix read (flash_attn_with_kvcache(..., shared_prefix=P),
mcamd_flash_attn_with_kvcache_ex): when every row's K/V at positions [0, P) are copies of row
0's -- rows replicated from one prompt by KVCache.prefill -- the bf16 / head_dim 128 decode reads
those keys from row 0 for every row. The values are the same, so outputs and cache contents must
be bit-identical to the call without it, on every path (the other paths read each row's own copy)
and for windows that end inside and outside the prefix. A planted difference in row 1's prefix
shows the reads really come from row 0, and a run of the sampling decoder gives the same tokens
and logits with and without it.
"""
import numpy as np
import pytest
import torch

from _util import bits, make_case
from modelcore_amd.kernels.flash_attn import flash_attn

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _note(*a):
    print("case:", *a, flush=True)


def _replicated(seqlens, P, H, H_kv, D, T_max, dtype, seed):
    c = make_case(seqlens, 1, H, H_kv, D, T_max, dtype, seed=seed)
    for name in ("k_cache", "v_cache"):
        c[name][1:, :P] = c[name][0:1, :P]  # every row's prefix is row 0's
    return c


def _call(c, window, shared):
    g = {n: t.to(DEV) for n, t in c.items()}
    out = flash_attn.flash_attn_with_kvcache(g["q"], g["k_cache"], g["v_cache"], k=g["k"],
                                             v=g["v"], cache_seqlens=g["cache_seqlens"],
                                             causal=True, window_size=(window, 0),
                                             shared_prefix=shared)
    torch.cuda.synchronize()
    return out, g


CASES = [
    # dtype, P, seqlens (all >= P), H, H_kv, D, T_max, window
    (torch.bfloat16, 2048, [2048, 2100, 2559, 2300, 2049, 2200, 2400, 2048], 32, 8, 128, 2600, -1),
    (torch.bfloat16, 700, [700, 705, 1200, 900], 16, 4, 128, 1300, -1),
    (torch.bfloat16, 700, [700, 705, 1200, 900], 16, 4, 128, 1300, 64),    # windows: inside, across
    (torch.bfloat16, 700, [700, 705, 1200, 900], 16, 4, 128, 1300, 300),   # and past the prefix
    (torch.bfloat16, 64, [64, 80, 64], 8, 2, 64, 128, -1),                 # general path: ignored
    (torch.float32, 64, [64, 80, 64], 8, 2, 128, 128, -1),
]


@pytest.mark.parametrize("dtype,P,seqlens,H,H_kv,D,T_max,window", CASES)
def test_shared_prefix_reads_give_bit_identical_results(dtype, P, seqlens, H, H_kv, D, T_max,
                                                        window):
    _note("shared prefix", dtype, P, seqlens, H, H_kv, D, T_max, window)
    c = _replicated(seqlens, P, H, H_kv, D, T_max, dtype, seed=41)
    want, gw = _call(c, window, 0)
    got, gg = _call(c, window, P)
    assert np.array_equal(bits(got), bits(want)), "outputs differ"
    assert np.array_equal(bits(gg["k_cache"]), bits(gw["k_cache"]))
    assert np.array_equal(bits(gg["v_cache"]), bits(gw["v_cache"]))


def test_shared_prefix_keys_come_from_row_0():
    # Row 1's prefix is planted different from row 0's: with the statement, row 1 attends row 0's
    # keys, i.e. it matches the call on a cache where row 1's prefix is replaced by row 0's.
    P, seqlens, H, H_kv, D, T_max = 500, [500, 640], 16, 4, 128, 700
    _note("shared prefix from row 0", P, seqlens)
    c = make_case(seqlens, 1, H, H_kv, D, T_max, torch.bfloat16, seed=42)
    fixed = {n: t.clone() for n, t in c.items()}
    for name in ("k_cache", "v_cache"):
        fixed[name][1, :P] = fixed[name][0, :P]
    got, _ = _call(c, -1, P)
    want, _ = _call(fixed, -1, 0)
    own, _ = _call(c, -1, 0)
    assert np.array_equal(bits(got), bits(want))
    assert not np.array_equal(bits(got)[1], bits(own)[1])
    assert np.array_equal(bits(got)[0], bits(own)[0])


def test_shared_prefix_outside_the_cache_is_refused():
    c = _replicated([10, 12], 8, 4, 2, 128, 16, torch.bfloat16, seed=43)
    with pytest.raises(ValueError):
        _call(c, -1, 17)
    with pytest.raises(ValueError):
        _call(c, -1, -1)
