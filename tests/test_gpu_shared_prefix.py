"""The decode operator's shared-prefix read (flash_attn_with_kvcache(..., shared_prefix=P),
mcamd_flash_attn_with_kvcache_ex): when every row's K/V at positions [0, P) are copies of row
0's -- rows replicated from one prompt by KVCache.prefill -- the bf16 / head_dim 128 decode takes
those keys from row 0 for every row, in one of two ways:
  * few queries per KV head, a short prefix or a window: the decode pass reads them from row 0
    itself; the values are the same, so outputs must be bit-identical to the call without it;
  * rows x query heads >= 64, no window, P >= 512: the prefix goes to the matrix cores (all rows'
    queries against row 0's prefix keys, in key ranges) and the decode pass covers each row's
    own keys; the partial sums then run in another order, so outputs must match the float64
    oracle within the bf16 tolerance and the call without it within a few bf16 units.
The caches must be bit-identical either way (the append does not change). A planted difference
in row 1's prefix shows the reads come from row 0, and the sampling decoder gives the same logits
with and without it, teacher-forced on one token stream.
"""
import numpy as np
import pytest
import torch

from _util import ATOL, bits, make_case, max_abs, to_np
from oracle import kv_oracle as ko
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


def _rows(n, lo, hi, seed):
    return [int(x) for x in np.random.default_rng(seed).integers(lo, hi, n)]


PREFIX_CASES = [
    # dtype, P, seqlens (all >= P), H, H_kv, D, T_max: the prefix on the matrix cores (key
    # ranges of at least 128 keys, at most sixteen, as many as fill the chip with jobs of 64
    # (row, query head) pairs; the merge folds in 4, 8 or 16 partial slots per unit)
    (torch.bfloat16, 2048, [2048] + _rows(63, 2048, 2560, 1), 32, 8, 128, 2560),  # 8 ranges
    (torch.bfloat16, 600, _rows(32, 600, 900, 2), 12, 4, 128, 1000),       # G = 3, 4 ranges
    (torch.bfloat16, 1000, _rows(100, 1000, 1100, 3), 16, 4, 128, 1200),   # 400 pairs, 7 ranges
    (torch.bfloat16, 777, _rows(40, 777, 800, 4), 64, 8, 128, 900),        # G = 8, 6 ranges
    (torch.bfloat16, 2100, _rows(8, 2100, 2300, 7), 16, 2, 128, 2400),     # 16 ranges, one pair block
    (torch.bfloat16, 1301, _rows(24, 1301, 1400, 8), 24, 8, 128, 1500),    # G = 3, 72 pairs: a ragged block
]

READ_CASES = [
    # dtype, P, seqlens (all >= P), H, H_kv, D, T_max, window: the decode pass reads the prefix
    # from row 0 itself (32 pairs per KV head, or a window), or the general path ignores it
    (torch.bfloat16, 2048, [2048, 2100, 2559, 2300, 2049, 2200, 2400, 2048], 32, 8, 128, 2600, -1),
    (torch.bfloat16, 700, [700, 705, 1200, 900], 16, 4, 128, 1300, -1),
    (torch.bfloat16, 700, [700, 705, 1200, 900], 16, 4, 128, 1300, 64),    # windows: inside, across
    (torch.bfloat16, 700, [700, 705, 1200, 900], 16, 4, 128, 1300, 300),   # and past the prefix
    (torch.bfloat16, 2048, [2048] + _rows(63, 2048, 2560, 5), 32, 8, 128, 2560, 600),
    # 512 query heads per KV head: more than the matrix-core kernel's 256 pairs per workgroup,
    # so the decode pass reads the prefix from row 0 even though rows x heads >= 64
    (torch.bfloat16, 600, [600, 700], 512, 1, 128, 800, -1),
    (torch.bfloat16, 64, [64, 80, 64], 8, 2, 64, 128, -1),                 # general path: ignored
    (torch.float32, 64, [64, 80, 64], 8, 2, 128, 128, -1),
]


@pytest.mark.parametrize("dtype,P,seqlens,H,H_kv,D,T_max,window", READ_CASES)
def test_shared_prefix_reads_give_bit_identical_results(dtype, P, seqlens, H, H_kv, D, T_max,
                                                        window):
    _note("shared prefix, read", dtype, P, len(seqlens), H, H_kv, D, T_max, window)
    c = _replicated(seqlens, P, H, H_kv, D, T_max, dtype, seed=41)
    want, gw = _call(c, window, 0)
    got, gg = _call(c, window, P)
    assert np.array_equal(bits(got), bits(want)), "outputs differ"
    assert np.array_equal(bits(gg["k_cache"]), bits(gw["k_cache"]))
    assert np.array_equal(bits(gg["v_cache"]), bits(gw["v_cache"]))


@pytest.mark.parametrize("dtype,P,seqlens,H,H_kv,D,T_max", PREFIX_CASES)
def test_shared_prefix_on_the_matrix_cores_matches_the_oracle(dtype, P, seqlens, H, H_kv, D,
                                                              T_max):
    _note("shared prefix, matrix cores", dtype, P, len(seqlens), H, H_kv, D, T_max)
    c = _replicated(seqlens, P, H, H_kv, D, T_max, dtype, seed=44)
    want, gw = _call(c, -1, 0)
    got, gg = _call(c, -1, P)
    assert np.array_equal(bits(gg["k_cache"]), bits(gw["k_cache"]))
    assert np.array_equal(bits(gg["v_cache"]), bits(gw["v_cache"]))
    y = to_np(got)
    assert np.isfinite(y).all()
    near = max_abs(y, to_np(want))
    assert near <= 4e-3, f"against each row's own reads: max-abs {near}"
    oracle = ko.flash_attn_with_kvcache(to_np(c["q"]), to_np(c["k_cache"]), to_np(c["v_cache"]),
                                        to_np(c["k"]), to_np(c["v"]), seqlens, -1)[0]
    err = max_abs(y, oracle)
    print(f"max-abs against the unshared call {near:.2e}, against the oracle {err:.2e}",
          flush=True)
    assert err <= ATOL[torch.bfloat16], f"against the oracle: max-abs {err}"
    # Accuracy guard (deterministic outputs): 4.0e-4 to 1.8e-3 measured on these cases.
    assert err <= 3e-3, f"against the oracle: max-abs {err}, below what this path delivers"


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


def test_captured_steps_with_the_prefix_on_the_matrix_cores_replay_the_eager_steps():
    # Three decode steps with the shared prefix on the matrix cores and the advance folded in,
    # captured once: every replay (eager work and synchronisations between them) must equal the
    # eager steps bit for bit, positions included.
    B, H, H_kv, D, T_max, P, steps = 32, 16, 4, 128, 1200, 1000, 3
    seqlens = _rows(B, P, 1100, 6)
    _note("graph, matrix-core prefix", B, P)
    c = _replicated(seqlens, P, H, H_kv, D, T_max, torch.bfloat16, seed=45)
    gen = torch.Generator().manual_seed(46)
    qs = torch.randn(steps, B, 1, H, D, generator=gen).to(torch.bfloat16).to(DEV)
    ks = torch.randn(steps, B, 1, H_kv, D, generator=gen).to(torch.bfloat16).to(DEV)
    vs = torch.randn(steps, B, 1, H_kv, D, generator=gen).to(torch.bfloat16).to(DEV)
    g = {n: t.to(DEV) for n, t in c.items()}
    outs = [torch.empty(B, 1, H, D, dtype=torch.bfloat16, device=DEV) for _ in range(steps)]

    def run_steps():
        for s in range(steps):
            outs[s].copy_(flash_attn.flash_attn_with_kvcache(
                qs[s], g["k_cache"], g["v_cache"], k=ks[s], v=vs[s],
                cache_seqlens=g["cache_seqlens"], causal=True, window_size=(-1, 0), advance=1,
                shared_prefix=P))

    def reset():
        g["k_cache"].copy_(c["k_cache"])
        g["v_cache"].copy_(c["v_cache"])
        g["cache_seqlens"].copy_(c["cache_seqlens"])

    run_steps()  # warm-up (workspace sized)
    reset()
    run_steps()
    torch.cuda.synchronize()
    eager = [bits(o) for o in outs]
    eager_k = bits(g["k_cache"])
    assert g["cache_seqlens"].tolist() == [p + steps for p in seqlens]
    reset()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run_steps()
    for rep in range(3):
        reset()
        torch.cuda.synchronize()
        for o in outs:
            o.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        assert g["cache_seqlens"].tolist() == [p + steps for p in seqlens], f"replay {rep}"
        assert np.array_equal(bits(g["k_cache"]), eager_k), f"replay {rep}: cache"
        for s in range(steps):
            assert np.array_equal(bits(outs[s]), eager[s]), f"replay {rep}, step {s}"
        run_steps()
        torch.cuda.synchronize()
