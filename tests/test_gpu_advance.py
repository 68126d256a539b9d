"""The operator with the decode step's position advance folded in
(mcamd_flash_attn_with_kvcache_ex, flash_attn_with_kvcache(..., advance=n)).

Its outputs and cache contents must be bit-identical to the plain operator call followed by the
separate advance (cache_seqlens += n, modelcore/cache.py:62-73), and every row's position must
have moved by n -- rows outside the cache included -- on each path: the single-token bf16 /
head_dim 128 decode (the advance runs in its merge pass), the general decode, chunked prefill and
a call with no new tokens. The merge pass no longer reads cache_seqlens, so a row that falls
outside the cache after a call in which it had keys must not pick up the earlier call's
descriptor: that case is checked against the float64 oracle.
"""
import numpy as np
import pytest
import torch

from _util import ATOL, bits, make_case, max_abs, to_np
from modelcore_amd import _ext
from modelcore_amd.kernels.flash_attn import flash_attn
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _note(*a):
    print("case:", *a, flush=True)


def _run(c, window, advance):
    g = {n: t.to(DEV) for n, t in c.items()}
    out = flash_attn.flash_attn_with_kvcache(g["q"], g["k_cache"], g["v_cache"], k=g["k"],
                                             v=g["v"], cache_seqlens=g["cache_seqlens"],
                                             causal=True, window_size=(window, 0),
                                             advance=advance)
    torch.cuda.synchronize()
    return out, g


CASES = [
    # dtype, seqlens, T_new, H, H_kv, D, T_max, window
    (torch.bfloat16, [700, 3, 1999, 2000], 1, 8, 2, 128, 2000, -1),  # fused decode; row 3 outside
    (torch.bfloat16, [1500, 60, 0], 1, 16, 4, 128, 1600, 64),        # fused decode, windowed
    (torch.bfloat16, [2500, 2400], 1, 32, 8, 128, 2600, -1),         # units of many segments
    (torch.float32, [40, 0, 77], 1, 8, 4, 64, 96, -1),               # general decode
    (torch.bfloat16, [33, 7, 96], 1, 4, 2, 80, 96, 16),              # general decode, head_dim 80
    (torch.bfloat16, [100, 0, 300], 37, 8, 2, 128, 400, -1),         # chunked prefill (MFMA)
    (torch.float32, [5, 50], 9, 4, 1, 32, 64, 8),                    # chunked prefill (general)
]


@pytest.mark.parametrize("dtype,seqlens,T_new,H,H_kv,D,T_max,window", CASES)
@pytest.mark.parametrize("advance", [1, 3])
def test_advance_matches_the_call_then_the_separate_advance(dtype, seqlens, T_new, H, H_kv, D,
                                                           T_max, window, advance):
    _note("advance", advance, dtype, seqlens, T_new, H, H_kv, D, T_max, window)
    c = make_case(seqlens, T_new, H, H_kv, D, T_max, dtype, seed=21)
    want_out, want = _run(c, window, 0)
    want["cache_seqlens"] += advance  # KVCache.advance after the plain call
    out, got = _run(c, window, advance)
    assert np.array_equal(bits(out), bits(want_out)), "outputs differ"
    assert np.array_equal(bits(got["k_cache"]), bits(want["k_cache"]))
    assert np.array_equal(bits(got["v_cache"]), bits(want["v_cache"]))
    assert got["cache_seqlens"].tolist() == [p + advance for p in seqlens]
    assert torch.equal(got["cache_seqlens"], want["cache_seqlens"])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_a_call_without_new_tokens_only_advances(dtype):
    seqlens = [4, 9, 0]
    c = make_case(seqlens, 1, 4, 2, 64, 16, dtype, seed=22)
    g = {n: t.to(DEV) for n, t in c.items()}
    lib = _ext.lib()
    _ext.check(lib.mcamd_flash_attn_with_kvcache_ex(
        g["q"].data_ptr(), None, None, g["k_cache"].data_ptr(), g["v_cache"].data_ptr(),
        g["cache_seqlens"].data_ptr(), g["q"].data_ptr(), 3, 0, 4, 2, 64, 16,
        g["k_cache"].stride(0), -1, 1, _ext.dtype_code(dtype), 5, 0, None, 0,
        _ext.stream_handle(DEV)), "advance only")
    torch.cuda.synchronize()
    assert g["cache_seqlens"].tolist() == [9, 14, 5]
    assert np.array_equal(bits(g["k_cache"]), bits(c["k_cache"]))


@pytest.mark.parametrize("advance", [0, 1])
def test_a_row_leaving_the_cache_drops_its_earlier_descriptor(advance):
    # Call 1: both rows have keys (row 0's units span several workgroups, so their descriptors
    # record several segments). Call 2, same workspace: row 0 sits past the cache. Its output
    # must be NaN and row 1's must match the oracle.
    H, H_kv, D, T_max = 16, 4, 128, 3000
    _note("descriptor reset", advance)
    first = make_case([2900, 1200], 1, H, H_kv, D, T_max, torch.bfloat16, seed=23)
    _run(first, -1, advance)
    c = make_case([T_max, 1200], 1, H, H_kv, D, T_max, torch.bfloat16, seed=24)
    out, g = _run(c, -1, advance)
    y = to_np(out)
    assert np.isnan(y[0]).all(), "row outside the cache must give NaN"
    want = ko.flash_attn_with_kvcache(to_np(c["q"][1:]), to_np(c["k_cache"][1:]),
                                      to_np(c["v_cache"][1:]), to_np(c["k"][1:]),
                                      to_np(c["v"][1:]), [1200], -1)[0]
    err = max_abs(y[1:], want)
    assert err <= ATOL[torch.bfloat16], f"row 1: max-abs {err}"
    assert g["cache_seqlens"].tolist() == [T_max + advance, 1200 + advance]


def test_captured_steps_with_the_folded_advance_replay_the_eager_steps():
    # Three decode steps (fused path) captured once; each replay must equal three eager steps
    # from the same state, with eager work and synchronisations between the replays.
    B, H, H_kv, D, T_max, steps = 6, 16, 4, 128, 1024, 3
    seqlens = [500, 17, 900, 1, 300, 1000]
    _note("graph", seqlens)
    c = make_case(seqlens, 1, H, H_kv, D, T_max, torch.bfloat16, seed=25)
    gen = torch.Generator().manual_seed(26)
    qs = torch.randn(steps, B, 1, H, D, generator=gen).to(torch.bfloat16).to(DEV)
    ks = torch.randn(steps, B, 1, H_kv, D, generator=gen).to(torch.bfloat16).to(DEV)
    vs = torch.randn(steps, B, 1, H_kv, D, generator=gen).to(torch.bfloat16).to(DEV)
    g = {n: t.to(DEV) for n, t in c.items()}
    outs = [torch.empty(B, 1, H, D, dtype=torch.bfloat16, device=DEV) for _ in range(steps)]

    def run_steps():
        for s in range(steps):
            outs[s].copy_(flash_attn.flash_attn_with_kvcache(
                qs[s], g["k_cache"], g["v_cache"], k=ks[s], v=vs[s],
                cache_seqlens=g["cache_seqlens"], causal=True, window_size=(-1, 0), advance=1))

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
    eager_pos = g["cache_seqlens"].tolist()
    assert eager_pos == [p + steps for p in seqlens]
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
        assert g["cache_seqlens"].tolist() == eager_pos, f"replay {rep}: positions"
        assert np.array_equal(bits(g["k_cache"]), eager_k), f"replay {rep}: cache"
        for s in range(steps):
            assert np.array_equal(bits(outs[s]), eager[s]), f"replay {rep}, step {s}"
        run_steps()  # eager work between replays
        torch.cuda.synchronize()
