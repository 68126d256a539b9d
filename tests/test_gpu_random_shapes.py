"""A seeded sweep of operator shapes against the float64 oracle, beyond the hand-picked cases:
random batch sizes (1-70 rows, ragged, some rows empty), GQA ratios (1-16 query heads per KV
head), head dims (16-256, including ones that are not powers of two), windows (none, 0, short,
longer than the history), T_new of 1 (decode, fused or split-K path) and 2-70 (chunked prefill,
matrix-core or generic path), bf16 and fp32, with the append checked bit for bit; and a second
sweep of bf16 / head_dim 128 chunks (2-600 queries, GQA 1-16 including ratios that do not divide
256, prefixes on and off the 64-key tiles, windows) for the chunked-prefill matrix-core kernel.
Every draw is fixed by its index, so a failure names a reproducible case.
"""
import numpy as np
import pytest
import torch

from _util import ATOL, bits, make_case, max_abs, to_np
from modelcore_amd.kernels.flash_attn import flash_attn
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _draw(i):
    r = np.random.default_rng(1000 + i)
    dtype = torch.bfloat16 if r.random() < 0.75 else torch.float32
    H_kv = int(r.choice([1, 2, 4, 8]))
    G = int(r.choice([1, 2, 3, 4, 8, 16]))
    D = int(r.choice([16, 48, 64, 80, 96, 128, 128, 128, 192, 256, 384, 512]))
    T_new = 1 if r.random() < 0.6 else int(r.integers(2, 71))
    B = int(r.choice([1, 2, 3, 5, 16, 33, 70])) if T_new == 1 else int(r.integers(1, 4))
    T_max = int(r.integers(T_new + 8, 1500 if T_new == 1 else 700))
    lens = r.integers(0, T_max - T_new + 1, B)
    lens[r.random(B) < 0.15] = 0  # some rows with no history
    window = int(r.choice([-1, -1, 0, 7, 64, 5000]))
    return dtype, [int(x) for x in lens], T_new, G * H_kv, H_kv, D, T_max, window


@pytest.mark.parametrize("i", range(40))
def test_random_operator_shapes_match_the_oracle(i):
    dtype, seqlens, T_new, H, H_kv, D, T_max, window = _draw(i)
    print("case: random", i, dtype, len(seqlens), "rows", T_new, H, H_kv, D, T_max, window, flush=True)
    c = make_case(seqlens, T_new, H, H_kv, D, T_max, dtype, seed=2000 + i)
    g = {k: v.to(DEV) for k, v in c.items()}
    out = flash_attn.flash_attn_with_kvcache(g["q"], g["k_cache"], g["v_cache"], k=g["k"], v=g["v"],
                                             cache_seqlens=g["cache_seqlens"], causal=True,
                                             window_size=(window, 0))
    torch.cuda.synchronize()
    want = ko.flash_attn_with_kvcache(to_np(c["q"]), to_np(c["k_cache"]), to_np(c["v_cache"]),
                                      to_np(c["k"]), to_np(c["v"]), seqlens, window)[0]
    err = max_abs(to_np(out), want)
    assert err <= ATOL[dtype], f"case {i}: max-abs {err}"
    ek, ev = ko.append(bits(c["k_cache"]), bits(c["v_cache"]), bits(c["k"]), bits(c["v"]), seqlens)
    assert np.array_equal(bits(g["k_cache"]), ek) and np.array_equal(bits(g["v_cache"]), ev)


def _draw_mfma(i):
    """bf16 / head_dim 128 multi-token shapes: the chunked-prefill matrix-core kernel (256
    (position, head) pairs per workgroup, 64-key tiles, lazy softmax rescale)."""
    r = np.random.default_rng(5000 + i)
    H_kv = int(r.choice([1, 2, 4, 8]))
    G = int(r.choice([1, 2, 3, 4, 5, 6, 8, 12, 16]))
    T_new = int(r.choice([int(r.integers(2, 64)), int(r.integers(64, 257)),
                          int(r.integers(257, 601))]))
    B = int(r.integers(1, 5))
    T_max = int(r.integers(T_new + 1, T_new + 1500))
    lens = r.integers(0, T_max - T_new + 1, B)
    lens[r.random(B) < 0.2] = 0
    on_tile = r.random(B) < 0.3  # some prefixes on a 64-key tile boundary
    lens[on_tile] = (lens[on_tile] // 64) * 64
    window = int(r.choice([-1, -1, -1, 0, 31, 64, 200, 5000]))
    return [int(x) for x in lens], T_new, G * H_kv, H_kv, T_max, window


@pytest.mark.parametrize("i", range(24))
def test_random_matrix_core_prefill_shapes_match_the_oracle(i):
    seqlens, T_new, H, H_kv, T_max, window = _draw_mfma(i)
    print("case: mfma prefill", i, len(seqlens), "rows", seqlens, T_new, H, H_kv, T_max, window,
          flush=True)
    c = make_case(seqlens, T_new, H, H_kv, 128, T_max, torch.bfloat16, seed=6000 + i)
    g = {k: v.to(DEV) for k, v in c.items()}
    out = flash_attn.flash_attn_with_kvcache(g["q"], g["k_cache"], g["v_cache"], k=g["k"], v=g["v"],
                                             cache_seqlens=g["cache_seqlens"], causal=True,
                                             window_size=(window, 0))
    torch.cuda.synchronize()
    want = ko.flash_attn_with_kvcache(to_np(c["q"]), to_np(c["k_cache"]), to_np(c["v_cache"]),
                                      to_np(c["k"]), to_np(c["v"]), seqlens, window)[0]
    err = max_abs(to_np(out), want)
    assert err <= ATOL[torch.bfloat16], f"case {i}: max-abs {err}"
    ek, ev = ko.append(bits(c["k_cache"]), bits(c["v_cache"]), bits(c["k"]), bits(c["v"]), seqlens)
    assert np.array_equal(bits(g["k_cache"]), ek) and np.array_equal(bits(g["v_cache"]), ev)
