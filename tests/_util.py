"""Shared helpers for the tests: seeded inputs (drawn on the CPU, so the oracle and the GPU see
identical bytes), dtype views and tolerances."""
import numpy as np
import torch

# Tolerances of the attention parity checks, per compute dtype (max-abs, after the output is
# rounded to that dtype): bf16 inputs with fp32 accumulation, and fp32 throughout.
ATOL = {torch.bfloat16: 2e-2, torch.float32: 2e-5}


def gen(seed):
    return torch.Generator().manual_seed(seed)


def randn(g, *shape, dtype=torch.float32):
    return torch.randn(*shape, generator=g).to(dtype)


def to_np(t):
    """Float values as a float64 numpy array (bf16 widens exactly)."""
    return t.detach().cpu().to(torch.float64).numpy()


def bits(t):
    """Raw bit patterns of a tensor as numpy (bf16 -> int16, fp32 -> int32)."""
    t = t.detach().cpu().contiguous()
    view = {torch.bfloat16: torch.int16, torch.float32: torch.int32}[t.dtype]
    return t.view(view).numpy()


def make_case(seqlens, T_new, H, H_kv, D, T_max, dtype, seed=0, fill_stale=True):
    """Cache history [0, L_b) per row plus fresh q, k, v, drawn on the CPU from one generator.
    Positions past a row's history hold random data too when fill_stale (a reused cache)."""
    g = gen(seed)
    B = len(seqlens)
    k_cache = randn(g, B, T_max, H_kv, D, dtype=dtype)
    v_cache = randn(g, B, T_max, H_kv, D, dtype=dtype)
    if not fill_stale:
        for b, L in enumerate(seqlens):
            k_cache[b, L:] = 0
            v_cache[b, L:] = 0
    q = randn(g, B, T_new, H, D, dtype=dtype)
    k = randn(g, B, T_new, H_kv, D, dtype=dtype)
    v = randn(g, B, T_new, H_kv, D, dtype=dtype)
    cs = torch.tensor(seqlens, dtype=torch.int32)
    return dict(q=q, k=k, v=v, k_cache=k_cache, v_cache=v_cache, cache_seqlens=cs)


def max_abs(a, b):
    return float(np.max(np.abs(np.asarray(a, dtype=np.float64) - np.asarray(b, dtype=np.float64))))
