"""Planted score patterns that drive the kernels' online softmax through its rare paths, checked
against the float64 oracle.

The decode and chunked-prefill kernels make each tile's weights against a running maximum and
take the tile's own maximum (rescaling the accumulated output) only when the weights outgrow a
limit. Random N(0, 1) inputs never exercise that past the first tile. Here the keys are planted
along one direction of the queries, so the scores:
  * climb along the keys (about 0.05 log2 units per key: the running maximum is overtaken every
    few hundred keys, deep inside long unmasked runs),
  * stay flat except for one late key whose score is ~200 log2 units above the rest (its weight
    overflows fp32 unless the tile is rescaled),
  * fall along the keys (every tile after the first has weights far below the maximum).
Each pattern runs through the chunked prefill (T_new 96, histories of 1500 and 700 keys) and the
decode path (T_new 1), with and without a window.
"""
import numpy as np
import pytest
import torch

from _util import ATOL, bits, max_abs, to_np
from modelcore_amd.kernels.flash_attn import flash_attn
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _planted(pattern, seqlens, T_new, H, H_kv, D, T_max, seed):
    g = torch.Generator().manual_seed(seed)
    B = len(seqlens)
    u = torch.randn(D, generator=g)
    u = u / u.norm()
    q = 8.0 * u.expand(B, T_new, H, D) + 0.05 * torch.randn(B, T_new, H, D, generator=g)
    pos = torch.arange(T_max, dtype=torch.float32)
    if pattern == "climb":
        beta = 0.05 * pos
    elif pattern == "fall":
        beta = 0.05 * (T_max - pos)
    else:
        beta = torch.zeros(T_max)
    k_cache = beta[None, :, None, None] * u + 0.3 * torch.randn(B, T_max, H_kv, D, generator=g)
    if pattern == "spike":
        for b, L in enumerate(seqlens):
            k_cache[b, max(L - 300, 0), :, :] = 200.0 * u
    v_cache = torch.randn(B, T_max, H_kv, D, generator=g)
    k = torch.randn(B, T_new, H_kv, D, generator=g)
    v = torch.randn(B, T_new, H_kv, D, generator=g)
    bf = lambda t: t.to(torch.bfloat16).contiguous()  # noqa: E731
    return dict(q=bf(q), k=bf(k), v=bf(v), k_cache=bf(k_cache), v_cache=bf(v_cache))


@pytest.mark.parametrize("pattern", ["climb", "spike", "fall"])
@pytest.mark.parametrize("T_new", [96, 1])
@pytest.mark.parametrize("window", [-1, 300])
def test_planted_scores_match_the_oracle(pattern, T_new, window):
    seqlens, H, H_kv, D, T_max = [1500, 700], 8, 2, 128, 1700
    print("case: planted", pattern, T_new, window, flush=True)
    c = _planted(pattern, seqlens, T_new, H, H_kv, D, T_max, seed=31)
    g = {n: t.to(DEV) for n, t in c.items()}
    cs = torch.tensor(seqlens, dtype=torch.int32)
    out = flash_attn.flash_attn_with_kvcache(g["q"], g["k_cache"], g["v_cache"], k=g["k"], v=g["v"],
                                             cache_seqlens=cs.to(DEV), causal=True,
                                             window_size=(window, 0))
    torch.cuda.synchronize()
    y = to_np(out)
    assert np.isfinite(y).all(), f"{pattern}: non-finite outputs"
    want = ko.flash_attn_with_kvcache(to_np(c["q"]), to_np(c["k_cache"]), to_np(c["v_cache"]),
                                      to_np(c["k"]), to_np(c["v"]), seqlens, window)[0]
    err = max_abs(y, want)
    assert err <= ATOL[torch.bfloat16], f"{pattern} T_new={T_new} window={window}: max-abs {err}"
    ek, ev = ko.append(bits(c["k_cache"]), bits(c["v_cache"]), bits(c["k"]), bits(c["v"]), seqlens)
    assert np.array_equal(bits(g["k_cache"]), ek) and np.array_equal(bits(g["v_cache"]), ev)
