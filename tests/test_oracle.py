"""Pins the CPU oracle (oracle/kv_oracle.py) before any kernel is compared with it.

Each check is independent of the oracle's own formula: pure-Python float64 brute force, torch's
scaled_dot_product_attention through the restated reference fallback (the library routine the
reference calls), closed forms, and the reference's own invariants (test_kernels.py:420-545,
test_cache.py:38-56) restated on the oracle. Planted mistakes in the oracle must fail them.
"""
import math

import numpy as np
import pytest
import torch

from _util import bits, gen, make_case, randn, to_np
from oracle import kv_oracle as ko
from oracle import sdpa_fallback as sf


def brute_force(q, kc, vc, seqlens, window):
    """Attention by explicit loops over (row, query, head, key), float64 via math.exp."""
    B, T, H, D = q.shape
    G = H // kc.shape[2]
    out = np.zeros((B, T, H, D))
    for b in range(B):
        for t in range(T):
            p = int(seqlens[b]) + t
            cols = [c for c in range(p + 1) if window < 0 or p - c <= window]
            for h in range(H):
                kvh = h // G
                s = [sum(q[b, t, h, d] * kc[b, c, kvh, d] for d in range(D)) / math.sqrt(D)
                     for c in cols]
                m = max(s)
                w = [math.exp(x - m) for x in s]
                z = sum(w)
                for d in range(D):
                    out[b, t, h, d] = sum(wi * vc[b, c, kvh, d] for wi, c in zip(w, cols)) / z
    return out


CASES = [
    # seqlens, T_new, H, H_kv, D, window
    ([5, 0, 9], 1, 2, 1, 4, -1),
    ([5, 0, 9], 1, 4, 2, 4, 3),
    ([3, 7], 3, 4, 4, 8, -1),
    ([3, 7], 3, 6, 2, 4, 2),
    ([6, 6], 2, 4, 1, 4, 0),
    ([0], 6, 2, 2, 4, 4),
    ([11], 1, 3, 1, 8, 5),
]


@pytest.mark.parametrize("seqlens,T_new,H,H_kv,D,window", CASES)
def test_oracle_attention_matches_brute_force(seqlens, T_new, H, H_kv, D, window):
    c = make_case(seqlens, T_new, H, H_kv, D, T_max=16, dtype=torch.float64, seed=len(seqlens) + D)
    out, kc, vc = ko.flash_attn_with_kvcache(to_np(c["q"]), to_np(c["k_cache"]), to_np(c["v_cache"]),
                                             to_np(c["k"]), to_np(c["v"]), seqlens, window)
    ref = brute_force(to_np(c["q"]), kc, vc, seqlens, window)
    np.testing.assert_allclose(out, ref, atol=1e-12, rtol=0)


SDPA_CASES = [
    # seqlens, T_new, H, H_kv, D, window, force_ragged -- covers every branch of the fallback:
    ([9, 9], 1, 4, 2, 16, -1, False),    # uniform single token, unmasked
    ([9, 9], 1, 4, 2, 16, 3, False),     # uniform single token, sliced window
    ([0, 0], 12, 4, 2, 16, -1, False),   # uniform prompt, is_causal
    ([0, 0], 12, 4, 1, 16, 5, False),    # uniform prompt, window < T: explicit mask
    ([7, 7], 5, 8, 2, 16, -1, False),    # uniform chunk against a prefix: explicit mask
    ([7, 7], 5, 8, 2, 16, 4, False),
    ([4, 17, 31, 9], 1, 4, 4, 16, -1, False),  # ragged decode
    ([4, 17, 31, 9], 3, 4, 2, 16, 8, False),   # ragged chunk + window
    ([13], 1, 4, 1, 16, 8, True),        # forced-ragged mask at batch 1
]


@pytest.mark.parametrize("seqlens,T_new,H,H_kv,D,window,force", SDPA_CASES)
def test_oracle_matches_reference_sdpa_fallback(seqlens, T_new, H, H_kv, D, window, force):
    c = make_case(seqlens, T_new, H, H_kv, D, T_max=48, dtype=torch.float64, seed=3)
    kc_t, vc_t = c["k_cache"].clone(), c["v_cache"].clone()
    y = sf.flash_attn_with_kvcache(c["q"], kc_t, vc_t, c["k"], c["v"], c["cache_seqlens"],
                                   (window, 0), force_ragged=force)
    out, kc, vc = ko.flash_attn_with_kvcache(to_np(c["q"]), to_np(c["k_cache"]), to_np(c["v_cache"]),
                                             to_np(c["k"]), to_np(c["v"]), seqlens, window)
    np.testing.assert_allclose(out, to_np(y), atol=1e-10, rtol=0)
    assert np.array_equal(kc, to_np(kc_t)) and np.array_equal(vc, to_np(vc_t))


def test_varlen_restatement_matches_brute_force_per_sequence():
    """The varlen form of the fallback (sequences packed along one token axis, each in its own
    cache row at that row's position) against pure-Python brute force per sequence, and the
    appends at each row's own positions; rows not listed keep their contents."""
    g = gen(5)
    B_cache, T_max, H, H_kv, D = 4, 20, 4, 2, 8
    kc = randn(g, B_cache, T_max, H_kv, D, dtype=torch.float64)
    vc = randn(g, B_cache, T_max, H_kv, D, dtype=torch.float64)
    rows, bases, lengths = [2, 0, 3], [4, 0, 9], [3, 6, 1]
    total = sum(lengths)
    q = randn(g, total, H, D, dtype=torch.float64)
    k = randn(g, total, H_kv, D, dtype=torch.float64)
    v = randn(g, total, H_kv, D, dtype=torch.float64)
    seqlens = torch.zeros(B_cache, dtype=torch.int32)
    seqlens[rows] = torch.tensor(bases, dtype=torch.int32)
    cu = torch.tensor([0, 3, 9, 10], dtype=torch.int32)
    kc2, vc2 = kc.clone(), vc.clone()
    y = sf.flash_attn_varlen_with_kvcache(q, kc2, vc2, k, v, seqlens.clone(), cu, 6,
                                          torch.tensor(rows, dtype=torch.int32),
                                          window_size=(4, 0))
    a = 0
    for r, s0, n in zip(rows, bases, lengths):
        want_k, want_v = kc[r].clone(), vc[r].clone()
        want_k[s0:s0 + n], want_v[s0:s0 + n] = k[a:a + n], v[a:a + n]
        assert torch.equal(kc2[r], want_k) and torch.equal(vc2[r], want_v)
        want = brute_force(to_np(q[a:a + n])[None], to_np(want_k)[None], to_np(want_v)[None],
                           [s0], 4)[0]
        np.testing.assert_allclose(to_np(y[a:a + n]), want, atol=1e-10, rtol=0)
        a += n
    assert torch.equal(kc2[1], kc[1]) and torch.equal(vc2[1], vc[1])


def test_window_zero_returns_each_rows_own_value():
    """w = 0: every query sees only itself, so the output is its own V row exactly."""
    seqlens, T_new, H, H_kv = [3, 10], 4, 4, 2
    c = make_case(seqlens, T_new, H, H_kv, 8, 16, torch.float64, seed=5)
    out, _, vc = ko.flash_attn_with_kvcache(to_np(c["q"]), to_np(c["k_cache"]), to_np(c["v_cache"]),
                                            to_np(c["k"]), to_np(c["v"]), seqlens, 0)
    for b, L in enumerate(seqlens):
        for t in range(T_new):
            for h in range(H):
                np.testing.assert_allclose(out[b, t, h], vc[b, L + t, h // 2], atol=1e-15)


def test_constant_values_come_back_unchanged():
    c = make_case([6, 2], 2, 4, 2, 8, 16, torch.float64, seed=6)
    vconst = np.full(c["v_cache"].shape, 0.375)
    out = ko.attention(to_np(c["q"]), to_np(c["k_cache"]), vconst, [6, 2], -1)
    np.testing.assert_allclose(out, 0.375, atol=1e-15)


def test_equal_keys_average_the_visible_values():
    """All keys equal: uniform weights, so the output is the mean of the visible V rows."""
    seqlens, window = [9, 4], 3
    c = make_case(seqlens, 1, 2, 1, 4, 16, torch.float64, seed=7)
    kc = np.broadcast_to(to_np(c["k_cache"])[:, :1], c["k_cache"].shape).copy()
    vc = to_np(c["v_cache"])
    out = ko.attention(to_np(c["q"]), kc, vc, seqlens, window)
    for b, L in enumerate(seqlens):
        lo = max(0, L - window)
        np.testing.assert_allclose(out[b, 0, 0], vc[b, lo:L + 1, 0].mean(axis=0), atol=1e-14)


# --- the reference's invariants (modelcore/tests/test_kernels.py:420-545), on the oracle --------

@pytest.mark.parametrize("window", [-1, 8])
@pytest.mark.parametrize("T_new", [1, 3])
def test_batched_ragged_equals_each_row_alone(window, T_new):
    seqlens = [4, 17, 31, 9]
    c = make_case(seqlens, T_new, 4, 4, 16, 48, torch.float64, seed=0)
    args = [to_np(c[n]) for n in ("q", "k_cache", "v_cache", "k", "v")]
    out, _, _ = ko.flash_attn_with_kvcache(*args, seqlens, window)
    for b, L in enumerate(seqlens):
        row = [a[b:b + 1] for a in args]
        o, _, _ = ko.flash_attn_with_kvcache(*row, [L], window)
        np.testing.assert_allclose(out[b:b + 1], o, atol=1e-13)


def test_stale_kv_beyond_a_rows_content_is_unreachable():
    seqlens = [4, 17, 31, 9]
    c = make_case(seqlens, 1, 4, 4, 16, 48, torch.float64, seed=1)
    args = [to_np(c[n]) for n in ("q", "k_cache", "v_cache", "k", "v")]
    clean, _, _ = ko.flash_attn_with_kvcache(*args, seqlens)
    dk, dv = args[1].copy(), args[2].copy()
    for b, L in enumerate(seqlens):
        dk[b, L + 1:] = 1e4
        dv[b, L + 1:] = -1e4
    dirty, _, _ = ko.flash_attn_with_kvcache(args[0], dk, dv, args[3], args[4], seqlens)
    assert np.array_equal(clean, dirty)


def test_new_tokens_land_at_each_rows_own_offset():
    seqlens = [4, 17, 31, 9]
    c = make_case(seqlens, 1, 4, 4, 16, 48, torch.bfloat16, seed=2)
    kb, kcb = bits(c["k"]), bits(c["k_cache"])
    kc2, _ = ko.append(kcb, bits(c["v_cache"]), kb, bits(c["v"]), seqlens)
    for b, L in enumerate(seqlens):
        assert np.array_equal(kc2[b, L], kb[b, 0])
        untouched = np.ones(48, dtype=bool)
        untouched[L] = False
        assert np.array_equal(kc2[b][untouched], kcb[b][untouched])


def test_sliding_window_is_measured_from_each_rows_own_position():
    window = 8
    c = make_case([3, 20], 1, 4, 4, 16, 48, torch.float64, seed=3)
    q, kc, vc, k, v = (to_np(c[n]) for n in ("q", "k_cache", "v_cache", "k", "v"))
    base, _, _ = ko.flash_attn_with_kvcache(q, kc, vc, k, v, [3, 20], window)
    far = kc.copy()
    far[1, :10] += 5.0  # row 1 (position 20) sees only [12, 20]
    assert np.array_equal(base[1], ko.flash_attn_with_kvcache(q, far, vc, k, v, [3, 20], window)[0][1])
    near = kc.copy()
    near[0, 0] += 5.0  # row 0 (position 3) sees its whole history
    assert not np.array_equal(base[0], ko.flash_attn_with_kvcache(q, near, vc, k, v, [3, 20], window)[0][0])


def test_append_matches_explicit_loops_and_rejects_overflow():
    seqlens, T_new = [0, 5, 11], 3
    c = make_case(seqlens, T_new, 2, 2, 8, 14, torch.float32, seed=4)
    kc, vc = bits(c["k_cache"]), bits(c["v_cache"])
    k, v = bits(c["k"]), bits(c["v"])
    kc2, vc2 = ko.append(kc, vc, k, v, seqlens)
    ek, ev = kc.copy(), vc.copy()
    for b, L in enumerate(seqlens):
        for t in range(T_new):
            for h in range(2):
                for d in range(8):
                    ek[b, L + t, h, d] = k[b, t, h, d]
                    ev[b, L + t, h, d] = v[b, t, h, d]
    assert np.array_equal(kc2, ek) and np.array_equal(vc2, ev)
    with pytest.raises(IndexError):
        ko.append(kc, vc, k, v, [0, 5, 12])


def test_replicate_matches_the_reference_broadcast():
    g = gen(5)
    src_k, src_v = randn(g, 2, 1, 7, 2, 8), randn(g, 2, 1, 7, 2, 8)
    dst_k, dst_v = torch.zeros(2, 4, 24, 2, 8), torch.zeros(2, 4, 24, 2, 8)
    ok, ov = ko.replicate(dst_k.numpy(), dst_v.numpy(), src_k.numpy(), src_v.numpy(), 7, range(4))
    sf.replicate(dst_k, dst_v, src_k, src_v, 7)
    assert np.array_equal(ok, dst_k.numpy()) and np.array_equal(ov, dst_v.numpy())
    for r in range(4):
        assert np.array_equal(ok[:, r, :7], src_k.numpy()[:, 0])
    assert not ok[:, :, 7:].any()
    one_k, _ = ko.replicate(torch.zeros(2, 3, 24, 2, 8).numpy(), torch.zeros(2, 3, 24, 2, 8).numpy(),
                            src_k.numpy(), src_v.numpy(), 7, [1])
    assert not one_k[:, 0].any() and not one_k[:, 2].any()


# --- planted mistakes: each must be caught by the brute-force check -----------------------------

def _planted(kind, q, kc, vc, seqlens, window):
    H, H_kv = q.shape[2], kc.shape[2]
    if kind == "window_off_by_one":
        return ko.attention(q, kc, vc, seqlens, window + 1)
    if kind == "gqa_modulo_map":
        return ko.attention(q, kc, vc, seqlens, window, head_map=np.arange(H) % H_kv)
    if kind == "no_scale":
        return ko.attention(q, kc, vc, seqlens, window, scale=1.0)
    if kind == "positions_from_zero":
        return ko.attention(q, kc, vc, [0] * len(seqlens), window)
    raise ValueError(kind)


@pytest.mark.parametrize("kind", ["window_off_by_one", "gqa_modulo_map", "no_scale",
                                  "positions_from_zero"])
def test_planted_oracle_mistakes_are_caught(kind):
    seqlens, window = [6, 9], 3
    c = make_case(seqlens, 2, 4, 2, 4, 16, torch.float64, seed=8)
    q, kc, vc, k, v = (to_np(c[n]) for n in ("q", "k_cache", "v_cache", "k", "v"))
    kc, vc = ko.append(kc, vc, k, v, seqlens)
    ref = brute_force(q, kc, vc, seqlens, window)
    assert np.max(np.abs(_planted(kind, q, kc, vc, seqlens, window) - ref)) > 1e-3
