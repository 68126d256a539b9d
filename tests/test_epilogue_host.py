"""Pins the oracle of the pre-attention step (oracle/epilogue.py) on the CPU.

The checks do not retype its formula: it must equal the model harness's own RoPE / RMSNorm /
x1.2 composition (the modules the reference goldens pin, tests/test_model_host.py), RoPE at
position 0 must be the identity, a rotation must keep each (j, j + D/2) pair's length and make
q.k depend only on the distance of the two positions, the rotation must run by -theta (the
reference's convention, modelcore/components/rope.py:6-7), the norm must leave unit mean
square, and the append must touch the new positions only. A planted sign error must fail.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from modelcore_amd.model import RMSNorm, Rotary, rope_tables
from modelcore_amd.runtime import Runtime
from oracle import epilogue as ep


class _Cache:
    """What Rotary reads from a KV cache: the uniform position, or the per-row lengths."""

    def __init__(self, seqlens, uniform):
        self.cache_seqlens = seqlens
        self._uniform = uniform

    def uniform_pos(self):
        return int(self.cache_seqlens[0]) if self._uniform else None


def _harness(q, k, seqlens, uniform, dtype, n_pos, eps=None):
    rt = Runtime()
    rt.compute_dtype = dtype
    D = q.shape[-1]
    rope = Rotary(D, n_pos, 1, rt)
    norm = RMSNorm(eps)
    qr, kr = rope(q, k, _Cache(seqlens, uniform))
    return norm(qr) * 1.2, norm(kr) * 1.2, rope


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("uniform", [True, False])
def test_oracle_equals_the_harness_composition(dtype, uniform):
    g = torch.Generator().manual_seed(1)
    B, T, H, H_kv, D, n_pos = 3, 4, 6, 2, 64, 40
    q = torch.randn(B, T, H, D, generator=g).to(dtype)
    k = torch.randn(B, T, H_kv, D, generator=g).to(dtype)
    seqlens = torch.tensor([7, 7, 7] if uniform else [0, 13, 30], dtype=torch.int32)
    hq, hk, rope = _harness(q, k, seqlens, uniform, dtype, n_pos)
    oq = ep.rope_norm_scale(q, rope.cos, rope.sin, seqlens)
    ok = ep.rope_norm_scale(k, rope.cos, rope.sin, seqlens)
    assert torch.equal(oq, hq) and torch.equal(ok, hk)


def test_rope_at_position_zero_is_the_identity():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 1, 4, 32, generator=g).to(torch.bfloat16)
    cos, sin = rope_tables(8, 32, "cpu", torch.bfloat16)
    zero = torch.zeros(2, dtype=torch.int32)
    got = ep.rope_norm_scale(x, cos, sin, zero, scale=1.0)
    assert torch.equal(got, F.rms_norm(x, (32,)))


def test_rotation_keeps_pair_lengths_and_depends_on_distance_only():
    g = torch.Generator().manual_seed(3)
    D = 16
    cos, sin = rope_tables(64, D, "cpu", torch.float32)
    q = torch.randn(1, 1, 1, D, generator=g, dtype=torch.float64).float()
    k = torch.randn(1, 1, 1, D, generator=g, dtype=torch.float64).float()

    def rot(x, p):
        c, s = ep._windows(cos, sin, torch.tensor([p], dtype=torch.int32), 1)
        return ep.apply_rotary(x, c, s)

    y = rot(q, 37)
    h = D // 2
    before = q[..., :h] ** 2 + q[..., h:] ** 2
    after = y[..., :h] ** 2 + y[..., h:] ** 2
    torch.testing.assert_close(after, before, rtol=1e-5, atol=1e-6)
    dots = [float((rot(q, p + 5) * rot(k, p)).sum()) for p in (0, 9, 30)]
    assert max(dots) - min(dots) < 1e-4


def test_rotation_runs_by_minus_theta():
    # One pair (D = 2) at angle pi/2: x = (1, 0) goes to (cos, -sin) = (0, -1).
    cos = torch.tensor([[1.0], [0.0]])
    sin = torch.tensor([[0.0], [1.0]])
    x = torch.tensor([1.0, 0.0]).view(1, 1, 1, 2)
    c, s = ep._windows(cos, sin, torch.tensor([1], dtype=torch.int32), 1)
    assert ep.apply_rotary(x, c, s).flatten().tolist() == [0.0, -1.0]


def test_norm_leaves_unit_mean_square_times_the_scale():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 3, 5, 64, generator=g) * 7
    cos, sin = rope_tables(16, 64, "cpu", torch.float32)
    y = ep.rope_norm_scale(x, cos, sin, torch.tensor([2, 9], dtype=torch.int32), scale=1.2)
    ms = (y / 1.2).pow(2).mean(-1)
    torch.testing.assert_close(ms, torch.ones_like(ms), rtol=1e-5, atol=1e-5)


def test_append_writes_only_the_new_positions():
    g = torch.Generator().manual_seed(5)
    B, T, H, H_kv, D, T_max = 2, 3, 4, 2, 16, 12
    q = torch.randn(B, T, H, D, generator=g)
    k = torch.randn(B, T, H_kv, D, generator=g)
    v = torch.randn(B, T, H_kv, D, generator=g)
    kc = torch.randn(B, T_max, H_kv, D, generator=g)
    vc = torch.randn(B, T_max, H_kv, D, generator=g)
    kc0, vc0 = kc.clone(), vc.clone()
    cos, sin = rope_tables(T_max, D, "cpu", torch.float32)
    seqlens = torch.tensor([1, 6], dtype=torch.int32)
    ep.rope_norm_scale_append(q, cos, sin, seqlens, k, v, kc, vc)
    kt = ep.rope_norm_scale(k, cos, sin, seqlens)
    for b, p in enumerate([1, 6]):
        assert torch.equal(kc[b, p:p + T], kt[b]) and torch.equal(vc[b, p:p + T], v[b])
        keep = [i for i in range(T_max) if not p <= i < p + T]
        assert torch.equal(kc[b, keep], kc0[b, keep]) and torch.equal(vc[b, keep], vc0[b, keep])


def test_a_planted_sign_error_is_caught(monkeypatch):
    def wrong(x, cos, sin):
        d = x.shape[3] // 2
        x1, x2 = x[..., :d], x[..., d:]
        return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], 3)  # rotates by +theta

    monkeypatch.setattr(ep, "apply_rotary", wrong)
    with pytest.raises(AssertionError):
        test_oracle_equals_the_harness_composition(torch.float32, False)
    with pytest.raises(AssertionError):
        test_rotation_runs_by_minus_theta()


@pytest.mark.parametrize("T", [1, 3])
def test_views_of_a_fused_projection_are_taken_in_place(T):
    """q/k/v views of a (B, T, H*D + 2*H_kv*D) projection reach the kernel without a copy, one
    token per row (a decode step, where torch gives the size-1 token dim an arbitrary stride)
    included; their token stride is the projection's row width."""
    from modelcore_amd.kernels.qk_epilogue import _token_rows
    B, H, H_kv, D = 4, 8, 2, 16
    n = (H + 2 * H_kv) * D
    qkv = torch.zeros(B, T, n)
    for lo, heads in ((0, H), (H * D, H_kv), ((H + H_kv) * D, H_kv)):
        view = qkv[..., lo:lo + heads * D].view(B, T, heads, D)
        t, stride = _token_rows(view)
        assert t.data_ptr() == view.data_ptr() and stride == n
    c = torch.zeros(B, T, H, D).transpose(0, 1)  # rows not evenly strided: copied
    t, stride = _token_rows(c)
    assert t.is_contiguous() and stride == H * D
