"""The fused residual step (mcamd_residual_rmsnorm) and the unsummed GEMM partials
(mcamd_linear_bf16_partials) against torch on the CPU:

* x_out = x + f is bit-exact against torch's bf16 add, with f the bf16 product or the fixed-order
  sum of the K-split partials rounded to bf16 (the sum linear_bf16 itself makes: its output is
  bit-identical to rounding the partials of linear_bf16_partials);
* h = rms_norm(x_out) within one bf16 rounding (2^-8 relative) of F.rms_norm in fp32, whose sum
  of squares runs in another order.
"""
import pytest
import torch
import torch.nn.functional as F

from modelcore_amd.kernels.linear import Partials, linear_bf16, linear_bf16_partials
from modelcore_amd.kernels.residual import residual_rmsnorm

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
EPS = float(torch.finfo(torch.float32).eps)


def _note(*a):
    print("case:", *a, flush=True)


def _ordered_sum(part):
    acc = part[0].clone()
    for s in range(1, part.shape[0]):
        acc = acc + part[s]
    return acc


def _want(x, y_bf16, eps):
    x_out = (x.float() + y_bf16.float()).to(torch.bfloat16)
    h = F.rms_norm(x_out.float(), (x.shape[-1],), eps=eps)
    return x_out, h


def _check(got, want):
    x_out, h = got
    wx, wh = want
    assert torch.equal(x_out.cpu(), wx)
    err = (h.cpu().float() - wh).abs()
    assert torch.all(err <= wh.abs() * 2.0 ** -8 + 1e-6), float(err.max())


@pytest.mark.parametrize("m,n,splits", [(1, 4096, 1), (7, 384, 2), (64, 4096, 4), (33, 8, 3),
                                          (3, 14336, 2), (2, 8200, 1)])
def test_partials_are_summed_added_and_normed(m, n, splits):
    _note("residual partials", m, n, splits)
    g = torch.Generator().manual_seed(m * 7 + n + splits)
    x = torch.randn(m, n, generator=g).to(torch.bfloat16)
    part = torch.randn(splits, m, n, generator=g)
    y = _ordered_sum(part).to(torch.bfloat16)
    got = residual_rmsnorm(x.to(DEV), Partials(part.to(DEV), splits, (m, n)))
    _check(got, _want(x, y, EPS))


def test_a_bf16_f_and_an_explicit_eps():
    _note("residual bf16 f")
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 3, 1536, generator=g).to(torch.bfloat16)
    y = torch.randn(2, 3, 1536, generator=g).to(torch.bfloat16)
    x[0, 0] *= 1e-3  # a small row, where eps weighs in
    x_out, h = residual_rmsnorm(x.to(DEV), y.to(DEV), eps=1e-2)
    assert x_out.shape == x.shape and h.shape == x.shape
    _check((x_out, h), _want(x, y, 1e-2))


@pytest.mark.parametrize("m,n,k", [(64, 4096, 4096), (20, 1024, 3584)])
def test_partials_of_the_gemm_round_to_its_output(m, n, k):
    _note("linear partials", m, n, k)
    g = torch.Generator().manual_seed(m + k)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(n, k, generator=g) * k ** -0.5).to(torch.bfloat16).to(DEV)
    p = linear_bf16_partials(x, w)
    assert p.part.shape == (p.splits, m, n) and p.shape == (m, n)
    assert torch.equal(_ordered_sum(p.part).to(torch.bfloat16), linear_bf16(x, w))
    for s in (1, 2):
        q = linear_bf16_partials(x, w, splits=s)
        assert torch.equal(_ordered_sum(q.part).to(torch.bfloat16), linear_bf16(x, w, s))


def test_bad_arguments_are_refused():
    from modelcore_amd import _ext
    lib = _ext.lib()
    x = torch.zeros(2, 16, dtype=torch.bfloat16, device=DEV)
    part = torch.zeros(1, 2, 16, device=DEV)
    out = torch.empty_like(x)
    assert lib.mcamd_residual_rmsnorm(x.data_ptr(), part.data_ptr(), 1, x.data_ptr(),
                                      out.data_ptr(), out.data_ptr(), 2, 16, EPS, None) < 0
    assert lib.mcamd_residual_rmsnorm(x.data_ptr(), None, 0, None, out.data_ptr(),
                                      out.data_ptr(), 2, 16, EPS, None) < 0
    assert lib.mcamd_residual_rmsnorm(x.data_ptr(), None, 0, x.data_ptr(), out.data_ptr(),
                                      out.data_ptr(), 2, 12, EPS, None) < 0
    with pytest.raises(ValueError):
        residual_rmsnorm(x, torch.zeros(2, 8, dtype=torch.bfloat16, device=DEV))


def test_the_residual_stream_can_be_updated_in_place():
    """x_out = x (the documented in-place form) gives the out-of-place result."""
    from modelcore_amd import _ext
    _note("residual in place")
    g = torch.Generator().manual_seed(21)
    m, n, s = 48, 4096, 4
    x = torch.randn(m, n, generator=g).to(torch.bfloat16).to(DEV)
    part = torch.randn(s, m, n, generator=g).to(DEV)
    want_x, want_h = residual_rmsnorm(x, Partials(part, s, (m, n)))
    h = torch.empty_like(x)
    st = _ext.lib().mcamd_residual_rmsnorm(x.data_ptr(), part.data_ptr(), s, None, x.data_ptr(),
                                           h.data_ptr(), m, n, EPS, _ext.stream_handle(DEV))
    _ext.check(st, "residual_rmsnorm")
    assert torch.equal(x, want_x) and torch.equal(h, want_h)
