"""The decode-sized bf16 product y = x . W^T (mcamd_linear_bf16) against float64 products of the
same bf16 values (numpy), for the projection shapes of the decode workloads and edge sizes.

Tolerance: the bf16 rounding of the output (2^-8 of |y|) plus fp32 accumulation, bounded by
1e-5 of sum_k |x_k w_k|. The kernel sums its K-split partials in a fixed order, so two calls with
the same split are bit-identical.
"""
import numpy as np
import pytest
import torch

from modelcore_amd.kernels.linear import linear_bf16, supported

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _note(*a):
    print("case:", *a, flush=True)


def _check(y, x, w):
    xd = x.float().cpu().double().numpy().reshape(-1, x.shape[-1])
    wd = w.float().cpu().double().numpy()
    ref = xd @ wd.T
    bound = np.abs(xd) @ np.abs(wd).T
    got = y.float().cpu().double().numpy().reshape(ref.shape)
    err = np.abs(got - ref)
    assert np.all(err <= np.abs(ref) * 2.0 ** -8 + 1e-5 * bound + 1e-30), float(err.max())


SHAPES = [(1, 1024, 512), (7, 4096, 4096), (33, 1024, 1536), (64, 14336, 4096),
          (64, 4096, 14336), (32, 6144, 4096), (64, 32768, 1024), (48, 28672, 4096),
          (16, 4096, 4096), (20, 24640, 512)]  # the last: 128-row tiles, the last one half full


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_products_match_float64(m, n, k):
    _note("linear", m, n, k)
    g = torch.Generator().manual_seed(m + n + k)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(n, k, generator=g) * k ** -0.5).to(torch.bfloat16).to(DEV)
    y = linear_bf16(x, w)
    _check(y, x, w)
    assert torch.equal(y, linear_bf16(x, w))  # deterministic


@pytest.mark.parametrize("splits", [1, 2, 4, 8])
def test_every_k_split_matches_float64(splits):
    _note("linear k_splits", splits)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(40, 2048, generator=g).to(torch.bfloat16).to(DEV)
    w = torch.randn(2048, 2048, generator=g).to(torch.bfloat16).to(DEV)
    y = linear_bf16(x, w, splits)
    _check(y, x, w)
    assert torch.equal(y, linear_bf16(x, w, splits))


def test_strided_rows_and_leading_dims():
    _note("linear strided")
    g = torch.Generator().manual_seed(10)
    wide = torch.randn(3, 4, 1536, generator=g).to(torch.bfloat16).to(DEV)
    x = wide[..., :1024]  # rows 1536 elements apart
    w = torch.randn(512, 1024, generator=g).to(torch.bfloat16).to(DEV)
    y = linear_bf16(x, w)
    assert y.shape == (3, 4, 512)
    _check(y, x, w)


def test_unsupported_shapes_are_refused():
    x = torch.zeros(65, 512, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(64, 512, dtype=torch.bfloat16, device=DEV)
    assert not supported(x, w)
    with pytest.raises(ValueError):
        linear_bf16(x, w)
    assert not supported(x[:8, :500], w[:, :500])  # k not a multiple of 128
    assert not supported(x[:8], w[:32])  # n not a multiple of 64
    assert not supported(x[:8].float(), w.float())


@pytest.mark.parametrize("tiled", [False, True], ids=["row-major", "tiled"])
@pytest.mark.parametrize("m,hid,k", [(64, 14336, 4096), (5, 768, 384), (64, 128, 1024)])
def test_gated_silu_product_matches_the_separate_bf16_ops(m, hid, k, tiled):
    """linear_bf16_gated on the interleaved [W_gate; W_up] against torch's silu(g) * u of the
    kernel's own bf16 products g = x W_gate^T, u = x W_up^T (one K split, so the same fp32 sums):
    within one bf16 rounding (torch's exp and this kernel's may differ in the last fp32 bit)."""
    from modelcore_amd.kernels.linear import interleave_gate_up, linear_bf16_gated, tile_weight
    _note("linear gated", m, hid, k, tiled)
    g = torch.Generator().manual_seed(m + hid + k)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16).to(DEV)
    wg = (torch.randn(hid, k, generator=g) * k ** -0.5).to(torch.bfloat16).to(DEV)
    wu = (torch.randn(hid, k, generator=g) * k ** -0.5).to(torch.bfloat16).to(DEV)
    w = interleave_gate_up(wg, wu)
    h = linear_bf16_gated(x, tile_weight(w) if tiled else w)
    gate, up = linear_bf16(x, wg, 1), linear_bf16(x, wu, 1)
    want = (torch.nn.functional.silu(gate.float()).to(torch.bfloat16).float() * up.float())
    err = (h.float() - want).abs()
    assert torch.all(err <= want.abs() * 2.0 ** -7 + 1e-6), float(err.max())
    assert (h.float() == want.to(torch.bfloat16).float()).float().mean() > 0.99


def test_a_captured_split_product_survives_a_larger_eager_call():
    """A graph captured around a K-split product holds the workspace's address. An eager call
    that needs a larger workspace replaces the buffer; the old one must stay allocated, so the
    replays (with other eager work and allocations between them) still match the eager result."""
    from modelcore_amd.kernels import linear as lin
    g = torch.Generator().manual_seed(81)
    x = torch.randn(16, 4096, generator=g).to(torch.bfloat16).to(DEV)
    w = torch.randn(1024, 4096, generator=g).to(torch.bfloat16).to(DEV)
    assert lin.k_splits(16, 1024, 4096) > 1
    lin._RETIRED.extend(lin._WS.values())  # start from a workspace just large enough for this
    lin._WS.clear()                         # product (earlier buffers stay alive)
    eager = linear_bf16(x, w).clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = linear_bf16(x, w)
    big_x = torch.randn(64, 8192, generator=g).to(torch.bfloat16).to(DEV)
    big_w = torch.randn(4096, 8192, generator=g).to(torch.bfloat16).to(DEV)
    old = lin._WS[DEV.index]
    linear_bf16(big_x, big_w, splits=16)  # grows the workspace
    assert lin._WS[DEV.index] is not old
    for i in range(3):
        junk = [torch.full((1 << 20,), 7.0, device=DEV) for _ in range(8)]  # reuse freed blocks
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), i
        del junk
