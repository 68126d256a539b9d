"""Parity of the fused pre-attention step (RoPE + QK-norm + x1.2 + append, one HIP launch) with
its oracle (oracle/epilogue.py: the reference's separate torch ops on the CPU).

The values appended to V and every cache position the call must not touch are bit-exact. q's
result and the appended K may differ from the separate ops by the order of the fp32 sum of
squares inside the norm: the tolerance is one unit in the last place of the storage dtype (bf16:
2^-7 of the value, and at most 2% of the values may differ at all; fp32: 2^-21, a few units).
"""
import pytest
import torch

from modelcore_amd import _ext
from modelcore_amd.kernels.qk_epilogue import rope_norm_scale_append
from modelcore_amd.model import rope_tables
from oracle import epilogue as ep

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
REL = {torch.bfloat16: 2.0 ** -7, torch.float32: 2.0 ** -21}


def _note(*a):
    print("case:", *a, flush=True)


def _close(got, want, dtype):
    got, want = got.float().cpu(), want.float()
    diff = (got - want).abs()
    assert torch.all(diff <= want.abs() * REL[dtype] + 1e-30), float(diff.max())
    if dtype == torch.bfloat16:  # a last-bit change of the fp32 norm factor rarely moves bf16
        assert (diff > 0).float().mean() <= 0.02


def _case(seed, B, T, H, H_kv, D, T_max, n_pos, dtype, seqlens):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g).to(dtype)  # noqa: E731
    cos, sin = rope_tables(n_pos, D, "cpu", dtype)
    return dict(q=r(B, T, H, D) * 3, k=r(B, T, H_kv, D) * 3, v=r(B, T, H_kv, D),
                kc=r(B, T_max, H_kv, D), vc=r(B, T_max, H_kv, D), cos=cos, sin=sin,
                seqlens=torch.tensor(seqlens, dtype=torch.int32))


CASES = [
    # dtype, D, H, H_kv, T, seqlens
    (torch.bfloat16, 128, 16, 4, 1, [5, 5, 5]),
    (torch.bfloat16, 128, 32, 8, 7, [0, 19, 40]),
    (torch.bfloat16, 64, 6, 6, 3, [11, 2, 0]),
    (torch.float32, 64, 12, 4, 1, [3, 60, 9]),
    (torch.float32, 128, 8, 2, 5, [0, 0, 0]),
    (torch.bfloat16, 256, 4, 1, 2, [7, 1, 30]),
]


@pytest.mark.parametrize("dtype,D,H,H_kv,T,seqlens", CASES)
def test_fused_step_matches_the_separate_ops(dtype, D, H, H_kv, T, seqlens):
    _note("epilogue", dtype, D, H, H_kv, T, seqlens)
    B, T_max = len(seqlens), 64
    c = _case(1, B, T, H, H_kv, D, T_max, T_max, dtype, seqlens)
    kc, vc = c["kc"].clone(), c["vc"].clone()
    want_q = ep.rope_norm_scale_append(c["q"], c["cos"], c["sin"], c["seqlens"], c["k"], c["v"],
                                       kc, vc)
    gkc, gvc = c["kc"].to(DEV), c["vc"].to(DEV)
    got_q = rope_norm_scale_append(c["q"].to(DEV), c["cos"].to(DEV), c["sin"].to(DEV),
                                   c["seqlens"].to(DEV), c["k"].to(DEV), c["v"].to(DEV), gkc,
                                   gvc)
    torch.cuda.synchronize()
    _close(got_q, want_q, dtype)
    assert torch.equal(gvc.cpu(), vc)  # V appended bit-exact, nothing else touched
    for b, p in enumerate(seqlens):
        _close(gkc[b, p:p + T], kc[b, p:p + T], dtype)
        keep = [i for i in range(T_max) if not p <= i < p + T]
        assert torch.equal(gkc[b, keep].cpu(), c["kc"][b, keep])


@pytest.mark.parametrize("T", [5, 1])
def test_strided_views_of_a_fused_projection_are_read_in_place(T):
    _note("epilogue strided qkv", T)
    dtype = torch.bfloat16
    B, H, H_kv, D, T_max = 3, 8, 2, 128, 32
    c = _case(6, B, T, H, H_kv, D, T_max, T_max, dtype, [0, 4, 20])
    qkv = torch.cat([c["q"].reshape(B, T, -1), c["k"].reshape(B, T, -1),
                     c["v"].reshape(B, T, -1)], dim=-1).to(DEV)
    q = qkv[..., :H * D].view(B, T, H, D)
    k = qkv[..., H * D:(H + H_kv) * D].view(B, T, H_kv, D)
    v = qkv[..., (H + H_kv) * D:].view(B, T, H_kv, D)
    assert not q.is_contiguous()
    dev = {n: c[n].to(DEV) for n in ("cos", "sin", "seqlens")}
    kc1, vc1 = c["kc"].to(DEV), c["vc"].to(DEV)
    kc2, vc2 = kc1.clone(), vc1.clone()
    a = rope_norm_scale_append(q, dev["cos"], dev["sin"], dev["seqlens"], k, v, kc1, vc1)
    b = rope_norm_scale_append(q.contiguous(), dev["cos"], dev["sin"], dev["seqlens"],
                               k.contiguous(), v.contiguous(), kc2, vc2)
    assert torch.equal(a, b) and torch.equal(kc1, kc2) and torch.equal(vc1, vc2)


def test_queries_only_for_kv_sharing_consumers():
    _note("epilogue q only")
    dtype = torch.bfloat16
    c = _case(2, 2, 4, 8, 2, 128, 32, 32, dtype, [3, 17])
    want = ep.rope_norm_scale(c["q"], c["cos"], c["sin"], c["seqlens"])
    got = rope_norm_scale_append(c["q"].to(DEV), c["cos"].to(DEV), c["sin"].to(DEV),
                                 c["seqlens"].to(DEV))
    _close(got, want, dtype)


def test_explicit_eps_and_scale_reach_the_kernel():
    _note("epilogue eps/scale")
    dtype = torch.float32
    c = _case(3, 2, 2, 4, 4, 64, 16, 16, dtype, [1, 9])
    c["q"][0, 0, 0] = 1e-4  # a tiny row, where eps dominates the norm
    want = ep.rope_norm_scale(c["q"], c["cos"], c["sin"], c["seqlens"], eps=1e-3, scale=0.5)
    got = rope_norm_scale_append(c["q"].to(DEV), c["cos"].to(DEV), c["sin"].to(DEV),
                                 c["seqlens"].to(DEV), eps=1e-3, scale=0.5)
    _close(got, want, dtype)


def test_positions_past_the_table_poison_q_and_leave_the_cache():
    _note("epilogue out of table")
    dtype = torch.bfloat16
    n_pos = 8
    c = _case(4, 2, 2, 4, 2, 64, 16, n_pos, dtype, [3, 7])  # row 1 reaches positions 7, 8
    gkc, gvc = c["kc"].to(DEV), c["vc"].to(DEV)
    got = rope_norm_scale_append(c["q"].to(DEV), c["cos"].to(DEV), c["sin"].to(DEV),
                                 c["seqlens"].to(DEV), c["k"].to(DEV), c["v"].to(DEV), gkc, gvc)
    got = got.cpu()
    assert torch.isnan(got[1, 1]).all() and not torch.isnan(got[1, 0]).any()
    assert torch.equal(gkc[1, 8].cpu(), c["kc"][1, 8])
    assert not torch.isnan(got[0]).any()


def test_the_step_is_stream_ordered_and_syncs_nothing():
    _note("epilogue graph capture")
    dtype = torch.bfloat16
    c = _case(5, 4, 1, 16, 4, 128, 64, 64, dtype, [9, 9, 9, 9])
    q, cos, sin = c["q"].to(DEV), c["cos"].to(DEV), c["sin"].to(DEV)
    k, v = c["k"].to(DEV), c["v"].to(DEV)
    seqlens = c["seqlens"].to(DEV)
    kc, vc = c["kc"].to(DEV), c["vc"].to(DEV)
    eager = rope_norm_scale_append(q, cos, sin, seqlens, k, v, kc, vc)
    ref_k = kc.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        rope_norm_scale_append(q, cos, sin, seqlens, k, v, kc, vc)  # warm-up on the side stream
        with torch.cuda.graph(graph, stream=s):
            out = rope_norm_scale_append(q, cos, sin, seqlens, k, v, kc, vc)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(3):
        kc.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        assert torch.equal(kc[:, 9], ref_k[:, 9]), i
    assert _ext.lib() is not None


@pytest.mark.parametrize("with_kv", [True, False], ids=["producer", "q-only"])
def test_partials_of_the_qkv_projection_give_the_summed_projection_result(with_kv):
    """The epilogue fed the unsummed K-split partials of the stacked QKV product equals, bit for
    bit, the epilogue fed that product's bf16 output (q, caches); the partials' in-order sum
    rounded to bf16 is exactly what the GEMM outputs."""
    from modelcore_amd.kernels.linear import linear_bf16, linear_bf16_partials
    from modelcore_amd.kernels.qk_epilogue import rope_norm_scale_append_partials
    _note("epilogue from qkv partials", with_kv)
    B, H, H_kv, D, T_max, K = 5, 8, 2, 128, 40, 1024
    g = torch.Generator().manual_seed(12)
    n = (H + (2 * H_kv if with_kv else 0)) * D
    x = torch.randn(B, 1, K, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(n, K, generator=g) * K ** -0.5).to(torch.bfloat16).to(DEV)
    cos, sin = (t.to(DEV) for t in rope_tables(64, D, "cpu", torch.bfloat16))
    seqlens = torch.tensor([0, 3, 17, 30, 38], dtype=torch.int32, device=DEV)
    kc = torch.randn(B, T_max, H_kv, D, generator=g).to(torch.bfloat16).to(DEV)
    vc = torch.randn(B, T_max, H_kv, D, generator=g).to(torch.bfloat16).to(DEV)
    kc2, vc2 = kc.clone(), vc.clone()
    part = linear_bf16_partials(x, w, splits=4)
    got = rope_norm_scale_append_partials(part, H, H_kv, cos, sin, seqlens,
                                          kc if with_kv else None, vc if with_kv else None)
    y = linear_bf16(x, w, 4)
    q = y[..., :H * D].view(B, 1, H, D)
    if with_kv:
        k = y[..., H * D:(H + H_kv) * D].view(B, 1, H_kv, D)
        v = y[..., (H + H_kv) * D:].view(B, 1, H_kv, D)
        want = rope_norm_scale_append(q, cos, sin, seqlens, k, v, kc2, vc2)
    else:
        want = rope_norm_scale_append(q, cos, sin, seqlens)
    assert torch.equal(got, want)
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
