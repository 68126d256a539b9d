"""The cached-attention entry point that allocates nothing (mcamd_flash_attn_with_kvcache_noalloc):
its scratch is a static device array, and its results must be those of the workspace entry
point bit for bit (same kernels, same work split), call after call, also when a later call is
smaller than an earlier one (the array keeps the last call's partials), and against the oracle.
"""
import numpy as np
import pytest
import torch

from _util import ATOL, bits, make_case, max_abs, to_np
from modelcore_amd import _ext
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _run(entry, c, window, dtype):
    g = {k: v.to(DEV) for k, v in c.items()}
    B, T_new, H, D = g["q"].shape
    T_max, H_kv = g["k_cache"].shape[1], g["k_cache"].shape[2]
    out = torch.full((B, T_new, H, D), float("nan"), dtype=dtype, device=DEV)
    lib = _ext.lib()
    args = [g["q"].data_ptr(), g["k"].data_ptr(), g["v"].data_ptr(), g["k_cache"].data_ptr(),
            g["v_cache"].data_ptr(), g["cache_seqlens"].data_ptr(), out.data_ptr(), B, T_new, H,
            H_kv, D, T_max, g["k_cache"].stride(0), window, 1, _ext.dtype_code(dtype)]
    stream = _ext.stream_handle(DEV)
    if entry == "noalloc":
        st = lib.mcamd_flash_attn_with_kvcache_noalloc(*args, stream)
    else:
        need = lib.mcamd_attn_workspace_bytes(B, T_new, H, H_kv, D, T_max, window)
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=DEV)
        st = lib.mcamd_flash_attn_with_kvcache(*args, ws.data_ptr(), need, stream)
    _ext.check(st, entry)
    torch.cuda.synchronize()
    return out, g


CALLS = [
    # seqlens, T_new, H, H_kv, D, T_max, window, dtype: a large call, then smaller ones
    ([int(x) for x in np.random.default_rng(8).integers(2048, 2560, 64)], 1, 32, 8, 128, 2560, -1,
     torch.bfloat16),
    ([int(x) for x in np.random.default_rng(9).integers(300, 4000, 32)], 1, 16, 4, 128, 4096, -1,
     torch.bfloat16),
    ([100, 7, 900], 1, 16, 4, 128, 1024, 64, torch.bfloat16),
    ([40, 3], 1, 8, 2, 64, 64, -1, torch.float32),
    ([30, 0], 40, 16, 4, 128, 128, -1, torch.bfloat16),
]


def test_noalloc_entry_point_equals_the_workspace_entry_point():
    for i, (seqlens, T_new, H, H_kv, D, T_max, window, dtype) in enumerate(CALLS):
        print("case: noalloc call", i, len(seqlens), "rows", T_new, H, H_kv, D, T_max, window,
              dtype, flush=True)
        c = make_case(seqlens, T_new, H, H_kv, D, T_max, dtype, seed=90 + i)
        a, ga = _run("workspace", c, window, dtype)
        b, gb = _run("noalloc", c, window, dtype)
        assert torch.equal(a, b), f"call {i}: outputs differ"
        assert torch.equal(ga["k_cache"], gb["k_cache"]) and torch.equal(ga["v_cache"], gb["v_cache"])
        want = ko.flash_attn_with_kvcache(to_np(c["q"]), to_np(c["k_cache"]), to_np(c["v_cache"]),
                                          to_np(c["k"]), to_np(c["v"]), seqlens, window)[0]
        err = max_abs(to_np(b), want)
        assert err <= ATOL[dtype], f"call {i}: max-abs {err}"
        ek, _ = ko.append(bits(c["k_cache"]), bits(c["v_cache"]), bits(c["k"]), bits(c["v"]), seqlens)
        assert np.array_equal(bits(gb["k_cache"]), ek)


def test_noalloc_refuses_sizes_beyond_its_scratch():
    lib = _ext.lib()
    fake = 1 << 20  # never dereferenced: the size check comes first
    B, H, H_kv, D, T_max = 4096, 16, 4, 128, 8192
    need = lib.mcamd_attn_workspace_bytes(B, 1, H, H_kv, D, T_max, -1)
    assert need > _ext.NOALLOC_SCRATCH_BYTES
    st = lib.mcamd_flash_attn_with_kvcache_noalloc(fake, fake, fake, fake, fake, fake, fake, B, 1,
                                                   H, H_kv, D, T_max, T_max * H_kv * D, -1, 1,
                                                   _ext.BF16, None)
    assert st == _ext.EWORKSPACE and b"static array" in lib.mcamd_last_error()


def test_noalloc_call_captured_in_a_hip_graph_replays_the_eager_result():
    """The entry point's purpose: a call recorded under graph capture (it allocates nothing, and
    records no memset) and replayed, with other calls on the same static scratch between the
    replays, gives the eager result bit for bit every time."""
    print("case: noalloc under graph capture", flush=True)
    lib = _ext.lib()
    seqlens = [int(x) for x in np.random.default_rng(12).integers(300, 3000, 24)]
    c = make_case(seqlens, 1, 16, 4, 128, 3072, torch.bfloat16, seed=95)
    g = {k: v.to(DEV) for k, v in c.items()}
    out = torch.empty(24, 1, 16, 128, dtype=torch.bfloat16, device=DEV)

    def call():
        return lib.mcamd_flash_attn_with_kvcache_noalloc(
            g["q"].data_ptr(), g["k"].data_ptr(), g["v"].data_ptr(), g["k_cache"].data_ptr(),
            g["v_cache"].data_ptr(), g["cache_seqlens"].data_ptr(), out.data_ptr(), 24, 1, 16, 4,
            128, 3072, g["k_cache"].stride(0), -1, 1, _ext.BF16, _ext.stream_handle(DEV))

    _ext.check(call(), "noalloc eager")
    torch.cuda.synchronize()
    eager = out.clone()
    k_after = g["k_cache"].clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st = call()
    _ext.check(st, "noalloc captured")
    other = make_case([900, 50, 2000], 1, 32, 8, 128, 2048, torch.bfloat16, seed=96)
    for i in range(3):
        out.fill_(float("nan"))
        _run("noalloc", other, 64, torch.bfloat16)  # another shape on the same scratch
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
    assert torch.equal(g["k_cache"], k_after)  # the replayed append rewrites the same token
    assert max_abs(to_np(eager), ko.flash_attn_with_kvcache(
        to_np(c["q"]), to_np(c["k_cache"]), to_np(c["v_cache"]), to_np(c["k"]), to_np(c["v"]),
        seqlens, -1)[0]) <= ATOL[torch.bfloat16]
