"""Parity of the HIP kernels with the CPU oracle, through the C ABI and the drop-in operator.

Append and replication must be bit-exact; attention must be within the tolerance of its dtype
(max-abs 2e-2 for bf16 inputs with fp32 accumulation, 2e-5 for fp32) of the float64 oracle.
Inputs are drawn on the CPU from a seeded generator and copied to the GPU, so both sides see
identical bytes.
"""
import os

import numpy as np
import pytest
import torch

from _util import ATOL, bits, gen, make_case, max_abs, to_np
from modelcore_amd import _ext
from modelcore_amd.cache import KVCache
from modelcore_amd.kernels.flash_attn import flash_attn
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _gpu(c):
    return {k: v.to(DEV) for k, v in c.items()}


def _note(*a):
    print("case:", *a, flush=True)


def test_the_hip_library_loads_on_the_gpu_box_with_one_hip_runtime():
    assert torch.cuda.is_available(), "no ROCm GPU visible"
    _ext.lib()
    torch.zeros(1, device=DEV)
    with open("/proc/self/maps") as f:
        hip = {line.split()[-1] for line in f if "libamdhip64" in line}
    assert len(hip) == 1, f"more than one HIP runtime mapped: {hip}"
    with open("/proc/self/maps") as f:
        assert any(str(_ext.LIB_PATH) in line for line in f)


# --- append -------------------------------------------------------------------------------------

APPEND_CASES = [
    # seqlens, T_new, H_kv, D, T_max
    ([0, 5, 11, 3], 1, 4, 128, 16),
    ([7, 7], 5, 8, 128, 32),
    ([0, 100, 37], 64, 2, 64, 200),
    ([2, 9], 3, 2, 16, 16),
    ([1, 0, 4], 2, 1, 16, 8),  # 32-byte rows of bf16: the 16-byte path; fp32 too
    # Chunk-sized copies: whole 1024-unit blocks plus a tail, token runs of 48 units (a division,
    # not a shift) and of 32 units (a shift), blocks that straddle tokens.
    ([0, 300, 1000], 512, 3, 128, 1600),
    ([5, 1], 700, 2, 128, 800),
    ([3, 0], 37, 1, 6, 64),  # 12-byte runs of bf16: the 4-byte path (24-byte fp32 runs too)
    ([2, 9], 33, 1, 5, 64),  # 10-byte runs of bf16: the 2-byte path (20-byte fp32: 4-byte)
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("seqlens,T_new,H_kv,D,T_max", APPEND_CASES)
def test_append_is_bit_exact(dtype, seqlens, T_new, H_kv, D, T_max):
    _note("append", dtype, seqlens, T_new, H_kv, D, T_max)
    c = make_case(seqlens, T_new, H_kv, H_kv, D, T_max, dtype, seed=11)
    g = _gpu(c)
    lib = _ext.lib()
    st = lib.mcamd_kv_append(g["k"].data_ptr(), g["v"].data_ptr(), g["k_cache"].data_ptr(),
                             g["v_cache"].data_ptr(), g["cache_seqlens"].data_ptr(), len(seqlens),
                             T_new, H_kv, D, T_max, g["k_cache"].stride(0), _ext.dtype_code(dtype),
                             _ext.stream_handle(DEV))
    _ext.check(st, "append")
    ek, ev = ko.append(bits(c["k_cache"]), bits(c["v_cache"]), bits(c["k"]), bits(c["v"]), seqlens)
    assert np.array_equal(bits(g["k_cache"]), ek)
    assert np.array_equal(bits(g["v_cache"]), ev)


def test_append_leaves_rows_past_the_cache_untouched():
    c = make_case([3, 15], 2, 2, 2, 64, 16, torch.bfloat16, seed=12)
    g = _gpu(c)
    lib = _ext.lib()
    _ext.check(lib.mcamd_kv_append(g["k"].data_ptr(), g["v"].data_ptr(), g["k_cache"].data_ptr(),
                                   g["v_cache"].data_ptr(), g["cache_seqlens"].data_ptr(), 2, 2, 2,
                                   64, 16, g["k_cache"].stride(0), _ext.BF16,
                                   _ext.stream_handle(DEV)), "append")
    got = bits(g["k_cache"])
    assert np.array_equal(got[1, :15], bits(c["k_cache"])[1, :15])
    assert np.array_equal(got[1, 15], bits(c["k"])[1, 0])  # position 15 fits, 16 does not
    assert np.array_equal(got[0, 3:5], bits(c["k"])[0])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_append_of_a_long_chunk_drops_only_the_positions_past_the_cache(dtype):
    # Row 1's chunk runs 112 positions past the cache: blocks wholly inside, straddling and wholly
    # past the end all occur; the rows that fit are copied, nothing else changes.
    seqlens, T_new, H_kv, D, T_max = [100, 600, 0], 512, 4, 128, 1000
    _note("append overflow", dtype, seqlens, T_new, H_kv, D, T_max)
    c = make_case(seqlens, T_new, H_kv, H_kv, D, T_max, dtype, seed=14)
    g = _gpu(c)
    lib = _ext.lib()
    _ext.check(lib.mcamd_kv_append(g["k"].data_ptr(), g["v"].data_ptr(), g["k_cache"].data_ptr(),
                                   g["v_cache"].data_ptr(), g["cache_seqlens"].data_ptr(),
                                   len(seqlens), T_new, H_kv, D, T_max, g["k_cache"].stride(0),
                                   _ext.dtype_code(dtype), _ext.stream_handle(DEV)), "append")
    for b, p in enumerate(seqlens):
        fit = min(T_new, T_max - p)
        ek, ev = ko.append(bits(c["k_cache"])[b:b + 1], bits(c["v_cache"])[b:b + 1],
                           bits(c["k"])[b:b + 1, :fit], bits(c["v"])[b:b + 1, :fit], [p])
        assert np.array_equal(bits(g["k_cache"])[b:b + 1], ek), f"row {b}"
        assert np.array_equal(bits(g["v_cache"])[b:b + 1], ev), f"row {b}"


# --- replication --------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("slots,rows,P,H_kv,D", [(2, 4, 7, 2, 8), (3, 64, 129, 8, 128),
                                                 (1, 5, 33, 1, 16),
                                                 # whole 4096-unit blocks plus a tail: 16-byte
                                                 # units, then 4-byte units (20-byte bf16 rows)
                                                 (2, 3, 1000, 3, 20), (2, 5, 1001, 1, 10)])
def test_prefill_replicates_bit_exactly(dtype, slots, rows, P, H_kv, D):
    _note("replicate", dtype, slots, rows, P, H_kv, D)
    g = gen(13)
    src = KVCache(1, H_kv, P, D, slots, DEV, dtype)
    src.k_cache.copy_(torch.randn(src.k_cache.shape, generator=g).to(dtype))
    src.v_cache.copy_(torch.randn(src.v_cache.shape, generator=g).to(dtype))
    src.advance(P)
    dst = KVCache(rows, H_kv, P + 5, D, slots, DEV, dtype)
    dst.prefill(src)
    assert dst.get_pos() == P and dst.cache_seqlens.tolist() == [P] * rows
    ek, ev = ko.replicate(bits(dst.k_cache) * 0, bits(dst.v_cache) * 0, bits(src.k_cache),
                          bits(src.v_cache), P, range(rows))
    assert np.array_equal(bits(dst.k_cache), ek) and np.array_equal(bits(dst.v_cache), ev)


def test_prefill_row_copies_only_its_row_and_tracks_raggedness():
    g = gen(14)

    def filled(n):
        c = KVCache(1, 2, n, 8, 2, DEV, torch.float32)
        c.k_cache.copy_(torch.randn(c.k_cache.shape, generator=g))
        c.v_cache.copy_(torch.randn(c.v_cache.shape, generator=g))
        c.advance(n)
        return c

    a, b = filled(5), filled(11)
    dst = KVCache(3, 2, 24, 8, 2, DEV, torch.float32)
    dst.prefill_row(1, a)
    assert dst.cache_seqlens.tolist() == [0, 5, 0]
    assert torch.equal(dst.k_cache[:, 1, :5], a.k_cache[:, 0, :5])
    assert dst.k_cache[:, 0].abs().sum() == 0 and dst.k_cache[:, 2].abs().sum() == 0
    dst.prefill_row(2, b)
    assert dst.cache_seqlens.tolist() == [0, 5, 11] and dst.uniform_pos() is None
    assert torch.equal(dst.v_cache[:, 2, :11], b.v_cache[:, 0, :11])
    assert not dst.v_cache[:, 2, 11:].any()


# --- attention ----------------------------------------------------------------------------------

def _run_op(c, window, with_append=True):
    g = _gpu(c)
    out = flash_attn.flash_attn_with_kvcache(
        g["q"], g["k_cache"], g["v_cache"], k=g["k"] if with_append else None,
        v=g["v"] if with_append else None, cache_seqlens=g["cache_seqlens"], causal=True,
        window_size=(window, 0))
    torch.cuda.synchronize()
    return out, g


def _oracle(c, window, with_append=True):
    q, kc, vc = to_np(c["q"]), to_np(c["k_cache"]), to_np(c["v_cache"])
    k = to_np(c["k"]) if with_append else None
    v = to_np(c["v"]) if with_append else None
    return ko.flash_attn_with_kvcache(q, kc, vc, k, v, c["cache_seqlens"].tolist(), window)[0]


# 80 ragged rows: past 64 rows the fused kernel's work split scans cache_seqlens in chunks of 64.
RAGGED_80 = [int(x) for x in np.random.default_rng(5).integers(0, 650, 80)]

DECODE_CASES = [
    # seqlens, H, H_kv, D, T_max, window
    ([37, 300, 0, 511], 16, 4, 128, 520, -1),
    ([37, 300, 0, 511], 16, 4, 128, 520, 64),
    ([1000, 1023, 5], 12, 4, 128, 1030, 100),
    ([77, 250], 32, 8, 128, 300, -1),
    ([255, 256, 257, 513], 8, 8, 64, 520, -1),
    ([9, 30], 2, 2, 16, 40, 8),
    ([60, 3], 16, 2, 64, 64, -1),   # G = 8
    ([60, 3], 16, 1, 64, 64, 0),    # G = 16: two head chunks; window 0
    ([300, 5, 777], 16, 2, 128, 800, -1),   # G = 8 at head_dim 128: two 4-head groups
    ([1030, 2], 16, 1, 128, 1040, 200),     # G = 16 at head_dim 128, windowed
    ([4095, 17], 4, 4, 128, 4100, 1024),    # MHA, 4 windowed splits
    ([0, 3], 16, 4, 128, 2000, -1),         # far fewer keys than waves
    ([1999, 0, 1], 16, 4, 128, 2000, 5),    # tiny windows in a long cache
    (RAGGED_80, 16, 4, 128, 700, -1),       # more rows than one wave scans
    (RAGGED_80, 16, 4, 128, 700, 100),
    # head dims that are not powers of two: run by the next power's kernel, lanes past D idle
    ([37, 300, 0, 511], 16, 4, 80, 520, -1),
    ([100, 7], 12, 4, 96, 128, 33),
    ([300, 5, 77], 8, 2, 192, 320, -1),
    ([60, 3], 4, 4, 48, 64, -1),
    # head dims above 256 (up to 512): the general prefill kernel with one query per row
    ([37, 300, 0, 5], 8, 2, 512, 320, -1),
    ([100, 7], 6, 2, 384, 128, 33),
    ([31], 4, 1, 320, 40, -1),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("seqlens,H,H_kv,D,T_max,window", DECODE_CASES)
def test_decode_matches_the_oracle(dtype, seqlens, H, H_kv, D, T_max, window):
    _note("decode", dtype, seqlens, H, H_kv, D, T_max, window)
    c = make_case(seqlens, 1, H, H_kv, D, T_max, dtype, seed=21)
    out, g = _run_op(c, window)
    ref = _oracle(c, window)
    err = max_abs(to_np(out), ref)
    assert err <= ATOL[dtype], f"max-abs {err}"
    ek, _ = ko.append(bits(c["k_cache"]), bits(c["v_cache"]), bits(c["k"]), bits(c["v"]), seqlens)
    assert np.array_equal(bits(g["k_cache"]), ek)


def test_repeated_decode_calls_are_deterministic():
    """The workspace is scratch shared by every call on the device: repeated calls, also after a
    call of another shape that left its own partials in it, give identical bits."""
    c = make_case([700, 31, 2000, 256], 1, 16, 4, 128, 2100, torch.bfloat16, seed=23)
    first, _ = _run_op(c, -1)
    other = make_case([90, 1500], 1, 32, 8, 128, 1600, torch.bfloat16, seed=24)
    _run_op(other, 64)
    for _ in range(3):
        again, _ = _run_op(c, -1)
        assert torch.equal(first, again)
    assert max_abs(to_np(first), _oracle(c, -1)) <= ATOL[torch.bfloat16]


def test_decode_replayed_from_a_hip_graph_matches_eager():
    """A captured decode step (append + attention) replayed several times, with eager work and
    synchronisations between the replays, matches the eager result of the same step each time."""
    c = make_case([513, 64, 1999], 1, 16, 4, 128, 2048, torch.bfloat16, seed=25)
    g = _gpu(c)
    kc0, vc0 = g["k_cache"].clone(), g["v_cache"].clone()

    def step():
        return flash_attn.flash_attn_with_kvcache(g["q"], g["k_cache"], g["v_cache"], k=g["k"],
                                                  v=g["v"], cache_seqlens=g["cache_seqlens"],
                                                  causal=True, window_size=(-1, 0))

    eager = step().clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    for i in range(4):
        g["k_cache"].copy_(kc0)
        g["v_cache"].copy_(vc0)
        _run_op(make_case([40], 1, 8, 2, 128, 64, torch.bfloat16, seed=26 + i), -1)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        assert torch.equal(g["k_cache"][0, 513].cpu(), c["k"][0, 0])


@pytest.mark.parametrize("D", [128, 64])
def test_rows_past_the_cache_get_nan_and_leave_the_cache_alone(D):
    """A row whose position is outside the cache cannot be attended (the reference raises an
    index error there): its output is NaN, its cache row is untouched, other rows are exact."""
    seqlens = [64, 10, 63]
    c = make_case(seqlens, 1, 8, 2, D, 64, torch.bfloat16, seed=27)
    out, g = _run_op(c, -1)
    assert torch.isnan(out[0].float()).all()
    assert torch.equal(g["k_cache"][0].cpu(), c["k_cache"][0])
    ok = {k: v[1:] for k, v in c.items()}
    assert max_abs(to_np(out[1:]), _oracle(ok, -1)) <= ATOL[torch.bfloat16]


def test_decode_without_append_reads_the_cache():
    seqlens = [40, 7]
    c = make_case(seqlens, 1, 8, 2, 128, 64, torch.bfloat16, seed=22)
    out, g = _run_op(c, -1, with_append=False)
    assert max_abs(to_np(out), _oracle(c, -1, with_append=False)) <= ATOL[torch.bfloat16]
    assert torch.equal(g["k_cache"].cpu(), c["k_cache"])


PREFILL_CASES = [
    # seqlens, T_new, H, H_kv, D, T_max, window
    ([0, 0], 40, 8, 2, 128, 64, -1),
    ([0, 0], 40, 8, 2, 128, 64, 9),
    ([17, 3], 25, 16, 4, 128, 64, -1),
    ([100, 0, 31], 70, 12, 4, 64, 200, 50),
    ([5, 9], 3, 2, 2, 16, 16, -1),
    ([0], 12, 2, 2, 16, 12, 8),
    ([33, 2], 130, 32, 8, 128, 200, 0),
    # bf16 / head_dim 128 shapes of the matrix-core kernel: tiles of 64 keys, 256 (position,
    # head) pairs per workgroup, masks at the diagonal and at window edges inside a tile
    ([0, 64, 129], 200, 32, 8, 128, 400, -1),     # G = 4, prefixes on and off tile boundaries
    ([300, 17], 77, 12, 4, 128, 400, 100),        # G = 3 (85 positions per workgroup)
    ([250], 300, 8, 8, 128, 600, 63),             # MHA, window inside a tile
    ([5, 400], 40, 16, 2, 128, 448, 64),          # G = 8
    ([1000], 64, 16, 1, 128, 1100, -1),           # G = 16: 16 positions per workgroup
    ([8000, 6913], 64, 32, 2, 128, 8100, -1),     # G = 16 over long prefixes (126 key tiles)
    ([7000, 100], 96, 24, 2, 128, 7200, 1500),    # G = 12, a window of 1500 in a long cache
    ([7, 0], 1, 32, 8, 128, 16, -1),              # a single query through the prefill path
    ([17, 3], 25, 16, 4, 80, 64, -1),             # head dims that are not powers of two
    ([100, 0, 31], 70, 12, 4, 96, 200, 50),
    ([5, 40], 33, 8, 2, 192, 80, -1),
    ([17, 3], 25, 8, 2, 384, 64, -1),             # head dims above 256, up to 512
    ([100, 0], 20, 4, 4, 512, 140, 50),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("seqlens,T_new,H,H_kv,D,T_max,window", PREFILL_CASES)
def test_chunked_prefill_matches_the_oracle(dtype, seqlens, T_new, H, H_kv, D, T_max, window):
    _note("prefill", dtype, seqlens, T_new, H, H_kv, D, T_max, window)
    c = make_case(seqlens, T_new, H, H_kv, D, T_max, dtype, seed=31)
    out, g = _run_op(c, window)
    err = max_abs(to_np(out), _oracle(c, window))
    assert err <= ATOL[dtype], f"max-abs {err}"
    ek, ev = ko.append(bits(c["k_cache"]), bits(c["v_cache"]), bits(c["k"]), bits(c["v"]), seqlens)
    assert np.array_equal(bits(g["k_cache"]), ek) and np.array_equal(bits(g["v_cache"]), ev)


def test_chunked_prefill_of_a_long_prompt_at_gqa_32_8():
    """One 512-token chunk at position 1536 (a 2048-key prefix), 32 q / 8 kv heads, bf16: the
    chunk shape of the 16384-token chunked-prefill workload, against the float64 oracle."""
    c = make_case([1536], 512, 32, 8, 128, 2048, torch.bfloat16, seed=33)
    out, g = _run_op(c, -1)
    err = max_abs(to_np(out), _oracle(c, -1))
    print(f"max-abs against the float64 oracle {err:.2e}", flush=True)
    assert err <= ATOL[torch.bfloat16], f"max-abs {err}"
    # Accuracy guard, far inside the tolerance (deterministic output): 1.7e-3 measured with the
    # query scale rounded into the bf16 fragments, 1.3e-3 with it applied in fp32.
    assert err <= 5e-3, f"max-abs {err}: accuracy below what this path delivers"


def test_chunked_prefill_through_the_cache_equals_one_full_prefill():
    """Feeding a prompt in chunks (append at an offset, attend to the prefix) gives the outputs of
    one full-prompt call, position by position (modelcore/tests/test_recurrent.py:150-156)."""
    g = gen(34)
    B, T, H, H_kv, D, C = 2, 384, 16, 4, 128, 128
    q = torch.randn(B, T, H, D, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(B, T, H_kv, D, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(B, T, H_kv, D, generator=g).to(torch.bfloat16).to(DEV)
    for window in (-1, 100):
        full_k = torch.zeros(B, T, H_kv, D, dtype=torch.bfloat16, device=DEV)
        full_v = torch.zeros_like(full_k)
        zero = torch.zeros(B, dtype=torch.int32, device=DEV)
        whole = flash_attn.flash_attn_with_kvcache(q, full_k, full_v, k=k, v=v, cache_seqlens=zero,
                                                   causal=True, window_size=(window, 0))
        cache = KVCache(B, H_kv, T, D, 1, DEV, torch.bfloat16)
        kc, vc = cache.get_slot_cache(0)
        parts = []
        for a in range(0, T, C):
            parts.append(flash_attn.flash_attn_with_kvcache(
                q[:, a:a + C], kc, vc, k=k[:, a:a + C], v=v[:, a:a + C],
                cache_seqlens=cache.cache_seqlens, causal=True, window_size=(window, 0)))
            cache.advance(C)
        assert torch.equal(kc, full_k) and torch.equal(vc, full_v)
        assert torch.equal(torch.cat(parts, dim=1), whole), f"window {window}"


def test_no_cache_attention_equals_prefill_from_empty():
    c = make_case([0, 0], 48, 8, 2, 128, 48, torch.bfloat16, seed=32)
    g = _gpu(c)
    y = flash_attn.flash_attn_func(g["q"], g["k_cache"], g["v_cache"], causal=True,
                                   window_size=(16, 0))
    ref = ko.attention(to_np(c["q"]), to_np(c["k_cache"]), to_np(c["v_cache"]), [0, 0], 16)
    assert max_abs(to_np(y), ref) <= ATOL[torch.bfloat16]


# --- the decode microbenchmark's own shape, at full size -----------------------------------------

def test_decode_at_batch_32_gqa_16_4_hd128_context_8k():
    """B=32, H=16, H_kv=4, D=128, cache 8192+8, lengths U[512, 8192] (seed 0): one step."""
    g = gen(0)
    B, H, H_kv, D, T_max = 32, 16, 4, 128, 8192 + 8
    seqlens = torch.randint(512, 8192 + 1, (B,), generator=g, dtype=torch.int32)
    kc = torch.randn(B, T_max, H_kv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(B, T_max, H_kv, D, generator=g).to(torch.bfloat16)
    q = torch.randn(B, 1, H, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, 1, H_kv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, 1, H_kv, D, generator=g).to(torch.bfloat16)
    c = dict(q=q, k=k, v=v, k_cache=kc, v_cache=vc, cache_seqlens=seqlens)
    out, gg = _run_op(c, -1)
    out = to_np(out)
    kcn, vcn = to_np(kc), to_np(vc)
    worst = 0.0
    for b in range(B):
        L = int(seqlens[b])
        kb, vb = kcn[b:b + 1, :L + 1].copy(), vcn[b:b + 1, :L + 1].copy()
        kb[0, L], vb[0, L] = to_np(k)[b, 0], to_np(v)[b, 0]
        ref = ko.attention(to_np(q)[b:b + 1], kb, vb, [L], -1)
        worst = max(worst, max_abs(out[b:b + 1], ref))
    print(f"max-abs against the float64 oracle {worst:.2e}", flush=True)
    assert worst <= ATOL[torch.bfloat16], f"max-abs {worst}"
    # Accuracy guard, far inside the tolerance: the outputs are deterministic, and with the split
    # partials' o rounded to bf16 once this shape measures 9.8e-4 (6.4e-4 with fp32 partials).
    assert worst <= 2e-3, f"max-abs {worst}: accuracy below what this path delivers"
    got = gg["k_cache"]
    for b in range(B):
        assert torch.equal(got[b, int(seqlens[b])].cpu(), k[b, 0])


# --- the reference's operator invariants (modelcore/tests/test_kernels.py:420-545) on the GPU ---

class TestRaggedOperator:
    H, D, T_MAX = 4, 16, 48

    def _make(self, seqlens, T_new=1, seed=0):
        return make_case(seqlens, T_new, self.H, self.H, self.D, self.T_MAX, torch.bfloat16, seed,
                         fill_stale=False)

    @pytest.mark.parametrize("window", [-1, 8])
    @pytest.mark.parametrize("T_new", [1, 3])
    def test_batched_ragged_matches_each_row_alone(self, window, T_new):
        seqlens = [4, 17, 31, 9]
        c = self._make(seqlens, T_new)
        out, _ = _run_op(c, window)
        for b in range(len(seqlens)):
            row = {k: v[b:b + 1] for k, v in c.items()}
            o, _ = _run_op(row, window)
            assert torch.equal(out[b:b + 1], o)

    def test_stale_kv_beyond_a_rows_content_is_unreachable(self):
        seqlens = [4, 17, 31, 9]
        c = self._make(seqlens)
        clean, _ = _run_op(c, -1)
        dirty = dict(c)
        dirty["k_cache"], dirty["v_cache"] = c["k_cache"].clone(), c["v_cache"].clone()
        for b, L in enumerate(seqlens):
            dirty["k_cache"][b, L + 1:] = 1e4
            dirty["v_cache"][b, L + 1:] = float("nan")
        assert torch.equal(clean, _run_op(dirty, -1)[0])

    def test_new_tokens_land_at_each_rows_own_offset(self):
        seqlens = [4, 17, 31, 9]
        c = self._make(seqlens)
        _, g = _run_op(c, -1)
        kc = g["k_cache"].cpu()
        for b, L in enumerate(seqlens):
            assert torch.equal(kc[b, L], c["k"][b, 0])
            keep = torch.ones(self.T_MAX, dtype=torch.bool)
            keep[L] = False
            assert torch.equal(kc[b][keep], c["k_cache"][b][keep])

    def test_sliding_window_is_measured_from_each_rows_own_position(self):
        window = 8
        c = self._make([3, 20])
        base, _ = _run_op(c, window)
        far = dict(c, k_cache=c["k_cache"].clone())
        far["k_cache"][1, :10] += 5.0
        assert torch.equal(base[1], _run_op(far, window)[0][1])
        near = dict(c, k_cache=c["k_cache"].clone())
        near["k_cache"][0, 0] += 5.0
        assert not torch.equal(base[0], _run_op(near, window)[0][0])

    def test_uniform_positions_agree_with_the_oracle_and_the_ragged_rows(self):
        for window in (-1, 8):
            c = self._make([13, 13])
            out, _ = _run_op(c, window)
            assert max_abs(to_np(out), _oracle(c, window)) <= ATOL[torch.bfloat16]
            alone, _ = _run_op({k: v[1:] for k, v in c.items()}, window)
            assert torch.equal(out[1:], alone)


def test_prefill_then_decode_through_the_cache_object():
    """TestSDPAOnly.test_kvcache (modelcore/tests/test_kernels.py:372-414), checked against the
    oracle at each call: a 16-token prefill then single tokens, positions advancing."""
    B, T_max, H, D = 2, 64, 4, 32
    cache = KVCache(batch_size=B, n_kv_head=H, seq_len=T_max, head_dim=D, num_kv_slots=1,
                    device=DEV, dtype=torch.bfloat16)
    kc, vc = cache.get_slot_cache(0)
    g = gen(40)
    ref_k, ref_v = np.zeros((B, T_max, H, D)), np.zeros((B, T_max, H, D))
    for T_new in (16, 1, 1, 1):
        q, k, v = (torch.randn(B, T_new, H, D, generator=g).to(torch.bfloat16) for _ in range(3))
        pos = cache.get_pos()
        y = flash_attn.flash_attn_with_kvcache(q.to(DEV), kc, vc, k=k.to(DEV), v=v.to(DEV),
                                               cache_seqlens=cache.cache_seqlens, causal=True,
                                               window_size=(T_max, 0))
        cache.advance(T_new)
        assert y.shape == (B, T_new, H, D) and cache.get_pos() == pos + T_new
        want, ref_k, ref_v = ko.flash_attn_with_kvcache(to_np(q), ref_k, ref_v, to_np(k), to_np(v),
                                                        [pos] * B, T_max)
        assert max_abs(to_np(y), want) <= ATOL[torch.bfloat16]
    assert np.array_equal(to_np(kc), ref_k)
