"""The byte/FLOP model every roofline divides by, and the runtime's dtype and peak denominators.

The counts in modelcore_amd.stats are pinned three ways: by brute force against the oracle's
key-visibility mask (itself pinned by float64 brute force in test_oracle.py), by closed forms,
and against the reference's own per-layer formulas (modelcore/stats.py:33-35, :55-73, :98-107),
restated in stats.ref_*; where the two conventions differ (a windowed query's own key), the
difference is asserted exactly.
"""
import numpy as np
import pytest
import torch

from modelcore_amd import runtime, stats
from oracle import kv_oracle as ko


def _brute_keys(L, t_new, window):
    """Distinct key columns any of the row's t_new queries may see, from the oracle's mask."""
    keep = ko.visible([L], t_new, L + t_new, window)[0]
    return int(keep.any(axis=0).sum())


def _brute_pairs(seqlens, t_new, window):
    return int(ko.visible(seqlens, t_new, max(seqlens) + t_new, window).sum())


@pytest.mark.parametrize("window", [-1, 0, 1, 7, 64, 1000])
def test_keys_seen_counts_the_oracle_mask(window):
    rng = np.random.default_rng(3)
    for _ in range(40):
        L, t = int(rng.integers(0, 300)), int(rng.integers(1, 40))
        assert stats.keys_seen(L, t, window) == _brute_keys(L, t, window), (L, t, window)


@pytest.mark.parametrize("window", [-1, 0, 5, 33])
def test_prefill_pairs_count_the_oracle_mask(window):
    rng = np.random.default_rng(4)
    for _ in range(20):
        seqlens = [int(x) for x in rng.integers(0, 200, int(rng.integers(1, 5)))]
        t = int(rng.integers(1, 70))
        assert stats.prefill_pairs(seqlens, t, window) == _brute_pairs(seqlens, t, window)


def test_a_planted_off_by_one_in_the_window_fails_the_brute_force_check():
    def wrong(L, t, w):  # counts min(L, w) keys back without the query's own key
        return stats.keys_seen(L, t, w) - (1 if w >= 0 and L >= w else 0)
    assert any(wrong(L, 1, 8) != _brute_keys(L, 1, 8) for L in range(0, 40))


def test_decode_bytes_closed_form_full_attention():
    """sum_b (L_b + 1) * 2 * H_kv * D * s for the keys, 2 * B * H * D * s for q and the output,
    2 * B * H_kv * D * s for the append's write: the new token's K/V are counted once."""
    g = torch.Generator().manual_seed(0)
    seqlens = torch.randint(512, 8192 + 1, (32,), generator=g, dtype=torch.int32).tolist()
    B, H, H_kv, D, s = 32, 16, 4, 128, 2
    want = sum(L + 1 for L in seqlens) * 2 * H_kv * D * s + 2 * B * H * D * s + 2 * B * H_kv * D * s
    assert stats.decode_step_bytes(seqlens, H, H_kv, D, s) == want
    assert stats.decode_step_bytes(seqlens, H, H_kv, D, s, append=False) == \
        want - 2 * B * H_kv * D * s


def test_decode_bytes_and_flops_against_the_reference_formulas():
    """Full attention: the reference's per-row read at context L + 1 (the new token included)
    and its decode FLOPs are exactly this build's. Under a window w, the reference counts
    min(w, L + 1) keys and this build min(L, w) + 1: one more key once L >= w."""
    H, H_kv, D, s = 12, 4, 128, 2
    for L in (0, 1, 5, 1023, 1024, 1025, 4096):
        for w in (-1, 0, 1, 1024):
            ours = stats.decode_kv_bytes([L], H_kv, D, s, w)
            ref = stats.ref_kv_read_bytes([w], H_kv, D, s, L + 1)
            extra = 1 if 0 <= w <= L else 0
            assert ours == ref + extra * 2 * H_kv * D * s, (L, w)
            assert stats.decode_flops([L], H, D, w) == \
                stats.ref_decode_attn_flops([w], H, D, L + 1) + extra * 4 * H * D
    # A stack: the per-layer sum of the reference equals the sum of per-layer calls here.
    windows = [-1 if i % 4 == 3 else 1024 for i in range(24)]
    L = 4096
    ours = sum(stats.decode_kv_bytes([L], H_kv, D, s, w) for w in windows)
    assert ours == stats.ref_kv_read_bytes(windows, H_kv, D, s, L + 1) + 18 * 2 * H_kv * D * s


@pytest.mark.parametrize("T", [1, 2, 17, 512, 16384])
def test_prefill_flops_closed_form_and_reference(T):
    """A causal prompt from position 0: 4 H D T (T + 1) / 2 FLOPs, the reference's formula with
    window = T. Windowed, the reference's flat part counts w keys per query, this build w + 1."""
    H, D = 32, 128
    assert stats.prefill_flops([0], T, H, D) == 4 * H * D * T * (T + 1) // 2
    assert stats.prefill_flops([0], T, H, D) == stats.ref_prefill_attn_flops([-1], H, D, T)
    w = 100
    extra = max(0, T - w)
    assert stats.prefill_flops([0], T, H, D, w) == \
        stats.ref_prefill_attn_flops([w], H, D, T) + 4 * H * D * extra


def test_chunked_prefill_flops_sum_to_the_whole_prompt():
    """32 chunks of 512 at offsets 0, 512, ... attend exactly the pairs of one 16384-token
    prompt: 1.759e13 FLOPs at 8 rows, 32 heads, head_dim 128."""
    B, T, C, H, D = 8, 16384, 512, 32, 128
    chunks = sum(stats.prefill_flops([c * C] * B, C, H, D) for c in range(T // C))
    assert chunks == B * stats.prefill_flops([0], T, H, D) == B * 4 * H * D * T * (T + 1) // 2
    assert abs(chunks - 1.759e13) / 1.759e13 < 1e-3


def test_append_and_replication_bytes_closed_forms():
    assert stats.append_bytes(8, 512, 8, 128, 2) == 2 * 2 * 8 * 512 * 8 * 128 * 2
    S, R, P, H_kv, D = 32, 64, 2048, 8, 128
    per_copy = S * P * H_kv * D * 2 * 2
    assert stats.replicate_bytes(S, R, P, H_kv, D, 2) == per_copy * (R + 1)


# --- runtime ------------------------------------------------------------------------------------

def test_peaks_follow_the_reference_tables():
    assert runtime.peak_bandwidth("AMD Instinct MI355X") == 8.0e12
    assert runtime.peak_flops("AMD Instinct MI355X") == 2.5e15
    assert runtime.peak_bandwidth("AMD Instinct MI300X") == 5.3e12
    assert runtime.peak_flops("AMD Instinct MI300X") == 1.3074e15
    assert runtime.peak_flops("AMD Instinct MI300A") == 980.6e12
    assert runtime.peak_bandwidth("AMD Instinct MI250X") == 3.28e12
    logged = []
    assert runtime.peak_bandwidth("Some GPU", log=logged.append) == float("inf")
    assert runtime.peak_flops("Some GPU") == float("inf")
    assert logged and "Some GPU" in logged[0]


def test_compute_dtype_override_and_fallbacks(monkeypatch):
    monkeypatch.setenv("MODELCORE_DTYPE", "bfloat16")
    assert runtime.detect_compute_dtype() == (torch.bfloat16, "set via MODELCORE_DTYPE=bfloat16")
    assert runtime.Runtime().compute_dtype == torch.bfloat16
    monkeypatch.setenv("MODELCORE_DTYPE", "float32")
    assert runtime.detect_compute_dtype()[0] == torch.float32
    monkeypatch.setenv("MODELCORE_DTYPE", "float16")  # absent on purpose, as in the reference
    with pytest.raises(KeyError):
        runtime.detect_compute_dtype()
    monkeypatch.delenv("MODELCORE_DTYPE")
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    assert runtime.detect_compute_dtype() == (torch.float32, "auto-detected: no GPU (fp32)")
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "get_device_capability", lambda *a: (9, 5))
    assert runtime.detect_compute_dtype()[0] == torch.bfloat16
    monkeypatch.setattr(torch.cuda, "get_device_capability", lambda *a: (7, 5))
    assert runtime.detect_compute_dtype()[0] == torch.float32
    rt = runtime.Runtime(torch.float32)
    assert rt.compute_dtype == torch.float32 and rt.compute_dtype_reason == "explicit"


def test_device_peaks_by_name_or_by_architecture(monkeypatch):
    class Props:
        gcnArchName = "gfx950:sramecc+:xnack-"

    monkeypatch.setattr(torch.cuda, "get_device_properties", lambda i: Props())
    monkeypatch.setattr(torch.cuda, "get_device_name", lambda i: "AMD Instinct MI355X")
    bw, fl, how = runtime.device_peaks(0)
    assert (bw, fl) == (8.0e12, 2.5e15) and "name" in how
    monkeypatch.setattr(torch.cuda, "get_device_name", lambda i: "AMD Radeon Graphics")
    bw, fl, how = runtime.device_peaks(0)
    assert (bw, fl) == (8.0e12, 2.5e15) and "gfx950" in how
    Props.gcnArchName = "gfx1100"
    assert runtime.device_peaks(0)[0] == float("inf")
