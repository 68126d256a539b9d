"""Host-side behaviour of the drop-in KVCache and operator module, on CPU tensors: position
bookkeeping and the assertion messages of modelcore/tests/test_cache.py, the reference's backend
switch, and the loud refusal of any non-ROCm tensor (there is no CPU path)."""
import pytest
import torch

import modelcore_amd.kernels.flash_attn as fa
from modelcore_amd.cache import KVCache

H, D, T_MAX, SLOTS = 2, 8, 24, 2


def _cache(batch_size, seq_len=T_MAX):
    return KVCache(batch_size=batch_size, n_kv_head=H, seq_len=seq_len, head_dim=D,
                   num_kv_slots=SLOTS, device="cpu", dtype=torch.float32)


def _filled(length):
    c = _cache(1, seq_len=length)
    c.advance(length)
    return c


def test_layout_and_initial_state_match_the_reference():
    c = _cache(3)
    assert c.k_cache.shape == (SLOTS, 3, T_MAX, H, D) and c.v_cache.shape == c.k_cache.shape
    assert c.cache_seqlens.dtype == torch.int32 and c.cache_seqlens.tolist() == [0, 0, 0]
    assert not c.k_cache.any() and c.state == {}
    k, v = c.get_slot_cache(1)
    assert k.shape == (3, T_MAX, H, D) and k.data_ptr() == c.k_cache[1].data_ptr()


def test_shared_prefix_starts_at_zero_and_reset_clears_it():
    c = _cache(3)
    assert c.shared_prefix == 0
    c.shared_prefix = 7
    c.advance(9)
    assert c.shared_prefix == 7
    c.reset()
    assert c.shared_prefix == 0


def test_uniform_cache_reports_its_single_position():
    c = _cache(3)
    assert c.get_pos() == c.uniform_pos() == 0
    c.advance(5)
    assert c.get_pos() == c.uniform_pos() == 5
    assert c.cache_seqlens.tolist() == [5, 5, 5]
    c.reset()
    assert c.get_pos() == 0 and c.cache_seqlens.tolist() == [0, 0, 0]


def test_get_pos_raises_on_a_ragged_cache():
    c = _cache(2)
    c._pos_uniform = None
    assert c.uniform_pos() is None
    with pytest.raises(AssertionError, match="ragged"):
        c.get_pos()


def test_advance_preserves_row_differences():
    c = _cache(3)
    c.cache_seqlens.copy_(torch.tensor([3, 8, 5], dtype=torch.int32))
    c._pos_uniform = None
    for _ in range(4):
        c.advance(1)
    assert c.cache_seqlens.tolist() == [7, 12, 9] and c.uniform_pos() is None


def test_prefill_row_refusals_keep_the_reference_messages():
    dst = _cache(2)
    dst.cache_seqlens[0] = 4
    with pytest.raises(AssertionError, match="non-empty"):
        dst.prefill_row(0, _filled(4))
    with pytest.raises(AssertionError, match="batch=1"):
        dst.prefill_row(1, _cache(2))
    with pytest.raises(AssertionError, match="exceeds cache length"):
        dst.prefill_row(1, _filled(T_MAX + 1))


def test_prefill_refuses_a_non_empty_cache():
    dst = _cache(2)
    dst.advance(1)
    with pytest.raises(AssertionError, match="non-empty"):
        dst.prefill(_filled(3))


def test_copies_on_cpu_tensors_fail_loudly():
    dst = _cache(2)
    with pytest.raises(RuntimeError, match="ROCm device"):
        dst.prefill(_filled(3))


def test_operator_refuses_cpu_tensors():
    q = torch.zeros(1, 1, 2, 8)
    kc = torch.zeros(1, 4, 2, 8)
    with pytest.raises(RuntimeError, match="ROCm device"):
        fa.flash_attn.flash_attn_with_kvcache(q, kc, kc.clone(),
                                              cache_seqlens=torch.zeros(1, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="ROCm device"):
        fa.flash_attn.flash_attn_func(q, q, q, causal=True)


def test_backend_switch_keeps_the_reference_behaviour():
    """set_impl('fa3') must refuse with the reference's message; 'sdpa' / None resolve to False."""
    try:
        fa._override_impl = "fa3"
        with pytest.raises(AssertionError, match="Cannot override to FA3"):
            fa._resolve_use_fa3()
        for impl in ("sdpa", None):
            fa._override_impl = impl
            assert fa._resolve_use_fa3() is False
    finally:
        fa._override_impl = None
    assert fa.USE_FA3 is False and fa.HAS_FA3 is False and isinstance(fa.FA3_LOAD_ERROR, str)
