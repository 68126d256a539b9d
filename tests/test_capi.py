"""The C-ABI library on the CPU host: it loads, exports exactly what include/modelcore_amd.h
declares, and rejects bad arguments before touching the GPU (no kernel runs here)."""
import ctypes
import re

import pytest

from conftest import ROOT
from modelcore_amd import _ext

HEADER = ROOT / "include" / "modelcore_amd.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(mcamd_\w+)\s*\(", text))


def test_header_and_loader_agree_on_the_exported_functions():
    assert declared_functions() == set(_ext.SIGNATURES)


def test_library_loads_and_exports_every_declared_symbol():
    lib = _ext.lib()
    raw = ctypes.CDLL(str(_ext.LIB_PATH))
    for name in declared_functions():
        assert hasattr(raw, name), name
    assert lib.mcamd_abi_version() == _ext.ABI_VERSION


def test_bad_dtype_and_null_pointers_are_rejected_with_a_message():
    lib = _ext.lib()
    st = lib.mcamd_kv_append(None, None, None, None, None, 1, 1, 1, 8, 4, 32, 7, None)
    assert st == _ext.EINVAL and b"dtype" in lib.mcamd_last_error()
    st = lib.mcamd_kv_append(None, None, None, None, None, 1, 1, 1, 8, 4, 32, _ext.BF16, None)
    assert st == _ext.EINVAL and b"null" in lib.mcamd_last_error()


def test_attention_rejects_bad_head_grouping_and_small_workspace():
    lib = _ext.lib()
    fake = 1 << 20  # never dereferenced: the checks fail first
    st = lib.mcamd_decode_attention(fake, fake, fake, fake, fake, 2, 6, 4, 128, 64, 64 * 4 * 128,
                                    -1, _ext.BF16, fake, 1 << 30, None)
    assert st == _ext.EINVAL and b"multiple" in lib.mcamd_last_error()
    st = lib.mcamd_decode_attention(fake, fake, fake, fake, fake, 2, 8, 4, 128, 64, 64 * 4 * 128,
                                    -1, _ext.BF16, fake, 16, None)
    assert st == _ext.EWORKSPACE and b"workspace" in lib.mcamd_last_error()
    st = lib.mcamd_flash_attn_with_kvcache(fake, fake, None, fake, fake, fake, fake, 2, 1, 8, 4,
                                           128, 64, 64 * 4 * 128, -1, 1, _ext.BF16, fake, 1 << 30,
                                           None)
    assert st == _ext.EINVAL and b"both k and v" in lib.mcamd_last_error()


def test_workspace_size_follows_the_split_count():
    lib = _ext.lib()
    B, H, D, T_max = 32, 16, 128, 8300
    n_splits = -(-T_max // 256)
    general = B * H * n_splits * (D + 2) * 4  # per-(row, head, split) partials, general kernel
    # per-segment partials (16 heads: o in bf16, (m, l) in fp32), bf16 / D=128: a bucket of 16
    # slots per unit, an overflow area of 1024 + units slots, then one (first group, segments)
    # int pair per unit (H = 16 query heads over 4 KV heads: one unit per row)
    slot = 16 * D * 2 + 16 * 2 * 4
    fused = (16 * B + 1024 + B) * slot + B * 8
    # and, with no window and rows x query heads >= 64, sixteen shared-prefix partial slots per
    # unit past that (32 rows x 4 query heads per KV head here): o of 16 heads in bf16, then
    # their (m, l) in fp32
    prefix = B * 16 * slot
    base = -(-max(general, fused) // 256) * 256
    got = lib.mcamd_attn_workspace_bytes(B, 1, H, 4, D, T_max, -1)
    assert got == base + prefix  # scratch only, no counters
    # 8 rows x 4 query heads per KV head: too few for the matrix cores, no prefix slots
    general8 = 8 * H * n_splits * (D + 2) * 4
    fused8 = (16 * 8 + 1024 + 8) * slot + 8 * 8
    assert lib.mcamd_attn_workspace_bytes(8, 1, H, 4, D, T_max, -1) == \
        -(-max(general8, fused8) // 256) * 256
    windowed = lib.mcamd_attn_workspace_bytes(B, 1, H, 4, D, T_max, 1024)
    assert windowed <= got
    fp32 = lib.mcamd_attn_workspace_bytes(B, 1, H, 4, 64, T_max, 1024)  # general kernel only
    assert fp32 < lib.mcamd_attn_workspace_bytes(B, 1, H, 4, 64, T_max, -1)
    assert lib.mcamd_attn_workspace_bytes(B, 7, H, 4, D, T_max, -1) == 0  # prefill needs none


def _base_workspace(B, H, H_kv, D, T_max, window=-1):
    """The decode partials of the general and fused kernels (bf16, head_dim 128), rounded up."""
    n_splits = -(-(T_max if window < 0 else min(T_max, window + 1)) // 256)
    general = B * H * n_splits * (D + 2) * 4
    units = B * -(-H_kv // 4) * -(-(H // H_kv) // 4)
    fused = (16 * units + 1024 + units) * (16 * D * 2 + 16 * 2 * 4) + units * 8
    return -(-max(general, fused) // 256) * 256, units


def test_shared_prefix_slots_only_where_the_matrix_core_kernel_takes_the_geometry():
    """The shared prompt prefix goes to the matrix-core kernel only for geometries that kernel
    takes: at most 256 query heads per KV head, and one (row, KV head)'s cache within 32-bit byte
    offsets. Elsewhere the workspace holds no prefix slots and the decode pass reads row 0."""
    lib = _ext.lib()
    D = 128
    prefix_slots = lambda units: units * 16 * (16 * D * 2 + 16 * 2 * 4)  # noqa: E731
    # 16 KV heads at 2^16 positions: offsets fit; at 2^20 they do not
    for T_max, takes in ((1 << 16, True), (1 << 20, False)):
        base, units = _base_workspace(64, 32, 16, D, T_max)
        got = lib.mcamd_attn_workspace_bytes(64, 1, 32, 16, D, T_max, -1)
        assert got == base + (prefix_slots(units) if takes else 0), T_max
    # 256 query heads per KV head fill one workgroup's pairs; 512 would not fit
    for H, takes in ((256, True), (512, False)):
        base, units = _base_workspace(1, H, 1, D, 1024)
        got = lib.mcamd_attn_workspace_bytes(1, 1, H, 1, D, 1024, -1)
        assert got == base + (prefix_slots(units) if takes else 0), H


def test_a_missing_library_raises_with_its_reason(monkeypatch, tmp_path):
    monkeypatch.setattr(_ext, "LIB_PATH", tmp_path / "absent.so")
    _ext.reload()
    try:
        with pytest.raises(RuntimeError, match="not found"):
            _ext.lib()
        assert "absent.so" in _ext.LOAD_ERROR
    finally:
        monkeypatch.undo()
        _ext.reload()
    _ext.lib()


def test_epilogue_rejects_odd_head_dim_half_kv_and_bad_dtype():
    lib = _ext.lib()
    fake = 1 << 20  # never dereferenced: the checks fail first
    args = dict(n_pos=64, batch=2, t_new=1, n_head=8, n_kv_head=2, t_max=64, cb=64 * 2 * 128)

    def call(k, v, head_dim, dtype):
        return lib.mcamd_qk_rope_norm_append(fake, 8 * head_dim, k, 2 * head_dim, v,
                                             2 * head_dim, fake, fake, args["n_pos"], fake, fake,
                                             fake, fake, args["batch"], args["t_new"],
                                             args["n_head"], args["n_kv_head"], head_dim,
                                             args["t_max"], args["cb"], 1e-6, 1.2, dtype, None)

    assert call(fake, fake, 127, _ext.BF16) == _ext.EUNSUPPORTED
    assert b"even" in lib.mcamd_last_error()
    assert call(fake, None, 128, _ext.BF16) == _ext.EINVAL
    assert b"both k and v" in lib.mcamd_last_error()
    assert call(fake, fake, 128, 9) == _ext.EINVAL
    assert b"dtype" in lib.mcamd_last_error()
    st = lib.mcamd_qk_rope_norm_append(fake, 100, fake, 256, fake, 256, fake, fake, 64, fake, fake,
                                       fake, fake, 2, 1, 8, 2, 128, 64, 64 * 2 * 128, 1e-6, 1.2,
                                       _ext.BF16, None)
    assert st == _ext.EINVAL and b"token stride" in lib.mcamd_last_error()


def test_decode_loop_entry_points_reject_bad_shapes_before_any_launch():
    """The skinny GEMM family, the residual step and the partials epilogue refuse unsupported
    shapes and null buffers on the host, each with a message naming the problem."""
    lib = _ext.lib()
    fake = 1 << 20  # never dereferenced: the checks fail first
    # skinny GEMM: rows, n / k granularity, split range
    assert lib.mcamd_linear_bf16(fake, 512, fake, fake, 64, 65, 64, 512, 1, None, 0, None) \
        == _ext.EUNSUPPORTED and b"at most 64" in lib.mcamd_last_error()
    assert lib.mcamd_linear_bf16(fake, 512, fake, fake, 96, 4, 96, 512, 1, None, 0, None) \
        == _ext.EUNSUPPORTED and b"multiple of 64" in lib.mcamd_last_error()
    assert lib.mcamd_linear_bf16(fake, 512, fake, fake, 64, 4, 64, 512, 8, None, 0, None) \
        == _ext.EUNSUPPORTED and b"128 * k_splits" in lib.mcamd_last_error()
    assert lib.mcamd_linear_bf16(fake, 512, fake, fake, 64, 4, 64, 512, 2, None, 0, None) \
        == _ext.EWORKSPACE
    assert lib.mcamd_linear_bf16_partials(fake, 512, fake, None, 4, 64, 512, 1, None) \
        == _ext.EINVAL and b"part" in lib.mcamd_last_error()
    # gated product: activation and hidden granularity
    assert lib.mcamd_linear_bf16_gated(fake, 512, fake, fake, 64, 4, 64, 512, 7, 0, None) \
        == _ext.EUNSUPPORTED and b"silu" in lib.mcamd_last_error()
    assert lib.mcamd_linear_bf16_gated(fake, 512, fake, fake, 96, 4, 96, 512, _ext.ACT_SILU, 1,
                                       None) == _ext.EUNSUPPORTED
    # residual step: exactly one of part / y, n % 8, eps
    assert lib.mcamd_residual_rmsnorm(fake, fake, 1, fake, fake, fake, 2, 16, 1e-6, None) \
        == _ext.EINVAL and b"not both" in lib.mcamd_last_error()
    assert lib.mcamd_residual_rmsnorm(fake, None, 0, fake, fake, fake, 2, 12, 1e-6, None) \
        == _ext.EINVAL
    assert lib.mcamd_residual_rmsnorm(fake, None, 0, fake, fake, fake, 2, 16, -1.0, None) \
        == _ext.EINVAL and b"eps" in lib.mcamd_last_error()
    assert lib.mcamd_residual_rmsnorm(fake, fake, 0, None, fake, fake, 2, 16, 1e-6, None) \
        == _ext.EINVAL and b"splits" in lib.mcamd_last_error()
    # the epilogue on QKV partials: split range and a row narrower than its heads
    assert lib.mcamd_qk_rope_norm_append_partials(fake, 0, 12 * 128, fake, fake, 64, fake, fake,
                                                  fake, fake, 2, 1, 8, 2, 128, 64, 64 * 2 * 128,
                                                  1e-6, 1.2, 1, None) == _ext.EINVAL
    assert lib.mcamd_qk_rope_norm_append_partials(fake, 2, 10 * 128, fake, fake, 64, fake, fake,
                                                  fake, fake, 2, 1, 8, 2, 128, 64, 64 * 2 * 128,
                                                  1e-6, 1.2, 1, None) == _ext.EINVAL
    assert b"token stride" in lib.mcamd_last_error()


def test_head_dims_past_512_are_refused_before_any_launch():
    """Any head_dim of whole 16-byte rows up to 512 runs (the power-of-two kernel above it, with
    idle lanes); wider heads have no kernel and say so without touching the GPU -- also the
    operator with new k/v, whose append would otherwise run first."""
    lib = _ext.lib()
    fake = 1 << 20  # never dereferenced
    D, T_max = 640, 64
    st = lib.mcamd_decode_attention(fake, fake, fake, fake, fake, 2, 8, 4, D, T_max,
                                    T_max * 4 * D, -1, _ext.BF16, fake, 1 << 40, None)
    assert st == _ext.EUNSUPPORTED and b"at most 512" in lib.mcamd_last_error()
    st = lib.mcamd_prefill_attention(fake, fake, fake, fake, fake, 2, 5, 8, 4, D, T_max,
                                     T_max * 4 * D, -1, _ext.BF16, None)
    assert st == _ext.EUNSUPPORTED and b"at most 512" in lib.mcamd_last_error()
    st = lib.mcamd_flash_attn_with_kvcache(fake, fake, fake, fake, fake, fake, fake, 2, 1, 8, 4,
                                           D, T_max, T_max * 4 * D, -1, 1, _ext.BF16, fake,
                                           1 << 40, None)
    assert st == _ext.EUNSUPPORTED and b"at most 512" in lib.mcamd_last_error()
    # head dims above 256 need no decode workspace: they take the general prefill kernel
    assert lib.mcamd_attn_workspace_bytes(2, 1, 8, 4, 384, T_max, -1) == 0
