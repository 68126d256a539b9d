"""Loader for the HIP library ``modelcore_amd/_lib/libmodelcore_amd.so`` (C ABI in
``include/modelcore_amd.h``).

The library is opened with ctypes after ``import torch``: PyTorch-ROCm has then already mapped its
own ``libamdhip64.so`` (SONAME ``libamdhip64.so.7``), and the library's dependency on that SONAME
resolves to the same HIP runtime, so device pointers and ``hipStream_t`` handles from torch are
valid here. A failed load is recorded as a reason string (``LOAD_ERROR``) and every entry point
raises it through :func:`lib`; there is no other implementation to fall back to.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (must be imported first: it provides the HIP runtime)

LIB_PATH = Path(os.environ.get("MODELCORE_AMD_LIB",
                               Path(__file__).resolve().parent / "_lib" / "libmodelcore_amd.so"))

# Element-type and status codes of the C ABI.
F32, BF16 = 0, 1
ACT_SILU = 0  # mcamd_linear_bf16_gated activations
OK, EINVAL, EUNSUPPORTED, EWORKSPACE, ELAUNCH = 0, -1, -2, -3, -4
ABI_VERSION = 8
NOALLOC_SCRATCH_BYTES = 32 << 20  # MCAMD_NOALLOC_SCRATCH_BYTES

_i64 = ctypes.c_int64
_int = ctypes.c_int
_ptr = ctypes.c_void_p
_size = ctypes.c_size_t

# name -> (restype, argtypes); the exact set the header declares.
SIGNATURES = {
    "mcamd_abi_version": (_int, []),
    "mcamd_last_error": (ctypes.c_char_p, []),
    "mcamd_kv_append": (_int, [_ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _i64,
                               _int, _ptr]),
    "mcamd_kv_replicate": (_int, [_ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _i64,
                                  _i64, _i64, _i64, _int, _ptr]),
    "mcamd_attn_workspace_bytes": (_size, [_i64, _i64, _i64, _i64, _i64, _i64, _i64]),
    "mcamd_flash_attn_with_kvcache": (_int, [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64,
                                             _i64, _i64, _i64, _i64, _i64, _i64, _int, _int, _ptr,
                                             _size, _ptr]),
    "mcamd_flash_attn_with_kvcache_ex": (_int, [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64,
                                                _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int,
                                                _int, ctypes.c_int32, _i64, _ptr, _size, _ptr]),
    "mcamd_flash_attn_with_kvcache_noalloc": (_int, [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr,
                                                     _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                                     _i64, _int, _int, _ptr]),
    "mcamd_flash_attn_varlen_with_kvcache": (_int, [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr,
                                                    _ptr, _ptr, _i64, _i64, _i64, _i64, _i64,
                                                    _i64, _i64, _i64, _int, _int, _int, _ptr]),
    "mcamd_decode_attention": (_int, [_ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64,
                                      _i64, _i64, _int, _ptr, _size, _ptr]),
    "mcamd_prefill_attention": (_int, [_ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64,
                                       _i64, _i64, _i64, _i64, _int, _ptr]),
    "mcamd_sample_tokens": (_int, [_ptr, _i64, _i64, _i64, ctypes.c_float, _i64, _ptr, _ptr,
                                   _ptr, _ptr]),
    "mcamd_qk_rope_norm_append": (_int, [_ptr, _i64, _ptr, _i64, _ptr, _i64, _ptr, _ptr, _i64,
                                         _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64,
                                         _i64, _i64, ctypes.c_float, ctypes.c_float, _int,
                                         _ptr]),
    "mcamd_qk_rope_norm_append_partials": (_int, [_ptr, _i64, _i64, _ptr, _ptr, _i64, _ptr, _ptr,
                                                  _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _i64,
                                                  _i64, ctypes.c_float, ctypes.c_float, _int,
                                                  _ptr]),
    "mcamd_linear_bf16_workspace_bytes": (_size, [_i64, _i64, _i64]),
    "mcamd_linear_bf16": (_int, [_ptr, _i64, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _ptr,
                                 _size, _ptr]),
    "mcamd_linear_bf16_gated": (_int, [_ptr, _i64, _ptr, _ptr, _i64, _i64, _i64, _i64, _int,
                                       _int, _ptr]),
    "mcamd_linear_bf16_partials": (_int, [_ptr, _i64, _ptr, _ptr, _i64, _i64, _i64, _i64, _ptr]),
    "mcamd_residual_rmsnorm": (_int, [_ptr, _ptr, _i64, _ptr, _ptr, _ptr, _i64, _i64,
                                      ctypes.c_float, _ptr]),
}

_LIB = None
LOAD_ERROR: str | None = None


def _load():
    """Open the library once. Returns (handle_or_None, reason_or_None)."""
    if not LIB_PATH.exists():
        return None, f"{LIB_PATH} not found: build it with `python -m modelcore_amd.build`"
    try:
        handle = ctypes.CDLL(str(LIB_PATH))
    except OSError as e:
        return None, f"loading {LIB_PATH} failed: {e}"
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name, None)
        if fn is None:
            return None, f"{LIB_PATH} does not export {name}"
        fn.restype, fn.argtypes = res, args
    version = handle.mcamd_abi_version()
    if version != ABI_VERSION:
        return None, f"{LIB_PATH} has ABI version {version}, expected {ABI_VERSION}"
    return handle, None


def lib():
    """The loaded library; raises RuntimeError with the load failure's reason if it is missing."""
    global _LIB, LOAD_ERROR
    if _LIB is None:
        _LIB, LOAD_ERROR = _load()
        if _LIB is None:
            raise RuntimeError(f"modelcore_amd HIP library unavailable: {LOAD_ERROR}")
    return _LIB


def reload():
    """Forget the loaded handle and reason (tests point LIB_PATH elsewhere, then call this)."""
    global _LIB, LOAD_ERROR
    _LIB, LOAD_ERROR = None, None


def check(status: int, what: str):
    """Raise the library's own message for a non-zero status."""
    if status != OK:
        msg = lib().mcamd_last_error().decode(errors="replace")
        exc = ValueError if status in (EINVAL, EWORKSPACE) else RuntimeError
        raise exc(f"{what} failed (status {status}): {msg}")


def dtype_code(dtype) -> int:
    if dtype == torch.bfloat16:
        return BF16
    if dtype == torch.float32:
        return F32
    raise TypeError(f"modelcore_amd kernels take bfloat16 or float32 tensors, got {dtype}")


def stream_handle(device) -> int:
    """hipStream_t of torch's current stream on `device`, as an integer for ctypes."""
    return torch.cuda.current_stream(device).cuda_stream


_WORKSPACES: dict[int, torch.Tensor] = {}
_RETIRED: list[torch.Tensor] = []


def workspace(device, nbytes: int):
    """A device buffer of at least `nbytes` for the attention entry points, or None for 0.

    The workspace is scratch: a call needs no particular contents in it and leaves none that a
    later call relies on. One buffer per device is kept and reused by every call issued on that
    device's stream (calls on two streams at once would share it and race). A buffer that is
    outgrown is retired but kept alive, so a graph captured with it stays valid. During graph
    capture a too-small buffer is not replaced: the call gets one of its own from the graph's
    pool.
    """
    if nbytes == 0:
        return None
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ws = _WORKSPACES.get(idx)
    if ws is not None and ws.numel() >= nbytes:
        return ws
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(nbytes, dtype=torch.uint8, device=device)
    size = max(nbytes, 2 * ws.numel() if ws is not None else 0, 1 << 20)
    if ws is not None:
        _RETIRED.append(ws)
    ws = torch.empty(size, dtype=torch.uint8, device=device)
    _WORKSPACES[idx] = ws
    return ws


def require_rocm(*tensors, what: str):
    """Every tensor must live on a ROCm device: the HIP kernels are the only implementation."""
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(
                f"{what}: modelcore_amd runs its KV path only as HIP kernels on a ROCm device; "
                f"got a tensor on {t.device}")
