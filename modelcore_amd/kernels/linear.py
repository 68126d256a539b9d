"""Decode-sized products on the matrix cores: ``y = x . W^T`` for at most 64 rows of bf16
activations, the projection GEMMs of a decode step (``F.linear`` in the reference's
``Linear.forward``, modelcore/components/linear.py:13-14).

With 64 or fewer rows each weight byte is used at most 64 times, so the product is bound by
reading W once from HBM; ``mcamd_linear_bf16`` streams W with a K-split inside each workgroup
and sums the partials in a fixed order (deterministic, fp32 accumulation). ``supported`` says
which shapes it takes; the caller keeps ``F.linear`` for the rest (prefill-sized batches, fp32).
"""
from __future__ import annotations

import torch

from modelcore_amd import _ext

__all__ = ["supported", "linear_bf16"]

MAX_ROWS = 64


def supported(x: torch.Tensor, w: torch.Tensor) -> bool:
    """Whether ``linear_bf16(x, w)`` takes these operands (device, dtype, sizes, layout)."""
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or x.device.type != "cuda" \
            or w.device != x.device or w.dim() != 2 or not w.is_contiguous():
        return False
    n, k = w.shape
    if x.shape[-1] != k or n % 32 or k % 512:
        return False
    rows = x.numel() // k if k else 0
    return 0 < rows <= MAX_ROWS


def _rows_per_group(n: int) -> int:
    # 64 W rows per workgroup halves the activation re-reads but halves the workgroups; keep at
    # least ~2 k workgroups' worth of waves for the wide projections only.
    return 64 if n % 64 == 0 and n >= 16384 else 32


def linear_bf16(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """(..., k) bf16 x (n, k) bf16 -> (..., n) bf16, for at most 64 rows of x."""
    _ext.require_rocm(x, w, what="linear_bf16")
    if not supported(x, w):
        raise ValueError(f"linear_bf16 takes bf16 x with <= {MAX_ROWS} rows and a contiguous bf16 "
                         f"(n, k) weight, n % 32 == 0, k % 512 == 0; got x {tuple(x.shape)} "
                         f"{x.dtype}, w {tuple(w.shape)} {w.dtype}")
    n, k = w.shape
    x2 = x.reshape(-1, k)
    if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    y = torch.empty(x2.shape[0], n, dtype=torch.bfloat16, device=x.device)
    st = _ext.lib().mcamd_linear_bf16(x2.data_ptr(), x2.stride(0), w.data_ptr(), y.data_ptr(), n,
                                      x2.shape[0], n, k, _rows_per_group(n),
                                      _ext.stream_handle(x.device))
    _ext.check(st, "linear_bf16")
    return y.view(*x.shape[:-1], n)
