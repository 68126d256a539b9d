"""The residual update and the next RMS-norm of a block, fused into one HIP launch
(``mcamd_residual_rmsnorm``): given the residual stream x and a projection's output f (a bf16
tensor, or its unsummed K-split partials from ``linear_bf16_partials``), returns

    x_out = x + f                 (bf16, as torch adds two bf16 tensors)
    h     = rms_norm(x_out, eps)  (fp32 arithmetic, bf16 result)

Replaces, in a block of the reference (modelcore/components/block.py:57-59), the residual add
``x = x + mixer(...)`` / ``x = x + ffn(h)`` and the RMSNorm after it (modelcore/components/norm.py:
43-44), together with the split-K sum of the projection: three launches become one. ``h`` equals
``F.rms_norm(x_out)`` up to the order of the fp32 sum of squares.
"""
from __future__ import annotations

import torch

from modelcore_amd import _ext
from modelcore_amd.kernels.linear import Partials
from modelcore_amd.kernels.qk_epilogue import default_eps

__all__ = ["residual_rmsnorm", "supported"]


def supported(x: torch.Tensor) -> bool:
    """Whether residual_rmsnorm takes this residual stream (bf16 on the GPU, rows of n % 8 == 0)."""
    return x.dtype == torch.bfloat16 and x.device.type == "cuda" and x.dim() >= 1 \
        and x.shape[-1] % 8 == 0 and x.numel() > 0


def residual_rmsnorm(x: torch.Tensor, f, eps: float | None = None):
    """(x + f, rms_norm(x + f)) for a bf16 residual stream x and f a bf16 tensor of x's shape or
    the Partials of the projection that makes it."""
    _ext.require_rocm(x, what="residual_rmsnorm")
    if not supported(x):
        raise ValueError(f"residual_rmsnorm takes a bf16 GPU tensor with rows of a multiple of 8; "
                         f"got {tuple(x.shape)} {x.dtype} on {x.device}")
    n = x.shape[-1]
    xc = x.contiguous()
    m = xc.numel() // n
    part, splits, y = None, 0, None
    if isinstance(f, Partials):
        if tuple(f.shape) != tuple(x.shape) or f.part.shape != (f.splits, m, n):
            raise ValueError(f"partials of shape {tuple(f.shape)} do not match x {tuple(x.shape)}")
        part, splits = f.part, f.splits
    else:
        if f.shape != x.shape or f.dtype != x.dtype or f.device != x.device:
            raise ValueError(f"f {tuple(f.shape)} {f.dtype} does not match x {tuple(x.shape)}")
        y = f.contiguous()
    x_out = torch.empty_like(xc)
    h = torch.empty_like(xc)
    st = _ext.lib().mcamd_residual_rmsnorm(
        xc.data_ptr(), None if part is None else part.data_ptr(), splits,
        None if y is None else y.data_ptr(), x_out.data_ptr(), h.data_ptr(), m, n,
        default_eps() if eps is None else float(eps), _ext.stream_handle(x.device))
    _ext.check(st, "residual_rmsnorm")
    return x_out, h
