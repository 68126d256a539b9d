"""Compute dtype and roofline denominators for the KV path.

``detect_compute_dtype`` follows modelcore/runtime.py:23-42: the ``MODELCORE_DTYPE`` environment
variable ("bfloat16" or "float32") wins; otherwise a GPU of capability >= (8, 0) computes in bf16
(every CDNA3/CDNA4 part reports 9.x) and anything else in fp32. The caches use this dtype
(modelcore/manager.py:286-291).

``peak_bandwidth`` / ``peak_flops`` are the MBU/MFU denominators the reference uses for MI355
(modelcore/runtime.py:162 and :200): 8.0e12 B/s of HBM3E and 2.5e15 dense bf16 FLOP/s.
"""
from __future__ import annotations

import os

import torch

_DTYPES = {"bfloat16": torch.bfloat16, "float32": torch.float32}
ENV_VAR = "MODELCORE_DTYPE"

# (name fragments, value); matched case-insensitively against the device name.
PEAK_BANDWIDTH = ((("mi355",), 8.0e12), (("mi325",), 6.0e12), (("mi300x",), 5.3e12))
PEAK_BF16_FLOPS = ((("mi355",), 2.5e15), (("mi325",), 1.3074e15), (("mi300x",), 1.3074e15))
MI355X_HBM_BYTES_PER_S = 8.0e12
MI355X_BF16_FLOPS = 2.5e15


def detect_compute_dtype():
    """(dtype, reason): the env override, else bf16 on a capable GPU, else fp32."""
    env = os.environ.get(ENV_VAR)
    if env is not None:
        if env not in _DTYPES:
            raise ValueError(f"{ENV_VAR} must be one of {sorted(_DTYPES)}, got {env!r}")
        return _DTYPES[env], f"set via {ENV_VAR}={env}"
    if torch.cuda.is_available():
        cap = torch.cuda.get_device_capability()
        if cap >= (8, 0):
            return torch.bfloat16, f"auto-detected: GPU capability {cap[0]}.{cap[1]} (bf16)"
        return torch.float32, f"auto-detected: GPU capability {cap[0]}.{cap[1]} (fp32)"
    return torch.float32, "auto-detected: no GPU (fp32)"


class Runtime:
    """Ambient values: the compute dtype and a log sink (modelcore/runtime.py:45-55)."""

    def __init__(self, compute_dtype=None, log=None):
        if compute_dtype is None:
            compute_dtype, reason = detect_compute_dtype()
        else:
            reason = "explicit"
        self.compute_dtype = compute_dtype
        self.compute_dtype_reason = reason
        self.log = log or (lambda msg: None)


def _lookup(table, device_name):
    name = device_name.lower()
    for fragments, value in table:
        if all(f in name for f in fragments):
            return value
    return float("inf")


def peak_bandwidth(device_name: str) -> float:
    """Peak HBM bytes/s for a device name; inf when unknown (so a ratio reads as 0)."""
    return _lookup(PEAK_BANDWIDTH, device_name)


def peak_flops(device_name: str) -> float:
    """Peak dense bf16 FLOP/s for a device name; inf when unknown."""
    return _lookup(PEAK_BF16_FLOPS, device_name)
