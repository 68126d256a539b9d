"""Compute dtype and roofline denominators for the KV path.

``detect_compute_dtype`` follows modelcore/runtime.py:23-42: the ``MODELCORE_DTYPE`` environment
variable ("bfloat16" or "float32") wins, and any other value raises KeyError as the reference's
table lookup does; otherwise a GPU of capability >= (8, 0) computes in bf16 (every CDNA3/CDNA4
part reports 9.x) and anything else in fp32. The caches use this dtype
(modelcore/manager.py:286-291).

``peak_bandwidth`` / ``peak_flops`` are the MBU/MFU denominators of the reference's tables for
AMD's CDNA parts (modelcore/runtime.py:162-167 and :200-205): MI355 = 8.0e12 B/s of HBM3E and
2.5e15 dense bf16 FLOP/s. An unknown name gives inf, so a ratio reads as 0 rather than a guess.
``device_peaks`` adds what the name tables cannot see: a ROCm device whose marketing name is not
reported (the name lookup needs a libdrm table some images lack) is recognised by its gfx950
architecture, the MI355X this path is built for.
"""
from __future__ import annotations

import os

import torch

_DTYPE_MAP = {"bfloat16": torch.bfloat16, "float32": torch.float32}
ENV_VAR = "MODELCORE_DTYPE"

# (name fragments, value); matched case-insensitively against the device name, first match wins.
PEAK_BF16_FLOPS_TABLE = (
    (["mi355"], 2.5e15),
    (["mi325"], 1.3074e15),
    (["mi300x"], 1.3074e15),
    (["mi300a"], 980.6e12),
    (["mi250x"], 383e12),
    (["mi250"], 362.1e12),
)
PEAK_BANDWIDTH_TABLE = (
    (["mi355"], 8.0e12),
    (["mi325"], 6.0e12),
    (["mi300x"], 5.3e12),
    (["mi300a"], 5.3e12),
    (["mi250x"], 3.28e12),
    (["mi250"], 3.28e12),
)
# gcnArchName prefix -> the name the tables know it by.
_ARCH_NAMES = {"gfx950": "mi355"}


def detect_compute_dtype():
    """(dtype, reason): the env override, else bf16 on a capable GPU, else fp32."""
    env = os.environ.get(ENV_VAR)
    if env is not None:
        return _DTYPE_MAP[env], f"set via {ENV_VAR}={env}"
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


def _lookup(table, device_name, what, log):
    name = device_name.lower()
    for fragments, value in table:
        if all(f in name for f in fragments):
            return value
    (log or (lambda msg: None))(f"Peak {what} undefined for: {device_name}")
    return float("inf")


def peak_bandwidth(device_name: str, table=PEAK_BANDWIDTH_TABLE, log=None) -> float:
    """Peak HBM bytes/s for a device name; inf when unknown (so a ratio reads as 0)."""
    return _lookup(table, device_name, "bandwidth", log)


def peak_flops(device_name: str, table=PEAK_BF16_FLOPS_TABLE, log=None) -> float:
    """Peak dense bf16 FLOP/s for a device name; inf when unknown."""
    return _lookup(table, device_name, "flops", log)


def device_peaks(index: int = 0):
    """(HBM bytes/s, dense bf16 FLOP/s, how they were found) for a visible GPU: by its name, or
    else by its architecture (gfx950 = MI355X)."""
    name = torch.cuda.get_device_name(index)
    bw, fl = peak_bandwidth(name), peak_flops(name)
    if bw != float("inf") and fl != float("inf"):
        return bw, fl, f"device name {name!r}"
    arch = getattr(torch.cuda.get_device_properties(index), "gcnArchName", "") or ""
    for prefix, alias in _ARCH_NAMES.items():
        if arch.startswith(prefix):
            return peak_bandwidth(alias), peak_flops(alias), f"architecture {arch} ({alias})"
    return bw, fl, f"device name {name!r} (not in the tables)"
