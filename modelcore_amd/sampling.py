"""On-device next-token sampling with a counter-based random stream per row.

``PhiloxSampler`` draws one token per row from softmax(logits / temperature) with the HIP kernel
``mcamd_sample_tokens`` (Gumbel-max with Philox4x32-10 noise; C ABI in include/modelcore_amd.h).
Row r is keyed by its own 64-bit seed (``base_seed + r`` by default) and a device-side counter
that each call advances, so:

* a row's tokens depend only on its seed, its logits and how many tokens it has drawn -- not on
  the batch it is decoded in, nor on the other rows;
* nothing is read back to the host, so a decode step that samples stays asynchronous.

This is the sampling half of modelcore/generate.py:18-34 (``sample_next_token`` with
temperature > 0, with or without top_k) restated for the device; the reference draws from one
torch.Generator for the whole batch, which has no per-row meaning. Temperature 0 is the argmax,
as in the reference. With top_k the draw is over the k largest logits of each row (ties at the
k-th value kept lowest index first).
"""
from __future__ import annotations

import torch

from modelcore_amd import _ext


class PhiloxSampler:
    def __init__(self, batch_size, device, base_seed=0, seeds=None):
        if seeds is None:
            seeds = [base_seed + r for r in range(batch_size)]
        if len(seeds) != batch_size:
            raise ValueError(f"need {batch_size} seeds, got {len(seeds)}")
        _ext.require_rocm(torch.empty(0, device=device), what="PhiloxSampler")
        self.batch_size = batch_size
        self.seeds = torch.tensor([s & (2 ** 64 - 1) for s in seeds], dtype=torch.uint64,
                                  device=device)
        self.offsets = torch.zeros(batch_size, dtype=torch.int64, device=device)

    def __call__(self, logits, temperature=1.0, top_k=None):
        """(B, V) logits -> (B, 1) int64 token ids; advances every row's counter by one."""
        _ext.require_rocm(logits, what="PhiloxSampler")
        if logits.dim() != 2 or logits.size(0) != self.batch_size:
            raise ValueError(f"logits must be ({self.batch_size}, vocab); got {tuple(logits.shape)}")
        if temperature < 0:
            raise ValueError("temperature must be non-negative")
        if logits.dtype != torch.float32:
            logits = logits.float()
        if logits.stride(1) != 1 or 0 < logits.stride(0) < logits.size(1):
            logits = logits.contiguous()  # a stride-0 (expanded) batch is read as is
        out = torch.empty(self.batch_size, dtype=torch.int64, device=logits.device)
        st = _ext.lib().mcamd_sample_tokens(
            logits.data_ptr(), self.batch_size, logits.size(1), logits.stride(0),
            float(temperature), int(top_k or 0), self.seeds.data_ptr(), self.offsets.data_ptr(),
            out.data_ptr(),
            _ext.stream_handle(logits.device))
        _ext.check(st, "sample_tokens")
        return out.view(-1, 1)
