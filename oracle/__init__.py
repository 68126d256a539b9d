"""CPU oracle for the KV-cache and cached-attention path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package, and only as the checker (or, for the baseline, the timed CPU restatement).
The product (``modelcore_amd``) never imports it and has no CPU path.

* ``kv_oracle`` -- numpy restatement of the reference algorithm:
  append (modelcore/kernels/flash_attn.py:336-346), replication (modelcore/cache.py:84-85,
  :106-107), the key-visibility rule (flash_attn.py:226-235, :246-264) and masked GQA attention
  (flash_attn.py:348-366), in float64.
* ``sdpa_fallback`` -- the reference's CPU fallback restated with the same torch ops
  (slice assign / index_put, sliced or masked ``scaled_dot_product_attention`` with
  ``enable_gqa``), used as the CPU baseline and as a second, library-routine check of
  ``kv_oracle``.

How each function is pinned (tests/test_oracle.py):
* append, replicate: bit-exact against explicit per-element loops and the reference's own
  known-answer tests restated (test_kernels.py:500-510, test_cache.py:38-56).
* visibility mask + attention: against pure-Python float64 brute force on tiny shapes, against
  torch's SDPA (the library routine the reference calls), against closed forms (window 0 returns
  the row's own value; constant V returns V; equal keys average the visible values), and against
  the reference's invariants (ragged batch == rows alone, stale data unreachable, per-row window).
  Planted mistakes (off-by-one window, wrong GQA head map, missing scale) must fail those checks.
"""
