"""modelcore_amd: the KV-cache and cached-attention path of modelcore, as hand-written HIP
kernels for the MI355X (gfx950) behind the reference's own Python surface.

* ``modelcore_amd.cache.KVCache`` -- drop-in for ``modelcore.cache.KVCache``.
* ``modelcore_amd.kernels.flash_attn.flash_attn`` -- drop-in for the FA3-style operator namespace
  ``modelcore.kernels.flash_attn.flash_attn``.
* ``modelcore_amd.build`` -- compiles ``csrc/*.hip`` into ``_lib/libmodelcore_amd.so``.
"""
__version__ = "0.1.0"

from modelcore_amd.cache import KVCache  # noqa: E402
from modelcore_amd.kernels.flash_attn import flash_attn  # noqa: E402

__all__ = ["KVCache", "flash_attn", "__version__"]
