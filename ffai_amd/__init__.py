"""ffai_amd: MI355X-native (gfx950, HIP) fused attention for FFAI's Whisper path.

The product is ``libffai_attn.so`` (C ABI: ``include/ffai_*.h``); this package builds it
(``ffai_amd.build``) and exposes it on torch device tensors:

* ``ffai_amd.flash_attn``: the mirror of the reference's ``serves`` / ``attend`` /
  ``attend_merged`` plus the general ``attention``;
* ``ffai_amd.kv_cache``: device-resident beam-search decode state (K/V append in place, beam
  reorder, the cross-attention cache build, prompt steps);
* ``ffai_amd.encoder``: the audio encoder's self-attention block (projections around the fused
  kernel);
* ``ffai_amd.gemv``: the decoder's single-row projections and the int8 vocabulary head.
"""

from . import _lib  # noqa: F401

__all__ = ["flash_attn", "kv_cache", "encoder", "gemv", "build"]
