"""ffai_amd: MI355X-native (gfx950, HIP) fused attention for FFAI's Whisper path.

The product is ``libffai_attn.so`` (C ABI: ``include/ffai_attn.h``); this package builds it
(``ffai_amd.build``) and exposes it on torch device tensors (``ffai_amd.flash_attn``: the mirror
of the reference's ``serves`` / ``attend`` / ``attend_merged`` plus the general ``attention``;
``ffai_amd.decode``: device-resident beam-search decode state).
"""

from . import _lib  # noqa: F401

__all__ = ["flash_attn", "build"]
