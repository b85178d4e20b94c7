"""MI355X-native hierarchical player/group/global attention (Multics hot path).

HIP kernels for gfx950 behind a C ABI (``include/hierattn.h``), driven from
Python through ctypes.  Public entry points mirror the reference's names:

* ``metadata``  -- ``_build_metadata``, ``build_hier_tiled_full_sequence_layouts``,
  ``build_hier_tiled_cached_layout`` (device builder, bit-exact arrays).
* ``kernels``   -- ``hierarchical_tiled_full_sequence_attention`` and the
  fused Q/K prologue.
"""

__version__ = "0.1.0"
