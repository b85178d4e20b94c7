"""CPU oracle for the hierarchical group attention path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package (``multics_amd``)
imports, calls or links anything in this directory.  It may be used only by
``tests/``, by ``__graft_entry__.smoke()`` and by the ``cpu_baseline`` leg of
``bench.py`` -- and there only as the checker or as the reported CPU baseline,
never as the thing measured or shipped.

Every function restates an algorithm of the reference (TencentARC/Multics) and
cites the reference file:line it follows.  Modules:

* ``metadata``   -- segmented key lists, Tiled128 packing, varlen plan
                    (``multics/models/kernels/hier_*_attention.py``).
* ``masks``      -- the dense hierarchical mask rule, labels / membership /
                    no-local forms (``multics/models/hier_masks.py:364-641``).
* ``attention``  -- masked SDPA in fp32, RMSNorm, camera Q/K adapter, RoPE
                    and freqs builders, camera12 (``multics/models/attention.py``,
                    ``multics/models/rope.py``, ``multics/data/*.py``).
* ``cached``     -- the rolling per-stream KV cache and the cached per-stream
                    forward of a rollout block (``multics/models/attention.py:
                    90-228, 456-1005``).
* ``ste``        -- the fp32 autograd definition of the membership
                    straight-through gradient (no reference counterpart).

Parity pins (what each function is checked against) are listed in the module
headers; a function with no independent check says "parity unpinned".
"""
