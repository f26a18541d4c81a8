"""CPU oracle for the AR-aware 3D block-sparse attention path.

TEST INFRASTRUCTURE ONLY.  This package restates, on the CPU and in numpy, the
reference's algorithm for the sparse-attention backend of Light Interaction
(tile gather / mean-pool, block-mask selection, block-sparse flash forward and
the inverse untile scatter).  It is the checker that the HIP implementation is
compared against.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product package never
does, and nothing here is ever the thing that is measured or shipped.

Reference files restated (paths relative to the reference repository root):

* ``hy-worldplay/files/hyvideo/models/transformers/modules/ar_sparse_operation.py``
  (tile geometry, gather/pool, untile, decode-path index builder)
* ``hy-worldplay/files/hyvideo/models/transformers/modules/bi_sparse_operation_for_KV_cache.py``
  (prefill index builder with the 3D neighbour bias)
* ``matrix-game-3.0/files/wan/modules/bi_sparse_operation.py`` (same, MG defaults)
* ``hy-worldplay/files/hyvideo/models/transformers/modules/longcat_kernel.py``
  (block-sparse flash-attention forward semantics)

Modules:

* :mod:`oracle.bf16`      -- bf16 round-to-nearest-even emulation on uint16 bit patterns.
* :mod:`oracle.geometry`  -- block geometry and the (t,h,w) tile permutation.
* :mod:`oracle.tile`      -- tile gather, fixed-order fp32 mean pool, untile.
* :mod:`oracle.mask`      -- pooled similarity with the reference's bf16 rounding
  points, forced-block rules, budgets and top-k selection.
* :mod:`oracle.attention` -- float64 block-sparse attention and the torch-CPU
  dense-masked baseline.

Pinning status of each function is stated in its module docstring.
"""
