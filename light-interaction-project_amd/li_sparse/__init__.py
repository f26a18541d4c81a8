"""MI355X-native AR-aware 3D block-sparse attention (Light Interaction's sparse backend).

Drop-in modules with the reference's call signatures:

* ``li_sparse.hy.ar_sparse_operation``: ``run_sparse_attention``, ``fast_generate_indices``,
  ``launch_q_prep``, ``launch_kv_prep``, ``launch_untile``
  (hy-worldplay/files/hyvideo/models/transformers/modules/ar_sparse_operation.py)
* ``li_sparse.hy.bi_sparse_operation_for_KV_cache``: ``run_sparse_prefill_attention``,
  ``generate_prefill_indices`` (.../bi_sparse_operation_for_KV_cache.py)
* ``li_sparse.hy.longcat_kernel`` / ``li_sparse.mg.longcat_kernel``: ``longcat_flash_attn``
* ``li_sparse.mg.bi_sparse_operation``: ``run_sparse_attention``, ``generate_prefill_indices``
  (matrix-game-3.0/files/wan/modules/bi_sparse_operation.py)

``ContextCache`` keeps the key-side preparation of the fixed context frames
and the text across the denoise steps of a chunk (``sparse_params`` keys
``context_cache`` and ``context_frames``).

All compute runs in the HIP kernels of ``libli_sparse_attn.so``; importing this
package fails if the library is not built.
"""
from . import _lib  # noqa: F401  (fails loudly when the native library is missing)
from ._pipeline import ContextCache  # noqa: F401
