"""Inference state used by the prefill entry point.

The reference reads ``hyvideo.commons.infer_state.get_infer_state()``
(bi_sparse_operation_for_KV_cache.py:8, 320-321).  Inside HY-WorldPlay that
module exists and is used; standalone, this module-level state stands in for it
(``current_chunk_index`` defaults to 0, like the reference's ``getattr`` default).
"""
try:  # the upstream model's own state when running inside HY-WorldPlay
    from hyvideo.commons.infer_state import get_infer_state  # noqa: F401
except ImportError:
    class _InferState:
        current_chunk_index = 0

    _STATE = _InferState()

    def get_infer_state():
        return _STATE
