"""bf16 emulation on uint16 bit patterns (oracle, test infrastructure only).

bf16 values are carried as ``numpy.uint16`` arrays holding the raw bit pattern.
Conversion from float32 is IEEE round-to-nearest-even, which is what
``tensor.to(torch.bfloat16)`` does (the reference casts its fp32 pooled means
with ``mean_val.to(val.dtype)``, ar_sparse_operation.py:69-70).

Pinned by tests/test_oracle_bf16.py against ``torch.Tensor.to(torch.bfloat16)``
on random, boundary (ties, overflow, denormal) and special values.
"""
import numpy as np


def bf16_to_f32(bits):
    """uint16 bf16 bit patterns -> float32 values (exact)."""
    b = np.asarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x):
    """float32 -> uint16 bf16 bit patterns, round to nearest even; NaN -> quiet NaN."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    bias = 0x7FFF + ((u >> 16) & 1)
    out = ((u + bias) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        out = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), out)
    return out


def round_bf16(x):
    """float32 -> float32 value after a round trip through bf16."""
    return bf16_to_f32(f32_to_bf16(x))


def bf16_order_key(bits):
    """Monotone integer key of bf16 bit patterns: a < b  <=>  key(a) < key(b).

    -0 and +0 map to adjacent keys (-1, 0); NaNs are not expected.
    """
    b = np.asarray(bits, dtype=np.uint16).astype(np.int32)
    return np.where(b & 0x8000, -(b & 0x7FFF) - 1, b)
