"""OCP e4m3 (float8_e4m3fn) codes and per-block quantization (oracle, test infrastructure only).

The reference has no fp8 path; this restates the fp8 variant of its
block-sparse attention (``_attn_fwd_bsa_align``, longcat_kernel.py:27-155)
in which Q and K enter the score product as e4m3 codes with one fp32 scale
per 128-token tile block:

* encode: round to nearest even on the e4m3 grid (subnormals down to 2^-9,
  largest finite 448 = 0x7E).  The code 0x7F is the NaN, so a magnitude that
  rounds to the next grid step (480, i.e. above 464; 464 itself ties to
  even, to 448) or is infinite becomes NaN; the sign bit is kept, also for
  zero.  This is what gfx950's ``v_cvt_pk_fp8_f32`` and
  ``torch.Tensor.to(torch.float8_e4m3fn)`` do for every non-NaN input (a NaN
  input gives 0xFF on the GPU and 0x7F | sign in torch).
* block quantization of a (..., BS, D) tile block x (fp32 values):
  ``amax = max |x|``; ``scale = amax / 448`` and ``inv = 448 / amax`` in
  fp32 (``scale = inv = 1`` for an all-zero block); codes ``e4m3(x * inv)``.
  ``|x * inv| <= 448 (1 + 2^-23)`` rounds to at most 448, so a finite block
  never produces NaN.  Dequantized values are ``decode(code) * scale``.

Pinned by tests/test_oracle_fp8.py: encode equals torch's float8_e4m3fn cast
on every finite bf16 bit pattern, on grid midpoints and their fp32
neighbours, and on random fp32; decode equals torch's cast back to float32
on all 256 codes; the block quantizer's codes never overflow, its
dequantized values are within half an e4m3 step of the input, and it is
exact on inputs that are e4m3 values times a power of two.
"""
import numpy as np

# Finite e4m3 magnitudes of codes 0x00..0x7E (0x7F is NaN).
_MAG = np.array([(m / 8.0) * 2.0 ** -6 if e == 0 else (1.0 + m / 8.0) * 2.0 ** (e - 7)
                 for e in range(16) for m in range(8)], dtype=np.float64)[:127]


def e4m3_decode(codes):
    """uint8 e4m3 codes -> float32 values (NaN for 0x7F / 0xFF)."""
    c = np.asarray(codes, dtype=np.uint8)
    mag = np.concatenate([_MAG, [np.nan]]).astype(np.float32)[c & 0x7F]
    return np.where(c & 0x80, -mag, mag).astype(np.float32)


def e4m3_encode(x):
    """float32 -> uint8 e4m3 codes: round to nearest even, magnitudes above 464 (and inf) -> NaN code.

    NaN inputs map to 0x7F | sign.
    """
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64)
    sign = np.signbit(x).astype(np.uint8) << 7
    # Extended grid: the 127 finite magnitudes plus 480 at code 0x7F, so that
    # rounding past 464 lands on the NaN code by itself.
    grid = np.concatenate([_MAG, [480.0]])
    hi = np.clip(np.searchsorted(grid, a, side="left"), 1, 127)
    lo = hi - 1
    dlo = a - grid[lo]
    dhi = grid[hi] - a
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    code = np.where(a <= grid[0], 0, code).astype(np.uint8)
    code = np.where((a > 464.0) | np.isnan(a), 0x7F, code).astype(np.uint8)
    return (code | sign).astype(np.uint8)


def quantize_blocks(x):
    """Per-block e4m3 quantization of (..., BS, D) float32 tile blocks.

    Returns (codes uint8 of x's shape, scales float32 of shape x.shape[:-2]).
    """
    x = np.asarray(x, dtype=np.float32)
    amax = np.abs(x).max(axis=(-2, -1)).astype(np.float32)
    zero = amax == 0
    safe = np.where(zero, np.float32(1.0), amax).astype(np.float32)
    scale = np.where(zero, np.float32(1.0), safe / np.float32(448.0)).astype(np.float32)
    inv = np.where(zero, np.float32(1.0), np.float32(448.0) / safe).astype(np.float32)
    codes = e4m3_encode((x * inv[..., None, None]).astype(np.float32))
    return codes, scale


def dequantize_blocks(codes, scales):
    """float32 values of quantized blocks: decode(code) * scale (exact in float64)."""
    return e4m3_decode(codes).astype(np.float64) * np.asarray(scales, dtype=np.float64)[..., None, None]
