"""Workload shapes and the seeded synthetic Q/K/V generator.

Inputs are a smooth low-frequency field over the latent (t, h, w) grid plus
0.5 * N(0, 1) noise, cast to bf16, with Q pre-scaled by 1/sqrt(D):

    x[t, h, w, :] = sum_{j<8} cos(2*pi*(kt_j*t/T + kh_j*h/H + kw_j*w/W) + phi_j) * u_j + 0.5 * n

with integer wave numbers |k| <= 2, phases phi_j ~ U(0, 2*pi) and amplitude
vectors u_j ~ N(0, 1/8)^D drawn per (tensor, head) from ``numpy.random.default_rng``.
Token order is the reference's linear (t, h, w) order with w fastest.
"""
import math
from dataclasses import dataclass, field

import numpy as np
import torch


@dataclass(frozen=True)
class Workload:
    name: str
    heads: int
    head_dim: int
    latent_hw: tuple
    frames_q: int
    frames_k: int
    tile: tuple
    ratio: float
    metric: str
    batch: int = 1
    force_diag: bool = True
    force_sink: bool = True
    ragged: tuple = None          # (min, max) per-row totals when rows are ragged
    qk_fp8: bool = False          # Q K^T on e4m3 codes with per-tile-block scales
    note: str = ""

    @property
    def lq(self):
        return self.frames_q * self.latent_hw[0] * self.latent_hw[1]

    @property
    def lk(self):
        return self.frames_k * self.latent_hw[0] * self.latent_hw[1]

    def sparse_params(self, nq_blk=None):
        p = {"tile_size": self.tile, "topk_ratio": self.ratio, "sim_metric": self.metric,
             "force_diag": self.force_diag, "force_sink": self.force_sink}
        if self.ragged is not None:
            p["row_budget"] = ragged_budgets(nq_blk, *self.ragged)
        if self.qk_fp8:
            p["qk_fp8"] = True
        return p


def ragged_budgets(nq, lo, hi, seed=7):
    """Per-query-row block totals spread over [lo, hi]: lo + round((hi-lo) * u^1.3), u = r/(nq-1), seeded permutation."""
    u = np.arange(nq) / max(nq - 1, 1)
    b = lo + np.round((hi - lo) * u ** 1.3).astype(np.int64)
    return np.random.default_rng(seed).permutation(b).tolist()


WORKLOADS = {
    "toy": Workload("toy", 4, 64, (32, 32), 2, 2, (4, 4, 4), 0.25, "scaled_dot_product",
                    note="B=1, 4 heads, D=64, T=2 x 32 x 32 (Lq = Lk = 2048), 4x4x4 tiles, 25% keep + diag + sink"),
    "hy": Workload("hy", 16, 128, (30, 52), 4, 12, (2, 8, 8), 0.3, "scaled_dot_product",
                   note="HY-WorldPlay shape: 16 heads, D=128, 30x52 latent, Lq=6240 (4 frames), "
                        "Lk=18720 (8 memory + 4 chunk frames), 2x8x8 tiles, 30% keep + diag + sink"),
    "mg": Workload("mg", 24, 128, (22, 40), 4, 20, (2, 8, 8), 0.25, "cosine",
                   note="Matrix-Game-3.0 shape: 24 heads, D=128, 22x40 latent, Lq=3520, Lk=17600, "
                        "2x8x8 tiles, 25% keep + diag + sink"),
    "hy_long": Workload("hy_long", 16, 128, (30, 52), 4, 64, (2, 8, 8), 0.1, "scaled_dot_product", ragged=(8, 200),
                        note="HY long rollout: Lq=6240, Lk=99840 (64 frames), ragged rows 8..200 blocks (~10%)"),
    "hy_fp8": Workload("hy_fp8", 16, 128, (30, 52), 4, 12, (2, 8, 8), 0.3, "scaled_dot_product", qk_fp8=True,
                       note="HY shape with Q, K as e4m3 codes and per-128-token-block fp32 scales (amax/448), "
                            "V bf16: e4m3 MFMA for Q K^T, bf16 for P V; the same selection as hy"),
    "hy_long_fp8": Workload("hy_long_fp8", 16, 128, (30, 52), 4, 64, (2, 8, 8), 0.1, "scaled_dot_product",
                            ragged=(8, 200), qk_fp8=True,
                            note="HY long rollout (as hy_long) with Q, K as e4m3 codes and per-128-token-block "
                                 "scales, V bf16; the same selection as hy_long"),
}


def smooth_field(rng, heads, frames, latent_hw, dim, noise=0.5):
    """float32 (heads, frames*H*W, dim) field + noise, token order (t, h, w) with w fastest."""
    H, W = latent_hw
    t = np.arange(frames, dtype=np.float64)[:, None, None]
    h = np.arange(H, dtype=np.float64)[None, :, None]
    w = np.arange(W, dtype=np.float64)[None, None, :]
    out = np.empty((heads, frames * H * W, dim), dtype=np.float32)
    for hd in range(heads):
        kv = rng.integers(-2, 3, size=(8, 3))
        phi = rng.uniform(0, 2 * math.pi, size=8)
        u = rng.standard_normal((8, dim)) / math.sqrt(8.0)
        basis = np.empty((frames * H * W, 8), dtype=np.float64)
        for j in range(8):
            arg = 2 * math.pi * (kv[j, 0] * t / max(frames, 1) + kv[j, 1] * h / H + kv[j, 2] * w / W) + phi[j]
            basis[:, j] = np.cos(arg).reshape(-1)
        out[hd] = (basis @ u).astype(np.float32)
        out[hd] += noise * rng.standard_normal((frames * H * W, dim), dtype=np.float32)
    return out


def make_qkv(wl, seed=0, device="cpu", layout="bhld"):
    """Seeded bf16 (q, k, v) of shape (B, H, L, D) for a workload.

    ``layout='blhd'`` returns (B, H, L, D) views of (B, L, H, D) storage, the
    transposed layout HY-WorldPlay passes in.
    """
    rng = np.random.default_rng(seed)
    B, NH, D = wl.batch, wl.heads, wl.head_dim
    out = []
    for which, frames, scale in (("q", wl.frames_q, 1.0 / math.sqrt(D)), ("k", wl.frames_k, 1.0),
                                 ("v", wl.frames_k, 1.0)):
        f = np.stack([smooth_field(rng, NH, frames, wl.latent_hw, D) for _ in range(B)])
        if scale != 1.0:
            f *= np.float32(scale)
        t = torch.from_numpy(f).to(torch.bfloat16)
        if layout == "blhd":
            t = t.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
        out.append(t.to(device))
    return tuple(out)
