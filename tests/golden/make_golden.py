"""Writes the golden block-selection fixtures (run from the repo root: python tests/golden/make_golden.py).

Inputs: seeded bf16 Q/K pools for small grids.  Expected outputs: the index
lists of the reference's index builders as written with the reference's own
torch calls (tests/torch_ref.py), plus the bf16 similarity scores they rank.
Ties in ``torch.topk`` are unspecified, so each case also stores which rows are
tie-free (k-th and (k+1)-th ranked non-forced scores at least two bf16 ulps
apart); tests compare on those rows.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import torch_ref  # noqa: E402

CASES = [
    # name, mode, B, H, D, grid (nt_q, nt_k, nh, nw), text_len, params
    ("decode_recent_sdp", "decode", 1, 3, 128, (2, 6, 4, 7), 0,
     {"tile_size": (2, 8, 8), "topk_ratio": 0.175, "recent_protect": 4, "sim_metric": "scaled_dot_product"}),
    ("decode_cosine_text", "decode", 2, 2, 64, (1, 5, 3, 5), 300,
     {"tile_size": (4, 4, 8), "topk_ratio": 0.3, "recent_protect": 4, "sim_metric": "cosine"}),
    ("decode_diag_sink", "decode", 1, 4, 128, (2, 6, 4, 7), 0,
     {"tile_size": (2, 8, 8), "topk_ratio": 0.3, "sim_metric": "scaled_dot_product",
      "force_diag": True, "force_sink": True}),
    ("decode_dot", "decode", 1, 2, 64, (1, 4, 8, 8), 0,
     {"tile_size": (4, 4, 4), "topk_ratio": 0.25, "recent_protect": 2, "sim_metric": "dot"}),
    ("prefill_sdp", "prefill", 1, 3, 128, (3, 3, 4, 7), 0,
     {"tile_size": (4, 8, 4), "topk_ratio": 0.3, "sim_metric": "scaled_dot_product"}),
    ("prefill_cosine_mg", "prefill", 1, 2, 128, (5, 5, 3, 5), 0,
     {"tile_size": (4, 4, 8), "topk_ratio": 0.2, "sim_metric": "cosine"}),
]


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def order_key(b):
    b = b.astype(np.int32)
    return np.where(b & 0x8000, -(b & 0x7FFF) - 1, b)


def tie_free_rows(score_bits, final, ntxt, biased):
    """Rows where the last selected and first unselected non-forced scores differ by >= 2 ulps."""
    B, H, nq, nk = score_bits.shape
    key = order_key(score_bits)
    out = np.ones((B, H, nq), dtype=bool)
    for b in range(B):
        for h in range(H):
            for r in range(nq):
                sel = np.zeros(nk, dtype=bool)
                sel[final[b, h, r, ntxt:] - ntxt] = True
                free = ~biased[b, h, r]
                s_in, s_out = key[b, h, r, sel & free], key[b, h, r, (~sel) & free]
                if s_in.size and s_out.size:
                    out[b, h, r] = s_in.min() - s_out.max() >= 2
    return out


def main():
    out = {}
    for ci, (name, mode, B, H, D, grid, text_len, params) in enumerate(CASES):
        nt_q, nt_k, nh, nw = grid
        nq, nk = nt_q * nh * nw, nt_k * nh * nw
        g = torch.Generator().manual_seed(1000 + ci)
        base = torch.randn(B, H, 1, D, generator=g)
        qp = (base + 0.7 * torch.randn(B, H, nq, D, generator=g)).to(torch.bfloat16)
        kp = (base + 0.7 * torch.randn(B, H, nk, D, generator=g)).to(torch.bfloat16)
        if mode == "decode":
            final, s, score = torch_ref.decode_select(qp, kp, text_len, (nt_q, nh, nw), (nt_k, nh, nw), params)
        else:
            final, s, score = torch_ref.prefill_select(qp, kp, text_len, (nt_k, nh, nw), params)
        bs = params["tile_size"][0] * params["tile_size"][1] * params["tile_size"][2]
        ntxt = (text_len + bs - 1) // bs
        biased = (score.float() - s.float()).numpy() > 1e5
        tf = tie_free_rows(bits(s), final.numpy(), ntxt, biased)
        out[f"{name}/q_pool"] = bits(qp)
        out[f"{name}/k_pool"] = bits(kp)
        out[f"{name}/indices"] = final.numpy().astype(np.int32)
        out[f"{name}/scores"] = bits(s)
        out[f"{name}/tie_free"] = tf
        print(f"{name}: indices {tuple(final.shape)}, tie-free rows {tf.mean():.3f}")
    np.savez_compressed(os.path.join(HERE, "mask_golden.npz"), **out)


if __name__ == "__main__":
    main()
