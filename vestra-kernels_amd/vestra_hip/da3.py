"""DA3-BASE encoder shapes, RoPE positions and seeded block weights.

Shapes follow the reference's fixed DA3-BASE kernels: 768-wide tokens, 12
heads of 64, MLP 3072 (src/specialized.rs:770-806, 996-1027), 865 tokens for
a 504x336 image = 1 CLS + a 24 x 36 grid of 14-px patches
(src/specialized.rs:27-31).
"""
from __future__ import annotations

import numpy as np

from . import seeded

DIM = 768
HEADS = 12
HEAD_DIM = 64
MLP = 3072
QKV = 3 * DIM
PATCH = 14
ROPE_FREQ = 100.0
LN_EPS = 1e-6
LAYERSCALE = 1e-5

BLOCK_FIELDS = ("ln1_gamma", "ln1_beta", "w_qkv", "b_qkv", "w_proj", "b_proj", "ls1",
                "ln2_gamma", "ln2_beta", "w_fc1", "b_fc1", "w_fc2", "b_fc2", "ls2")
# DA3 late blocks only (Q/K LayerNorm before the RoPE); absent for plain blocks.
QK_NORM_FIELDS = ("q_norm_gamma", "q_norm_beta", "k_norm_gamma", "k_norm_beta")


def grid(height_px: int, width_px: int) -> tuple[int, int]:
    """(rows, cols) of the patch grid; 504x336 (W x H) gives 24 x 36."""
    return height_px // PATCH, width_px // PATCH


def tokens_for(height_px: int, width_px: int) -> int:
    rows, cols = grid(height_px, width_px)
    return rows * cols + 1


def positions_yx(rows: int, cols: int, special: int = 1) -> np.ndarray:
    """DA3 local RoPE layout (src/specialized.rs:359-366): special tokens at
    (0, 0), patch p at (p / cols + 1, p % cols + 1).  Returns int64 [tokens*2]."""
    n = rows * cols
    pos = np.zeros((special + n, 2), np.int64)
    p = np.arange(n)
    pos[special:, 0] = p // cols + 1
    pos[special:, 1] = p % cols + 1
    return pos.reshape(-1)


def positions_global(rows: int, cols: int, special: int = 1) -> np.ndarray:
    """DA3 global layout (src/specialized.rs:353-358): every patch at (1, 1)."""
    pos = np.zeros((special + rows * cols, 2), np.int64)
    pos[special:] = 1
    return pos.reshape(-1)


def block_weights(seed: int, layer: int = 0, layerscale: float | str = LAYERSCALE,
                  w_std: float = 0.02, b_std: float = 0.02,
                  qk_norm: bool = False, ln_affine: bool = False) -> dict[str, np.ndarray]:
    """Seeded block parameters: weights N(0, w_std^2) row-major [in, out],
    biases N(0, b_std^2), LayerNorm gamma=1 / beta=0, LayerScale constant,
    or, with layerscale="uniform", drawn per channel from U(0.1, 1) (large
    enough that every branch moves the residual stream well past f32
    rounding, so an encoder's output checks each layer's arithmetic).
    With qk_norm (DA3's late blocks) the 64-wide Q and K LayerNorms get
    gamma ~ 1 + N(0, 0.1^2) and beta ~ N(0, b_std^2).  With ln_affine the
    block's two LayerNorms get gamma ~ U(0.5, 1.5) and beta ~ N(0, 0.1^2)
    per channel instead of 1 and 0."""
    def n(tid, count, std):
        return seeded.normal(seeded.tensor_seed(seed, layer, tid), count, std)

    def ls(tid):
        if layerscale == "uniform":
            u = seeded.uniform01(seeded.tensor_seed(seed, layer, tid), DIM)
            return (0.1 + 0.9 * u).astype(np.float32)
        return np.full(DIM, layerscale, np.float32)

    extra = {}
    if qk_norm:
        extra = {
            "q_norm_gamma": (1.0 + n(9, HEAD_DIM, 0.1)).astype(np.float32),
            "q_norm_beta": n(10, HEAD_DIM, b_std),
            "k_norm_gamma": (1.0 + n(11, HEAD_DIM, 0.1)).astype(np.float32),
            "k_norm_beta": n(12, HEAD_DIM, b_std),
        }
    def ln(tid_g, tid_b):
        if not ln_affine:
            return np.ones(DIM, np.float32), np.zeros(DIM, np.float32)
        u = seeded.uniform01(seeded.tensor_seed(seed, layer, tid_g), DIM)
        return (0.5 + u).astype(np.float32), n(tid_b, DIM, 0.1)

    ln1_g, ln1_b = ln(13, 14)
    ln2_g, ln2_b = ln(15, 16)
    return extra | {
        "ln1_gamma": ln1_g,
        "ln1_beta": ln1_b,
        "w_qkv": n(1, DIM * QKV, w_std),
        "b_qkv": n(2, QKV, b_std),
        "w_proj": n(3, DIM * DIM, w_std),
        "b_proj": n(4, DIM, b_std),
        "ls1": ls(20),
        "ln2_gamma": ln2_g,
        "ln2_beta": ln2_b,
        "w_fc1": n(5, DIM * MLP, w_std),
        "b_fc1": n(6, MLP, b_std),
        "w_fc2": n(7, MLP * DIM, w_std),
        "b_fc2": n(8, DIM, b_std),
        "ls2": ls(21),
    }
