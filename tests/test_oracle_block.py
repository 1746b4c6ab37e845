"""Pins the oracle's DA3-BASE block composition against an independent
float64 transcription of the pre-LN ViT block: LN ->
QKV (+bias) -> [late blocks: LayerNorm of each 64-wide Q/K head row] ->
2-D RoPE on Q, K -> softmax(QK^T/8)V -> out-proj (+bias) * LayerScale +
residual -> LN -> fc1 (+bias) -> exact-erf GELU -> fc2 (+bias) * LayerScale
+ residual.  A wrong head split, RoPE axis, missing bias or misplaced
LayerScale shows up far above the float32 noise here."""
import math

import numpy as np
import pytest

import oracle as O
from vestra_hip import da3, seeded

_erf = np.vectorize(math.erf)


def block64(x, w, T, pos, eps=1e-6, freq=100.0):
    D, H = 768, 12
    f = {k: np.asarray(v, np.float64) for k, v in w.items()}
    x = np.asarray(x, np.float64).reshape(T, D)

    def ln(z, g, b):
        mu = z.mean(1, keepdims=True)
        return (z - mu) / np.sqrt(((z - mu) ** 2).mean(1, keepdims=True) + eps) * g + b

    h = ln(x, f["ln1_gamma"], f["ln1_beta"])
    qkv = h @ f["w_qkv"].reshape(D, 3 * D) + f["b_qkv"]
    q, k, v = (qkv[:, i * D:(i + 1) * D].reshape(T, H, 64).transpose(1, 0, 2) for i in range(3))
    if "q_norm_gamma" in f:  # DA3 late block: LayerNorm of each 64-wide head row
        q = ln(q.reshape(-1, 64), f["q_norm_gamma"], f["q_norm_beta"]).reshape(H, T, 64)
        k = ln(k.reshape(-1, 64), f["k_norm_gamma"], f["k_norm_beta"]).reshape(H, T, 64)
    if pos is not None:
        theta = np.float32(freq) ** (-2.0 * np.arange(16) / 32.0)
        p = pos.reshape(T, 2).astype(np.float64)

        def rope(z):
            z = z.copy()
            for ax in range(2):
                ang = p[:, ax][:, None] * theta[None, :]
                s, c = np.sin(ang), np.cos(ang)
                a = z[:, :, ax * 32:ax * 32 + 16].copy()
                b = z[:, :, ax * 32 + 16:ax * 32 + 32].copy()
                z[:, :, ax * 32:ax * 32 + 16] = a * c - b * s
                z[:, :, ax * 32 + 16:ax * 32 + 32] = b * c + a * s
            return z

        q, k = rope(q), rope(k)
    s = q @ k.transpose(0, 2, 1) / 8.0
    pr = np.exp(s - s.max(-1, keepdims=True))
    att = (pr / pr.sum(-1, keepdims=True)) @ v
    att = att.transpose(1, 0, 2).reshape(T, D)
    x = x + (att @ f["w_proj"].reshape(D, D) + f["b_proj"]) * f["ls1"]
    h = ln(x, f["ln2_gamma"], f["ln2_beta"])
    m = h @ f["w_fc1"].reshape(D, 3072) + f["b_fc1"]
    m = 0.5 * m * (1 + _erf(m / math.sqrt(2)))
    x = x + (m @ f["w_fc2"].reshape(3072, D) + f["b_fc2"]) * f["ls2"]
    return x.reshape(-1), att.reshape(-1)


@pytest.mark.parametrize("rows,cols,rope", [(3, 4, True), (2, 5, False)])
def test_block_matches_float64_transcription(rows, cols, rope):
    T = rows * cols + 1
    w = da3.block_weights(seed=11, layerscale=1.0)
    x = seeded.normal(12, T * 768)
    pos = da3.positions_yx(rows, cols) if rope else None
    got, taps = O.vit_block(x, w, 1, T, pos, taps=True)
    ref, ref_att = block64(x, w, T, pos)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-5
    assert np.abs(taps["attn"] - ref_att).max() / np.abs(ref_att).max() < 1e-5


def test_block_da3_shape_flash_path_matches_float64():
    """865 tokens takes the DA3 flash path inside the oracle block."""
    T = 865
    w = da3.block_weights(seed=13, layerscale=1.0)
    x = seeded.normal(14, T * 768)
    pos = da3.positions_yx(24, 36)
    got = O.vit_block(x, w, 1, T, pos)
    ref, _ = block64(x, w, T, pos)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-5


def test_block_images_are_independent():
    T = 7
    w = da3.block_weights(seed=15)
    x = seeded.normal(16, 2 * T * 768)
    pos = da3.positions_yx(2, 3)
    both = O.vit_block(x, w, 2, T, pos)
    one = O.vit_block(x[T * 768:], w, 1, T, pos)
    assert np.array_equal(both[T * 768:], one)


def test_layerscale_1e5_keeps_residual_near_identity():
    T = 7
    w = da3.block_weights(seed=17)
    x = seeded.normal(18, T * 768)
    y = O.vit_block(x, w, 1, T, da3.positions_yx(2, 3))
    assert 0 < np.abs(y - x).max() < 1e-3


@pytest.mark.parametrize("layout", ["local", "global", "none"])
def test_late_block_qk_norm_matches_float64_transcription(layout):
    """DA3 late blocks (src/specialized.rs:278-316): Q/K LayerNorm before the
    RoPE, with the local layout, the global layout (every patch at (1, 1),
    src/specialized.rs:353-358) and without positions."""
    rows, cols = 3, 4
    T = rows * cols + 1
    w = da3.block_weights(seed=19, layerscale=1.0, qk_norm=True)
    x = seeded.normal(20, T * 768)
    pos = {"local": da3.positions_yx(rows, cols), "global": da3.positions_global(rows, cols),
           "none": None}[layout]
    got, taps = O.vit_block(x, w, 1, T, pos, taps=True)
    ref, ref_att = block64(x, w, T, pos)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-5
    assert np.abs(taps["attn"] - ref_att).max() / np.abs(ref_att).max() < 1e-5
    plain = O.vit_block(x, {k: v for k, v in w.items() if "norm" not in k or "ln" in k}, 1, T, pos)
    assert np.abs(plain - got).max() > 1e-3  # the norm is really applied
