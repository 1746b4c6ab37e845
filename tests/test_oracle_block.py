"""Pins the oracle's DA3-BASE block composition against an independent
float64 transcription of the pre-LN ViT block: LN ->
QKV (+bias) -> [late blocks: LayerNorm of each 64-wide Q/K head row] ->
2-D RoPE on Q, K -> softmax(QK^T/8)V -> out-proj (+bias) * LayerScale +
residual -> LN -> fc1 (+bias) -> exact-erf GELU -> fc2 (+bias) * LayerScale
+ residual.  A wrong head split, RoPE axis, missing bias or misplaced
LayerScale shows up far above the float32 noise here."""
import numpy as np
import pytest

import oracle as O
from block64 import block64
from vestra_hip import da3, seeded


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
