"""GPU parity of the DA3-BASE encoder block and the 12-layer encoder.

Bars: max relative error (max|gpu-cpu| / max|cpu|)
<= 1e-4 per block and <= 1e-3 after the full 12-layer encoder, in f32.
LayerScale 1e-5 makes the block output nearly the input, so the branch
outputs (attention, MLP hidden) are also checked before LayerScale, and a
LayerScale-1 variant checks the residual stream where branches dominate.
"""
import numpy as np
import pytest

import oracle as O
from conftest import max_rel
import vestra_hip as vh
from vestra_hip import da3, seeded

pytestmark = pytest.mark.gpu

BLOCK_TOL = 1e-4
ENCODER_TOL = 1e-3


def _branch(x_out, x_in):
    return np.asarray(x_out, np.float64) - np.asarray(x_in, np.float64)


@pytest.mark.parametrize("layerscale", [da3.LAYERSCALE, 1.0])
def test_block_config3_vs_oracle(rt, layerscale):
    T = 865
    w = da3.block_weights(seed=3, layer=0, layerscale=layerscale)
    x = seeded.normal(300, T * 768)
    pos = da3.positions_yx(24, 36)
    exp = O.vit_block(x, w, 1, T, pos)
    blk = rt.prepare_block(w)
    xt = rt.upload_f32(x)
    rt.vit_block_run(blk, xt, 1, T, pos)
    got = rt.download_f32(xt)
    assert max_rel(got, exp) <= BLOCK_TOL
    if layerscale == 1.0:
        # With unit LayerScale the branches dominate the residual stream, so
        # the block output is a direct check of attention and MLP arithmetic.
        assert max_rel(_branch(got, x), _branch(exp, x)) <= BLOCK_TOL * 10


def test_block_batch_images_match_single_image_runs(rt):
    """Images of a batch are independent: the batched launch matches the
    per-image oracle and a per-image GPU run (tile and split choices depend on
    the batch, so the summation order and hence the last bits may differ)."""
    T, B = 865, 2
    w = da3.block_weights(seed=4)
    x = seeded.normal(400, B * T * 768)
    pos = da3.positions_yx(24, 36)
    exp = O.vit_block(x, w, B, T, pos)
    blk = rt.prepare_block(w)
    xt = rt.upload_f32(x)
    rt.vit_block_run(blk, xt, B, T, pos)
    got = rt.download_f32(xt)
    assert max_rel(got, exp) <= BLOCK_TOL
    single = rt.upload_f32(x[T * 768:])
    rt.vit_block_run(blk, single, 1, T, pos)
    assert max_rel(rt.download_f32(single), got[T * 768:]) <= 1e-6


def test_block_no_rope_and_odd_tokens(rt):
    T = 97
    w = da3.block_weights(seed=5, layerscale=1.0)
    x = seeded.normal(500, T * 768)
    exp = O.vit_block(x, w, 1, T, None)
    blk = rt.prepare_block(w)
    xt = rt.upload_f32(x)
    rt.vit_block_run(blk, xt, 1, T, None)
    assert max_rel(rt.download_f32(xt), exp) <= BLOCK_TOL


def _encoder_case(rt, images, rows, cols, layers):
    T = rows * cols + 1
    ws = [da3.block_weights(seed=7, layer=l) for l in range(layers)]
    x = seeded.normal(700 + images, images * T * 768)
    pos = da3.positions_yx(rows, cols)
    exp = O.encoder(x, ws, images, T, pos)
    blocks = [rt.prepare_block(w) for w in ws]
    xt = rt.upload_f32(x)
    rt.encoder_run(blocks, xt, images, T, pos)
    got = rt.download_f32(xt)
    return got, exp, x


def test_encoder_config5a_batch4_12_layers(rt):
    got, exp, x = _encoder_case(rt, images=4, rows=24, cols=36, layers=12)
    assert max_rel(got, exp) <= ENCODER_TOL


def test_encoder_config5b_long_sequence_12_layers(rt):
    """1008x672 -> 48 x 72 grid + CLS = 3457 tokens (the CPU oracle takes the
    crate's generic attention path, not the 865-token flash gate), the full
    12 layers of BASELINE config 5 (about 1 s of oracle time per layer)."""
    got, exp, x = _encoder_case(rt, images=1, rows=48, cols=72, layers=12)
    assert max_rel(got, exp) <= ENCODER_TOL


@pytest.mark.parametrize("images, T", [(1, 865), (2, 97)])
def test_encoder_fused_norms_match_block_by_block_runs(rt, images, T):
    """Inside the encoder each fc2 reduction also writes the next layer's
    LayerNorm1 input; block by block, a separate LayerNorm kernel does.  Both
    round every element the same way, so three layers agree bit for bit."""
    ws = [da3.block_weights(seed=9, layer=l, layerscale=0.5) for l in range(3)]
    x = seeded.normal(900 + T, images * T * 768)
    pos = da3.positions_yx(24, 36) if T == 865 else None
    blocks = [rt.prepare_block(w) for w in ws]
    fused = rt.upload_f32(x)
    rt.encoder_run(blocks, fused, images, T, pos)
    step = rt.upload_f32(x)
    for b in blocks:
        rt.vit_block_run(b, step, images, T, pos)
    a, b = rt.download_f32(fused), rt.download_f32(step)
    assert np.isfinite(a).all()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("layout, T", [("local", 865), ("global", 865), ("none", 97)])
def test_late_block_qk_norm_vs_oracle(rt, layout, T):
    """DA3 late blocks: each 64-wide Q and K head row is LayerNormed before the
    RoPE (src/specialized.rs:278-316); the global layout puts every patch at
    (1, 1) (src/specialized.rs:353-358)."""
    w = da3.block_weights(seed=21, layerscale=1.0, qk_norm=True)
    x = seeded.normal(2100 + T, T * 768)
    pos = {"local": da3.positions_yx(24, 36), "global": da3.positions_global(24, 36),
           "none": None}[layout]
    exp = O.vit_block(x, w, 1, T, pos)
    blk = rt.prepare_block(w)
    xt = rt.upload_f32(x)
    rt.vit_block_run(blk, xt, 1, T, pos)
    got = rt.download_f32(xt)
    assert max_rel(_branch(got, x), _branch(exp, x)) <= BLOCK_TOL * 10
    assert max_rel(got, exp) <= BLOCK_TOL


def test_encoder_with_late_blocks_vs_oracle(rt):
    """Four layers, the last two DA3 late blocks (Q/K LayerNorm), 2 images."""
    T, layers, images = 865, 4, 2
    ws = [da3.block_weights(seed=23, layer=l, qk_norm=l >= 2) for l in range(layers)]
    x = seeded.normal(2300, images * T * 768)
    pos = da3.positions_yx(24, 36)
    exp = O.encoder(x, ws, images, T, pos)
    blocks = [rt.prepare_block(w) for w in ws]
    fused = rt.upload_f32(x)
    rt.encoder_run(blocks, fused, images, T, pos)
    got = rt.download_f32(fused)
    assert max_rel(got, exp) <= ENCODER_TOL
    step = rt.upload_f32(x)
    for b in blocks:
        rt.vit_block_run(b, step, images, T, pos)
    assert np.array_equal(got.view(np.uint32), rt.download_f32(step).view(np.uint32))


def test_late_block_needs_all_four_qk_norm_vectors(rt):
    w = da3.block_weights(seed=25, qk_norm=True)
    del w["k_norm_beta"]
    with pytest.raises(vh.InvalidArgument):
        rt.prepare_block(w)


def test_empty_inputs_are_no_ops(rt):
    """Zero tokens or images: the block, the encoder and the Q8_0 block return
    without launching; zero layers leave x unchanged."""
    w = da3.block_weights(seed=27)
    blk, qblk = rt.prepare_block(w), rt.prepare_block(w, q8_0=True)
    empty = rt.upload_f32(np.zeros(0, np.float32))
    rt.vit_block_run(blk, empty, 1, 0)
    rt.vit_block_run(qblk, empty, 0, 865)
    rt.encoder_run([blk, qblk], empty, 2, 0)
    x = seeded.normal(2700, 97 * 768)
    xt = rt.upload_f32(x)
    rt.encoder_run([], xt, 1, 97)
    assert np.array_equal(rt.download_f32(xt), x)
    with pytest.raises(vh.LengthMismatch):
        rt.vit_block_run(blk, xt, 1, 98)
