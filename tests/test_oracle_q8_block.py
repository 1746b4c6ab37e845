"""CPU checks of the Q8_0 projection and Q8_0 block oracle.

- the C oracle's Q8_0 block (vko_vit_block_q8_0) equals the composition of
  the separately pinned primitives (quantize_row_q8_0, Kernels::gemm_q8_0,
  add_bias_rows, layerscale, Kernels::gelu/add, LayerNorm, RoPE, attention)
  bit for bit, for plain, late (Q/K LayerNorm) and position-free blocks;
- a Q8_0 projection on losslessly quantisable operands equals the exact
  integer matrix product (closed form), which fixes the W^T orientation and
  the per-block scale indexing;
- the Q8_0 block stays near the f32 block (quantisation noise only).
"""
import numpy as np
import pytest

import oracle as O
from conftest import max_rel
from q8_compose import exact_int_blocks, q8_block, q8_linear, weight_blocks
from vestra_hip import da3, seeded


@pytest.mark.parametrize("T, layout, qk_norm", [(865, "local", False), (97, "none", False),
                                                (865, "global", True)])
def test_c_q8_block_equals_primitive_composition(T, layout, qk_norm):
    w = da3.block_weights(seed=31, layerscale=0.5, qk_norm=qk_norm)
    x = seeded.normal(3100 + T, T * 768)
    pos = {"local": da3.positions_yx(24, 36), "global": da3.positions_global(24, 36),
           "none": None}[layout]
    got = O.vit_block(x, w, 1, T, pos, q8_0=True)
    exp = q8_block(x, w, T, pos)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_c_q8_block_batches_images_independently():
    T = 97
    w = da3.block_weights(seed=32)
    x = seeded.normal(3200, 2 * T * 768)
    got = O.vit_block(x, w, 2, T, None, q8_0=True)
    for i in range(2):
        one = q8_block(x[i * T * 768:(i + 1) * T * 768], w, T)
        assert np.array_equal(got[i * T * 768:(i + 1) * T * 768].view(np.uint32),
                              one.view(np.uint32))


@pytest.mark.parametrize("rows, k, n", [(37, 768, 96), (5, 64, 33), (9, 64, 64)])
def test_q8_linear_exact_on_lossless_operands(rows, k, n):
    a = exact_int_blocks(1, rows, k)
    wt = exact_int_blocks(2, n, k)                     # rows of W^T
    w = np.ascontiguousarray(wt.T)                     # W [k, n]
    bias = np.arange(n, dtype=np.float32) * 0.5
    got = q8_linear(a, rows, k, n, weight_blocks(w, k, n), bias).reshape(rows, n)
    exact = a.astype(np.float64) @ w.astype(np.float64)
    assert np.abs(exact).max() < 2 ** 24
    assert np.array_equal(got, (exact.astype(np.float32) + bias).astype(np.float32))
    if n == k:
        # Quantising the rows of W instead of W^T gives another product.
        wrong = q8_linear(a, rows, k, n, weight_blocks(wt, k, n), bias).reshape(rows, n)
        assert not np.array_equal(wrong, got)


def test_q8_block_close_to_f32_block():
    """Q8_0 keeps about 7 bits per value; with unit LayerScale the branch
    outputs stay within a few percent of the f32 block's, and with DA3's
    LayerScale the residual stream barely moves."""
    T = 865
    pos = da3.positions_yx(24, 36)
    x = seeded.normal(3300, T * 768)
    for ls, tol in ((1.0, 5e-2), (da3.LAYERSCALE, 1e-6)):
        w = da3.block_weights(seed=33, layerscale=ls)
        q = O.vit_block(x, w, 1, T, pos, q8_0=True)
        f = O.vit_block(x, w, 1, T, pos)
        br = lambda a: np.asarray(a, np.float64) - x
        err = max_rel(br(q), br(f)) if ls == 1.0 else max_rel(q, f)
        assert err <= tol, (ls, err)
        assert err > 0
