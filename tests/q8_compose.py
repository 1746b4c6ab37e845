"""Q8_0 projections and the Q8_0 block composed from the oracle's pinned
primitives (test helper, not a test module).

Each projection is quantize_row_q8_0 of the input rows and of the rows of W^T
(src/q8_0_dot.rs:27-46), Kernels::gemm_q8_0 (src/dispatch.rs:91-105), then
add_bias_rows (src/scalar.rs:65-81), layerscale (src/scalar.rs:139-155),
Kernels::gelu / Kernels::add (src/dispatch.rs:56-83) as separate f32 passes.
"""
import numpy as np

import oracle as O
from vestra_hip import da3


def weight_blocks(w, k, n):
    """W [k, n] row-major -> BlockQ8_0 rows of W^T (n rows of k/32 blocks)."""
    wt = np.ascontiguousarray(np.asarray(w, np.float32).reshape(k, n).T)
    return O.quantize_rows_q8_0(wt, n, k)


def q8_linear(x, rows, k, n, wblocks, bias=None, gamma=None, mode="store", residual=None):
    c = O.gemm_q8_0(O.quantize_rows_q8_0(x, rows, k), wblocks, rows, n, k, impl="kernels")
    if bias is not None:
        c = O.add_bias_rows(c, rows, n, bias)
    if mode == "gelu":
        return O.kernels_gelu(c)
    if gamma is not None:
        c = O.layerscale(c, rows, n, gamma)
    if mode == "residual":
        return O.kernels_add(residual, c)
    return c


def q8_block(x, w, T, pos=None, attention=O.attention, layernorm=O.layernorm,
             eps=da3.LN_EPS, freq=da3.ROPE_FREQ):
    """One image of the Q8_0 block.  attention(q, k, v, heads, T, 64) and
    layernorm(x, rows, cols, gamma, beta, eps) are pluggable, so a device test
    can feed the device's own values for the two steps whose rounding differs
    from the oracle's and check everything else bit for bit."""
    D, F, H = 768, 3072, 12
    x = np.asarray(x, np.float32)
    h = layernorm(x, T, D, w["ln1_gamma"], w["ln1_beta"], eps)
    qkv = q8_linear(h, T, D, 3 * D, weight_blocks(w["w_qkv"], D, 3 * D), w["b_qkv"])
    q, k, v = O.split_qkv_hnd(qkv, T, H, 64)
    if w.get("q_norm_gamma") is not None:
        p = pos if pos is not None else np.zeros((T, 2), np.int64)
        q, k = O.qk_norm_rope(q, k, H, T, w["q_norm_gamma"], w["q_norm_beta"],
                              w["k_norm_gamma"], w["k_norm_beta"], p, freq, eps)
    elif pos is not None:
        q = O.rope2d(q, H, T, 64, pos, freq)
        k = O.rope2d(k, H, T, 64, pos, freq)
    att = O.hnd_to_token(attention(q, k, v, H, T, 64), T, H, 64)
    x = q8_linear(att, T, D, D, weight_blocks(w["w_proj"], D, D), w["b_proj"], w["ls1"],
                  "residual", x)
    h = layernorm(x, T, D, w["ln2_gamma"], w["ln2_beta"], eps)
    f = q8_linear(h, T, D, F, weight_blocks(w["w_fc1"], D, F), w["b_fc1"], mode="gelu")
    return q8_linear(f, T, F, D, weight_blocks(w["w_fc2"], F, D), w["b_fc2"], w["ls2"],
                     "residual", x)


def exact_int_blocks(seed, rows, k, exps=(0, 1)):
    """Rows whose every 32-block quantises losslessly: small integers in
    [-8, 8] times 2^e, with one element at +-127 * 2^e, so d = 2^e exactly,
    1/d is exact and q = x / d.  With k <= 768 every product and partial sum
    of the Q8_0 GEMM is an integer multiple of 2^(2 min e) below 2^24, so the
    GEMM must equal the exact matrix product."""
    rng = np.random.default_rng(seed)
    nb = k // 32
    v = rng.integers(-8, 9, size=(rows, nb, 32)).astype(np.float64)
    pos = rng.integers(0, 32, size=(rows, nb))
    sign = np.where(rng.integers(0, 2, size=(rows, nb)) == 0, -1.0, 1.0)
    np.put_along_axis(v, pos[..., None], (127.0 * sign)[..., None], axis=2)
    e = rng.choice(np.asarray(exps), size=(rows, nb))
    return (v * np.exp2(e)[..., None]).reshape(rows, k).astype(np.float32)
