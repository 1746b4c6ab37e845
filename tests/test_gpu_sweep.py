"""Randomized-shape parity sweep of the device projections, attention and
Q8_0 GEMM (fixed seed, so every run draws the same cases).

The per-shape tests elsewhere pin the DA3 shapes and the tiling edges that
the kernels' own logic names; this sweep adds ragged sizes nobody picked by
hand (M, K, N from 1 to a few thousand, round, near-round and arbitrary),
so that a tile, split or tail choice taken only for some shape class is
exercised with its neighbours.  Bars:
- projections (linear_bias_scale_f32_da3_base's Store, the fused GELU and
  Residual epilogues, src/specialized.rs:811-929) against float64, within
  the f32 accumulation bound (K + 2) * 6e-8 * (|A||W| + |b|) per output, the
  epilogue's own roundings, and for GELU the fast form's 1e-6 * max(1, |v|)
  (the erf of the float64 reference is exact to double precision);
- DA3 flash attention against float64 softmax attention, 2e-5 * max |V|;
- the Q8_0 GEMM (Kernels::gemm_q8_0, src/dispatch.rs:91-105) bit for bit
  against the oracle, and the Q8_0 projections (bias, LayerScale, GELU,
  residual) bit for bit against the oracle's composition of the engine's
  passes;
- the elementwise and DPT operations at random sizes against the oracle:
  Kernels::gelu, the CPU-order LayerNorm, quantize_row_q8_0, 2-D RoPE with
  head dims 16 to 128 and the resizes bit for bit, the two-pass LayerNorm
  within 1e-5, convolutions (any kernel size, stride and padding) and
  transposed convolutions within twice the f32 accumulation bound of the
  direct definition, bit for bit where the gather form applies;
- the routes that read a CHW or K-major operand in place (channel counts
  that are multiples of 32): direct convolutions, including small grids
  whose K is split past four pieces, transposed convolutions with
  kernel == stride, and gemm_row_major_f32 at M, K <= 1024, against the
  same bounds.
"""
import numpy as np
import pytest
from scipy.special import erf

import oracle as O
from conftest import assert_bits_equal, max_rel
from q8_compose import q8_linear, weight_blocks
from vestra_hip import da3

pytestmark = pytest.mark.gpu

_RNG = np.random.default_rng(20261202)


def _dim(lo, hi):
    r = _RNG.random()
    if r < 0.3:
        return int(_RNG.integers(lo, hi + 1))
    if r < 0.6:
        return int(min(hi, max(lo, 32 * _RNG.integers(1, hi // 32 + 1))))
    return int(min(hi, max(lo, 16 * _RNG.integers(1, hi // 16 + 1) + _RNG.integers(-2, 3))))


PROJ_CASES = [(str(_RNG.choice(["store", "gelu", "residual"])), _dim(1, 2000), _dim(1, 1600),
               _dim(1, 2500), bool(_RNG.random() < 0.6), int(_RNG.integers(1, 1 << 30)))
              for _ in range(36)]
FLASH_CASES = [(int(_RNG.integers(1, 7)), _dim(1, 1800), bool(_RNG.random() < 0.5),
                int(_RNG.integers(1, 1 << 30))) for _ in range(14)]
Q8_LINEAR_CASES = [(str(_RNG.choice(["store", "gelu", "residual"])), _dim(1, 1500),
                    32 * int(_RNG.integers(1, 60)), _dim(1, 2000), bool(_RNG.random() < 0.5),
                    int(_RNG.integers(1, 1 << 30))) for _ in range(10)]
Q8_CASES = [(_dim(1, 2000), _dim(1, 2100), 32 * int(_RNG.integers(1, 80)),
             int(_RNG.integers(1, 1 << 30))) for _ in range(12)]
ELEMENTWISE_CASES = [(str(op), int(_RNG.integers(1, 1 << 30)))
                     for op in _RNG.permutation(["gelu", "layernorm", "quantize", "rope", "resize",
                                                 "conv", "conv_transpose"] * 3)]
IN_PLACE_CASES = [(str(op), int(_RNG.integers(1, 1 << 30)))
                  for op in _RNG.permutation(["conv", "conv_transpose", "row_major"] * 4)]


@pytest.mark.parametrize("mode, m, k, n, gamma, seed", PROJ_CASES)
def test_projection_random_shapes_vs_float64(rt, mode, m, k, n, gamma, seed):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal(m * k).astype(np.float32)
    w = (rng.standard_normal(k * n) * 0.05).astype(np.float32)
    b = (rng.standard_normal(n) * 0.1).astype(np.float32)
    g = (0.1 + rng.random(n)).astype(np.float32) if gamma and mode != "gelu" else None
    lin = rt.prepare_linear_f32(k, n, w, b, g)
    A, W = a.reshape(m, k).astype(np.float64), w.reshape(k, n).astype(np.float64)
    v = A @ W + b
    bv = (k + 2) * 6e-8 * (np.abs(A) @ np.abs(W) + np.abs(b)) + 1e-30
    gg = np.ones(n) if g is None else g.astype(np.float64)
    if mode == "store":
        got = rt.download_f32(lin.run(rt.upload_f32(a), m)).reshape(m, n)
        exp = v * gg
        bound = bv * gg + 6e-8 * np.abs(exp)
    elif mode == "gelu":
        got = rt.download_f32(lin.run_gelu(rt.upload_f32(a), m)).reshape(m, n)
        exp = 0.5 * v * (1 + erf(v / np.sqrt(2)))
        bound = 1.2 * bv + 2e-6 * np.maximum(1, np.abs(v))
    else:
        x = rng.standard_normal(m * n).astype(np.float32)
        xt = rt.upload_f32(x)
        lin.run_residual(rt.upload_f32(a), m, xt)
        got = rt.download_f32(xt).reshape(m, n)
        exp = x.reshape(m, n) + v * gg
        bound = bv * gg + 1.2e-7 * (np.abs(exp) + np.abs(x.reshape(m, n)))
    assert np.all(np.abs(got - exp) <= bound), float((np.abs(got - exp) / bound).max())


@pytest.mark.parametrize("heads, tokens, token_major, seed", FLASH_CASES)
def test_flash_random_shapes_vs_float64(rt, heads, tokens, token_major, seed):
    rng = np.random.default_rng(seed)
    q, k, v = (rng.standard_normal(heads * tokens * 64).astype(np.float32) for _ in range(3))
    got = rt.download_f32(rt.flash_attention_f32_da3_base(
        rt.upload_f32(q), rt.upload_f32(k), rt.upload_f32(v), heads, tokens, token_major))
    Q, K, V = (t.reshape(heads, tokens, 64).astype(np.float64) for t in (q, k, v))
    s = Q @ K.transpose(0, 2, 1) / 8.0
    p = np.exp(s - s.max(-1, keepdims=True))
    o = (p / p.sum(-1, keepdims=True)) @ V
    if token_major:
        o = o.transpose(1, 0, 2)
    assert np.abs(got - o.reshape(-1)).max() <= 2e-5 * np.abs(V).max()


@pytest.mark.parametrize("m, n, k, seed", Q8_CASES)
def test_gemm_q8_0_random_shapes_bit_exact(rt, m, n, k, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(m * k).astype(np.float32)
    w = (rng.standard_normal(n * k) * 0.02).astype(np.float32)
    exp = O.gemm_q8_0(O.quantize_rows_q8_0(x, m, k), O.quantize_rows_q8_0(w, n, k), m, n, k,
                      impl="kernels")
    got = rt.download_f32(rt.gemm_q8_0(rt.quantize_q8_0(rt.upload_f32(x), m, k),
                                       rt.quantize_q8_0(rt.upload_f32(w), n, k), m, n, k))
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


@pytest.mark.parametrize("mode, m, k, n, gamma, seed", Q8_LINEAR_CASES)
def test_q8_linear_random_shapes_bit_exact(rt, mode, m, k, n, gamma, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(m * k).astype(np.float32)
    w = (rng.standard_normal(k * n) * 0.02).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.02).astype(np.float32)
    g = (0.1 + rng.random(n)).astype(np.float32) if gamma and mode != "gelu" else None
    wb = weight_blocks(w, k, n)
    lin = rt.prepare_linear_q8_0(k, n, wb, bias, g)
    xt = rt.upload_f32(x)
    if mode == "residual":
        r = rng.standard_normal(m * n).astype(np.float32)
        rt_r = rt.upload_f32(r)
        lin.run_residual(xt, m, rt_r)
        got, exp = rt.download_f32(rt_r), q8_linear(x, m, k, n, wb, bias, g, "residual", r)
    else:
        got = rt.download_f32(lin.run_gelu(xt, m) if mode == "gelu" else lin.run(xt, m))
        exp = q8_linear(x, m, k, n, wb, bias, g, mode)
    assert_bits_equal(got, exp, f"Q8_0 linear {mode} {m}x{k}x{n}")


@pytest.mark.parametrize("op, seed", ELEMENTWISE_CASES)
def test_elementwise_random_shapes_vs_oracle(rt, op, seed):
    rng = np.random.default_rng(seed)
    if op == "gelu":
        n = int(rng.integers(1, 1_000_000))
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        t = rt.upload_f32(x)
        rt.gelu_f32_in_place(t)
        assert_bits_equal(rt.download_f32(t), O.kernels_gelu(x), f"gelu n={n}")
    elif op == "layernorm":
        rows, cols = int(rng.integers(1, 3000)), int(rng.integers(1, 2100))
        rows = max(1, min(rows, 3_000_000 // cols))
        x = (rng.standard_normal(rows * cols) * rng.uniform(0.1, 5) + rng.uniform(-3, 3)).astype(np.float32)
        g = (rng.standard_normal(cols) * 0.2 + 1).astype(np.float32)
        b = (rng.standard_normal(cols) * 0.1).astype(np.float32)
        exp = O.layernorm(x, rows, cols, g, b, 1e-6)
        xt, gt, bt = rt.upload_f32(x), rt.upload_f32(g), rt.upload_f32(b)
        assert max_rel(rt.download_f32(rt.layernorm_f32(xt, gt, bt, rows, cols, 1e-6)), exp) <= 1e-5
        assert_bits_equal(rt.download_f32(rt.layernorm_f32_cpu_order(xt, gt, bt, rows, cols, 1e-6)),
                          exp, f"cpu-order LayerNorm {rows}x{cols}")
    elif op == "quantize":
        rows, k = int(rng.integers(1, 5000)), 32 * int(rng.integers(1, 100))
        rows = max(1, min(rows, 4_000_000 // k))
        x = (rng.standard_normal(rows * k) * rng.uniform(0.001, 10)).astype(np.float32)
        got = rt.q8_0_download(rt.quantize_q8_0(rt.upload_f32(x), rows, k))
        assert np.array_equal(got.view(np.uint8), np.asarray(O.quantize_rows_q8_0(x, rows, k)).view(np.uint8))
    elif op == "rope":
        hd = int(rng.choice([16, 32, 64, 128]))
        heads, gh, gw = int(rng.integers(1, 16)), int(rng.integers(1, 50)), int(rng.integers(1, 50))
        n = gh * gw + 1
        x = rng.standard_normal(heads * n * hd).astype(np.float32)
        pos = da3.positions_yx(gh, gw)
        t = rt.upload_f32(x)
        rt.rope2d_f32_in_place(t, heads, n, hd, pos, 100.0)
        assert_bits_equal(rt.download_f32(t), O.rope2d(x, heads, n, hd, pos, 100.0), f"rope hd={hd}")
    elif op == "resize":
        c, ih, iw = int(rng.integers(1, 64)), int(rng.integers(1, 80)), int(rng.integers(1, 80))
        oh, ow = int(rng.integers(1, 200)), int(rng.integers(1, 200))
        x = rng.standard_normal(c * ih * iw).astype(np.float32)
        xt = rt.upload_f32(x)
        assert_bits_equal(rt.download_f32(rt.bilinear_resize_f32(xt, c, ih, iw, oh, ow)),
                          O.bilinear_resize(x, c, ih, iw, oh, ow), "half-pixel resize")
        assert_bits_equal(rt.download_f32(rt.bilinear_resize_align_corners_f32(xt, c, ih, iw, oh, ow)),
                          O.bilinear_resize_align_corners(x, c, ih, iw, oh, ow), "align-corners resize")
    elif op == "conv":
        in_c, out_c = int(rng.integers(1, 200)), int(rng.integers(1, 200))
        kk, s = int(rng.choice([1, 3, 5])), int(rng.choice([1, 1, 2]))
        p = int(rng.integers(0, kk // 2 + 2))
        ih, iw = int(rng.integers(kk, 60)), int(rng.integers(kk, 60))
        x = rng.standard_normal(in_c * ih * iw).astype(np.float32)
        w = (rng.standard_normal(out_c * in_c * kk * kk) / np.sqrt(in_c * kk * kk)).astype(np.float32)
        b = rng.standard_normal(out_c).astype(np.float32)
        got = rt.download_f32(rt.prepare_conv2d_f32(in_c, out_c, kk, kk, s, p, w, b).run(
            rt.upload_f32(x), ih, iw))
        exp = O.conv2d_naive(x, in_c, ih, iw, w, out_c, kk, kk, s, p, b)
        absb = O.conv2d_naive(np.abs(x), in_c, ih, iw, np.abs(w), out_c, kk, kk, s, p, np.abs(b))
        assert np.all(np.abs(got.astype(np.float64) - exp) <=
                      2 * (in_c * kk * kk + 2) * 6e-8 * absb.astype(np.float64) + 1e-30)
    else:
        in_c, out_c = int(rng.integers(1, 200)), int(rng.integers(1, 100))
        kk = int(rng.choice([2, 3, 4, 5]))
        s = int(rng.choice([kk, kk, 2, 3]))
        ih, iw = int(rng.integers(1, 30)), int(rng.integers(1, 30))
        x = rng.standard_normal(in_c * ih * iw).astype(np.float32)
        w = (rng.standard_normal(in_c * out_c * kk * kk) / np.sqrt(in_c)).astype(np.float32)
        b = rng.standard_normal(out_c).astype(np.float32)
        got = rt.download_f32(rt.conv_transpose2d_f32(rt.upload_f32(x), in_c, ih, iw, w, out_c, kk,
                                                      kk, s, b))
        exp = O.conv_transpose2d_naive(x, in_c, ih, iw, w, out_c, kk, kk, s, b)
        if s == kk:
            absb = O.conv_transpose2d_naive(np.abs(x), in_c, ih, iw, np.abs(w), out_c, kk, kk, s,
                                            np.abs(b))
            assert np.all(np.abs(got.astype(np.float64) - exp) <= 2 * (in_c + 2) * 6e-8 * absb + 1e-30)
        else:
            assert_bits_equal(got, exp, f"gather transposed conv k{kk} s{s}")


@pytest.mark.parametrize("op, seed", IN_PLACE_CASES)
def test_in_place_operand_routes_random_shapes(rt, op, seed):
    rng = np.random.default_rng(seed)
    if op == "conv":
        in_c, out_c = 32 * int(rng.integers(1, 25)), int(rng.integers(1, 200))
        kk, s = int(rng.choice([1, 3, 3, 5])), int(rng.choice([1, 1, 2]))
        p = int(rng.integers(0, kk // 2 + 2))
        ih, iw = int(rng.integers(kk, 40)), int(rng.integers(kk, 40))
        x = rng.standard_normal(in_c * ih * iw).astype(np.float32)
        w = (rng.standard_normal(out_c * in_c * kk * kk) / np.sqrt(in_c * kk * kk)).astype(np.float32)
        b = rng.standard_normal(out_c).astype(np.float32)
        got = rt.download_f32(rt.prepare_conv2d_f32(in_c, out_c, kk, kk, s, p, w, b).run(
            rt.upload_f32(x), ih, iw))
        exp = O.conv2d_naive(x, in_c, ih, iw, w, out_c, kk, kk, s, p, b)
        absb = O.conv2d_naive(np.abs(x), in_c, ih, iw, np.abs(w), out_c, kk, kk, s, p, np.abs(b))
        assert np.all(np.abs(got.astype(np.float64) - exp) <=
                      2 * (in_c * kk * kk + 2) * 6e-8 * absb.astype(np.float64) + 1e-30)
    elif op == "conv_transpose":
        in_c, out_c = 32 * int(rng.integers(1, 13)), int(rng.integers(1, 100))
        kk = int(rng.choice([2, 3, 4]))
        ih, iw = int(rng.integers(1, 30)), int(rng.integers(1, 30))
        x = rng.standard_normal(in_c * ih * iw).astype(np.float32)
        w = (rng.standard_normal(in_c * out_c * kk * kk) / np.sqrt(in_c)).astype(np.float32)
        b = rng.standard_normal(out_c).astype(np.float32)
        got = rt.download_f32(rt.conv_transpose2d_f32(rt.upload_f32(x), in_c, ih, iw, w, out_c, kk,
                                                      kk, kk, b))
        exp = O.conv_transpose2d_naive(x, in_c, ih, iw, w, out_c, kk, kk, kk, b)
        absb = O.conv_transpose2d_naive(np.abs(x), in_c, ih, iw, np.abs(w), out_c, kk, kk, kk,
                                        np.abs(b))
        assert np.all(np.abs(got.astype(np.float64) - exp) <= 2 * (in_c + 2) * 6e-8 * absb + 1e-30)
    else:
        m, k, n = _rand_dim(rng, 1, 1024), 32 * int(rng.integers(1, 33)), _rand_dim(rng, 1, 3000)
        a = rng.standard_normal(m * k).astype(np.float32)
        bm = (rng.standard_normal(k * n) * 0.05).astype(np.float32)
        got = rt.download_f32(rt.gemm_row_major_f32(rt.upload_f32(a), rt.upload_f32(bm), m, k, n))
        ref = a.reshape(m, k).astype(np.float64) @ bm.reshape(k, n).astype(np.float64)
        bound = (k + 2) * 6e-8 * (np.abs(a.reshape(m, k)).astype(np.float64) @ np.abs(bm.reshape(k, n)))
        assert np.all(np.abs(got.reshape(m, n) - ref) <= bound + 1e-30)


def _rand_dim(rng, lo, hi):
    return int(rng.integers(lo, hi + 1)) if rng.random() < 0.5 else int(min(hi, 32 * rng.integers(1, hi // 32 + 1)))
