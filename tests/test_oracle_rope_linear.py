"""Pins the oracle's RoPE (src/rope.rs, src/specialized.rs:273-454) and
projection (src/specialized.rs:770-1300) restatements."""
import numpy as np
import pytest

import oracle as O
from vestra_hip import da3, seeded


# ---- RoPE ---------------------------------------------------------------------

def _rope64(x, heads, n, hd, pos, freq):
    """float64 2-D rotate-half RoPE from the module doc (src/rope.rs:1-20)."""
    x = x.reshape(heads, n, hd).astype(np.float64).copy()
    half, quarter = hd // 2, hd // 4
    i = np.arange(quarter)
    theta = np.float32(freq) ** (-2.0 * i / half)
    for axis in range(2):
        p = pos.reshape(n, 2)[:, axis].astype(np.float64)[:, None] * theta[None, :]
        s, c = np.sin(p), np.cos(p)
        a = x[:, :, axis * half: axis * half + quarter].copy()
        b = x[:, :, axis * half + quarter: (axis + 1) * half].copy()
        x[:, :, axis * half: axis * half + quarter] = a * c - b * s
        x[:, :, axis * half + quarter: (axis + 1) * half] = b * c + a * s
    return x.reshape(-1)


def test_rope2d_matches_float64_rotation_small_case():
    """src/rope.rs:133-154 inputs: heads 3, n 7, head_dim 16, positions (i, 3i)."""
    heads, n, hd = 3, 7, 16
    x = ((np.arange(heads * n * hd, dtype=np.float32) - 43.0) * 0.0625).astype(np.float32)
    pos = np.array([[i, 3 * i] for i in range(n)], np.int64).reshape(-1)
    got = O.rope2d(x, heads, n, hd, pos, 100.0)
    ref = _rope64(x, heads, n, hd, pos, 100.0)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-6
    # rotations preserve each pair's norm
    g = got.reshape(heads, n, 2, 2, 4).astype(np.float64)
    xx = x.reshape(heads, n, 2, 2, 4).astype(np.float64)
    assert np.allclose((g ** 2).sum(3), (xx ** 2).sum(3), rtol=1e-5)


def test_rope_cls_identity_and_da3_layout():
    pos = da3.positions_yx(24, 36)
    assert pos[:2].tolist() == [0, 0]
    assert pos[2:6].tolist() == [1, 1, 1, 2]           # patch 0 -> (1,1), patch 1 -> (1,2)
    assert pos[-2:].tolist() == [24, 36]               # last patch -> (24, 36)
    x = seeded.normal(9, 12 * 865 * 64)
    got = O.rope2d(x, 12, 865, 64, pos, 100.0).reshape(12, 865, 64)
    assert np.array_equal(got[:, 0], x.reshape(12, 865, 64)[:, 0])  # CLS at angle 0
    assert np.abs(got.reshape(-1) - _rope64(x, 12, 865, 64, pos, 100.0)).max() < 2e-5
    g = da3.positions_global(24, 36)
    assert g[:2].tolist() == [0, 0] and set(g[2:].tolist()) == {1}


def test_rope_table_matches_float64_and_rope2d():
    pos = da3.positions_yx(24, 36)
    rot = O.rope_rotations(pos, 865, 100.0).reshape(865, 2, 16, 2)
    inv = np.array([np.float32(100.0) ** np.float32(-2.0 * i / 32.0) for i in range(16)], np.float64)
    ang = pos.reshape(865, 2).astype(np.float64)[:, :, None] * inv[None, None, :]
    assert np.abs(rot[..., 0] - np.sin(ang)).max() < 2e-6
    assert np.abs(rot[..., 1] - np.cos(ang)).max() < 2e-6


def test_fused_qk_norm_rope_equals_separate_bitwise():
    """src/specialized.rs:3403-3441 inputs: fused LN+RoPE == LN then RoPE."""
    H, T, Dm = 12, 865, 64
    src = np.array([((i * 31 % 997) - 498.0) * 0.001 for i in range(H * T * Dm)], np.float32)
    gamma = np.array([0.8 + i * 0.003 for i in range(Dm)], np.float32)
    beta = np.array([-0.1 + i * 0.002 for i in range(Dm)], np.float32)
    pos = np.array([[i // 24, i % 24] for i in range(T)], np.int64).reshape(-1)
    fq, fk = O.qk_norm_rope(src, src, H, T, gamma, beta, gamma, beta, pos, 100.0, 1e-5)
    sep = O.rope2d(O.layernorm(src, H * T, Dm, gamma, beta, 1e-5), H, T, Dm, pos, 100.0)
    assert np.array_equal(fq.view(np.uint32), sep.view(np.uint32))
    assert np.array_equal(fk.view(np.uint32), sep.view(np.uint32))


# ---- projections -------------------------------------------------------------

def test_linear_kats():
    """src/cuda.rs:1405-1452: product, bias-scale and chained linear answers."""
    left = [1, 2, 3, 4, 5, 6]
    w1 = [7, 8, 9, 10, 11, 12]
    assert O.linear(left, w1, 2, 2, 3).tolist() == [58, 64, 139, 154]
    first = O.linear_bias_scale(left, w1, [1.0, -4.0], [0.5, 2.0], 2, 2, 3)
    assert first.tolist() == [29.5, 120.0, 70.0, 300.0]
    second = O.linear_bias_scale(first, [2.0, -1.0], [3.0], [1.0], 2, 1, 2)
    assert second.tolist() == [-58.0, -157.0]


@pytest.mark.skipif(not O.has_avx512(), reason="host without AVX-512")
def test_avx512_tiles_equal_fma_chain_bitwise():
    """src/specialized.rs:3300-3331 inputs: every tiling keeps the ascending-K
    FMA chain, so the 6x64 AVX-512 tiles equal the scalar fmaf chain."""
    m, n, k = 865, 768, 768
    a = np.sin(np.arange(m * k, dtype=np.float32) * np.float32(0.013)).astype(np.float32)
    b = np.cos(np.arange(k * n, dtype=np.float32) * np.float32(0.007)).astype(np.float32)
    assert np.array_equal(O.linear(a, b, m, n, k).view(np.uint32),
                          O.linear_fma_scalar(a, b, m, n, k).view(np.uint32))


def test_bias_scale_and_qkv_epilogues_bitwise():
    """src/specialized.rs:3334-3400: (acc+bias)*scale, and the head-major QKV
    equals linear + bias + split (bit for bit)."""
    m = 37
    rng = np.random.default_rng(4)
    a = rng.standard_normal(m * 768).astype(np.float32)
    w = (rng.standard_normal(768 * 2304) * 0.02).astype(np.float32)
    bias = (rng.standard_normal(2304) * 0.02).astype(np.float32)
    acc = O.linear_fma_scalar(a, w, m, 2304, 768)
    tm = (acc.reshape(m, 2304) + bias).reshape(-1)
    eq, ek, ev = O.split_qkv_hnd(tm, m, 12, 64)
    q, k, v = O.qkv(a, w, bias, m)
    for got, exp in ((q, eq), (k, ek), (v, ev)):
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
    scale = (0.75 + np.cos(np.arange(2304) * 0.011)).astype(np.float32)
    bs = O.linear_bias_scale(a, w, bias, scale, m, 2304, 768)
    assert np.array_equal(bs.view(np.uint32), ((acc.reshape(m, 2304) + bias) * scale).reshape(-1).view(np.uint32))


def test_linear_matches_float64_and_scalar_gemm_agrees():
    """tests/gemm_backends_agree.rs:15-30 shape and tolerance (LCG inputs):
    the FMA-chain projection and scalar::gemm_f32 agree to 1e-3 + 1e-3|c|."""
    def lcg(n, seed):
        s, out = seed, []
        for _ in range(n):
            s = (s * 6364136223846793005 + 1) & 0xFFFFFFFFFFFFFFFF
            out.append(np.float32(np.float32(s >> 33) / np.float32(4294967295.0)) - np.float32(0.5))
        return np.array(out, np.float32)

    m, n, k = 64, 48, 80
    a, b = lcg(m * k, 1), lcg(k * n, 2)
    cs = O.gemm_f32(a, b, m, n, k)
    cf = O.linear(a, b, m, n, k)
    assert np.all(np.abs(cs - cf) <= 1e-3 + 1e-3 * np.abs(cs))
    ref = a.reshape(m, k).astype(np.float64) @ b.reshape(k, n).astype(np.float64)
    assert np.abs(cf.reshape(m, n) - ref).max() < 1e-5
