"""Pins the oracle's Q8_0 restatement (src/q8_0_dot.rs:27-46,
src/scalar.rs:25-56, src/simd_avx512.rs:262-351, src/lib.rs:42-50) and the
f16 conversions (half 2.7.1 from_f32 / to_f32, IEEE round-to-nearest-even).
"""
import numpy as np
import pytest

import oracle as O


def test_f16_conversions_match_f16c_on_every_input():
    """Every f32 bit pattern through the software RNE conversion equals F16C
    vcvtps2ph (imm 0), and every f16 widens as vcvtph2ps does."""
    assert O.f16_sweep(1) == 0


def test_f16_known_values():
    assert O.f32_to_f16(1.0) == 0x3C00 and O.f32_to_f16(-2.0) == 0xC000
    assert O.f32_to_f16(65504.0) == 0x7BFF and O.f32_to_f16(65520.0) == 0x7C00  # ties to inf
    assert O.f32_to_f16(2.0 ** -24) == 0x0001 and O.f32_to_f16(2.0 ** -25) == 0x0000  # tie-even
    assert O.f16_to_f32(0x3555) == np.float32(0.33325195)


def test_q8_0_gemm_close_to_f32():
    """tests/q8_0_dot_matches_f32.rs:23-62 with its exact inputs and tolerance."""
    m, n, k = 8, 8, 64
    a = np.array([((i % 17) - 8.0) * 0.1 for i in range(m * k)], np.float32)
    b = np.array([((i % 13) - 6.0) * 0.1 for i in range(k * n)], np.float32)
    bt = b.reshape(k, n).T.copy().reshape(-1)
    aq, bq = O.quantize_rows_q8_0(a, m, k), O.quantize_rows_q8_0(bt, n, k)
    c = O.gemm_q8_0(aq, bq, m, n, k, impl="kernels")
    a_de = O.dequantize_q8_0(aq)
    b_de = O.dequantize_q8_0(bq).reshape(n, k).T.copy().reshape(-1)
    c_ref = O.gemm_f32(a_de, b_de, m, n, k)
    assert np.all(np.abs(c - c_ref) < 1e-2 + 1e-2 * np.abs(c_ref))


@pytest.mark.skipif(not O.has_avx512(), reason="host without AVX-512 VNNI")
@pytest.mark.parametrize("m,n,k", [(37, 53, 96), (4, 9, 32), (16, 16, 768)])
def test_vnni_equals_scalar_bitwise(m, n, k):
    """The reference's VNNI kernel keeps the scalar acc += (da*db)*isum order
    (src/simd_avx512.rs:334-345 vs src/scalar.rs:51); odd block counts hit the
    scalar tail block."""
    rng = np.random.default_rng(m * n)
    aq = O.quantize_rows_q8_0(rng.standard_normal(m * k).astype(np.float32), m, k)
    bq = O.quantize_rows_q8_0((rng.standard_normal(n * k) * 0.02).astype(np.float32), n, k)
    s = O.gemm_q8_0(aq, bq, m, n, k, impl="scalar")
    v = O.gemm_q8_0(aq, bq, m, n, k, impl="avx512")
    assert np.array_equal(s.view(np.uint32), v.view(np.uint32))


def test_quantize_known_answers():
    # amax 127 -> d = 1 exactly, q = x.
    x = np.array([127, -127] + list(range(-15, 15)), np.float32)
    blk = O.quantize_rows_q8_0(x, 1, 32)[0]
    assert blk["d"] == 0x3C00 and blk["qs"].tolist() == x.astype(int).tolist()
    # amax 254 -> d = 2: halves round away from zero (f32::round), not to even.
    x = np.array([254, 5, -5, 3, -3, 1, -1, 7] + [0] * 24, np.float32)
    blk = O.quantize_rows_q8_0(x, 1, 32)[0]
    assert blk["d"] == 0x4000
    assert blk["qs"][:8].tolist() == [127, 3, -3, 2, -2, 1, -1, 4]
    # all-zero block: d = 0, inv = 0, q = 0
    blk = O.quantize_rows_q8_0(np.zeros(32, np.float32), 1, 32)[0]
    assert blk["d"] == 0 and not blk["qs"].any()


def test_quantize_invariants_random():
    rng = np.random.default_rng(7)
    x = rng.standard_normal(865 * 768).astype(np.float32)
    q = O.quantize_rows_q8_0(x, 865, 768)
    xb = x.reshape(-1, 32).astype(np.float64)
    d32 = np.abs(xb).max(1) / np.float32(127.0)
    qs = q["qs"].astype(np.float64)
    # the block maximum lands on +-127 and the sign of every value survives
    assert np.all(np.abs(qs).max(1) == 127)
    assert np.all(np.sign(qs) * np.sign(xb) >= 0)
    # rounding error at most half a step, plus the f32 rounding of x * (1/d)
    # before round(): |x/d| <= 127, so at most 127 * 2^-23 of a step more.
    assert np.all(np.abs(xb - qs * d32[:, None]) <= d32[:, None] * (0.5 + 127 * 2.0 ** -23))
    # stored scale is the f16 rounding of d
    d16 = np.array([O.f16_to_f32(int(h)) for h in q["d"][:200]])
    assert np.all(np.abs(d16 - d32[:200]) <= d32[:200] * 2.0 ** -11)


def test_dequantize_kat():
    blk = np.zeros(1, O.BLOCK_Q8_0)
    blk["d"] = 0x3800  # 0.5
    blk["qs"][0][:4] = [1, -2, 127, -127]
    assert O.dequantize_q8_0(blk)[:4].tolist() == [0.5, -1.0, 63.5, -63.5]


def test_gemm_q8_0_matches_float64_block_sum():
    m, n, k = 9, 11, 160
    rng = np.random.default_rng(3)
    aq = O.quantize_rows_q8_0(rng.standard_normal(m * k).astype(np.float32), m, k)
    bq = O.quantize_rows_q8_0(rng.standard_normal(n * k).astype(np.float32), n, k)
    c = O.gemm_q8_0(aq, bq, m, n, k)
    da = np.array([O.f16_to_f32(int(h)) for h in aq["d"]]).reshape(m, -1)
    db = np.array([O.f16_to_f32(int(h)) for h in bq["d"]]).reshape(n, -1)
    qa = aq["qs"].astype(np.int64).reshape(m, -1, 32)
    qb = bq["qs"].astype(np.int64).reshape(n, -1, 32)
    isum = np.einsum("ibl,jbl->ijb", qa, qb)
    ref = np.einsum("ib,jb,ijb->ij", da, db, isum.astype(np.float64))
    assert np.abs(c.reshape(m, n) - ref).max() <= 1e-6 * np.abs(ref).max()


def test_quantize_block_max_ignores_every_nan():
    """quantize_row_q8_0 folds amax from 0 with f32::max (src/q8_0_dot.rs:35),
    which returns the other operand when one is NaN and, unlike IEEE maxNum,
    treats signalling NaNs like quiet ones (core f32::max).  So a block of
    NaNs has amax 0 (d = 0, every value 0) and a NaN never hides the other
    values' maximum, wherever it sits in the block."""
    snan, qnan = np.uint32(0x7F800005), np.uint32(0x7FC00000)
    assert O.rust_max(1.0, float("nan")) == 1.0 and O.rust_max(float("nan"), 2.0) == 2.0
    for nan in (snan, qnan):
        block = np.full(32, nan, np.uint32).view(np.float32)
        b = O.quantize_rows_q8_0(block, 1, 32)
        assert b["d"][0] == 0 and not b["qs"].any()
        for pos in (0, 17, 31):
            bits = np.full(32, np.float32(1.0).view(np.uint32), np.uint32)
            bits[pos] = nan
            b = O.quantize_rows_q8_0(bits.view(np.float32), 1, 32)
            assert b["d"][0] == O.f32_to_f16(np.float32(1.0) / np.float32(127.0))
            q = b["qs"][0]
            assert q[pos] == 0 and (np.delete(q, pos) == 127).all()
