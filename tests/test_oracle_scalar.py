"""Pins the oracle's restatement of src/scalar.rs, src/simd_avx512.rs and
src/dispatch.rs (CPU only).

Every check is one the reference's own tests make (cited) or one fixed by
the mathematics (float64 closed forms, published error bounds), so a dropped
term, a swapped operand or a contracted FMA fails at least one of them.
"""
import math

import numpy as np
import pytest

import oracle as O


def f32(x):
    return np.asarray(x, np.float32)


# ---- tests/scalar_ops.rs ----------------------------------------------------

def test_gemm_2x2_identity():
    """tests/scalar_ops.rs:3-11"""
    assert O.gemm_f32([1, 2, 3, 4], [1, 0, 0, 1], 2, 2, 2).tolist() == [1, 2, 3, 4]


def test_gemm_kat():
    """src/cuda.rs:1405-1411: [1..6] x [7..12] = [58, 64, 139, 154]."""
    assert O.gemm_f32([1, 2, 3, 4, 5, 6], [7, 8, 9, 10, 11, 12], 2, 2, 3).tolist() == \
        [58, 64, 139, 154]


def test_softmax_rows_sums_to_one():
    """tests/scalar_ops.rs:13-20"""
    x = O.softmax_rows([1.0, 2.0, 3.0, 0.0, 0.0, 0.0], 2, 3)
    assert abs(x[:3].sum() - 1) < 1e-6 and abs(x[3:].sum() - 1) < 1e-6
    assert abs(x[3] - 1 / 3) < 1e-6
    e = np.exp(np.array([1.0, 2.0, 3.0]) - 3.0)
    assert np.abs(x[:3] - e / e.sum()).max() < 1e-7


def test_gelu_zero_and_large():
    """tests/scalar_ops.rs:22-29"""
    x = O.gelu([0.0, 10.0, -10.0])
    assert abs(x[0]) < 1e-6 and abs(x[1] - 10.0) < 1e-3 and abs(x[2]) < 1e-3


def test_layernorm_zero_mean_and_float64_closed_form():
    """tests/scalar_ops.rs:31-39 plus the float64 formula."""
    x = O.layernorm([1.0, 2.0, 3.0, 4.0], 1, 4, [1] * 4, [0] * 4, 1e-5)
    assert abs(x.mean()) < 1e-4
    d = np.array([1.0, 2.0, 3.0, 4.0]) - 2.5
    assert np.abs(x - d / np.sqrt((d * d).mean() + 1e-5)).max() < 1e-6


def test_layerscale_kat():
    """tests/scalar_ops.rs:41-47"""
    assert O.layerscale([1, 2, 3, 4, 5, 6], 2, 3, [10.0, -1.0, 0.5]).tolist() == \
        [10.0, -2.0, 1.5, 40.0, -5.0, 3.0]


def test_add_kat():
    """src/cuda.rs:1376-1379"""
    assert O.add([1.0, -2.0, 3.5], [0.5, 2.0, -1.0]).tolist() == [1.5, 0.0, 2.5]


# ---- src/scalar.rs:179-237 parallel == serial --------------------------------

def test_parallel_layernorm_is_bitwise_per_row_and_thread_invariant():
    rows, cols = 67, 64
    gamma = f32([0.1 + i * 0.01 for i in range(cols)])
    beta = f32([-0.2 + i * 0.02 for i in range(cols)])
    x = f32([((i * 37 % 101) - 50.0) * 0.03125 for i in range(rows * cols)])
    par = O.layernorm(x, rows, cols, gamma, beta, 1e-5)
    per_row = np.concatenate([O.layernorm(x[r * cols:(r + 1) * cols], 1, cols, gamma, beta, 1e-5)
                              for r in range(rows)])
    assert np.array_equal(par.view(np.uint32), per_row.view(np.uint32))
    O.set_threads(1)
    try:
        one = O.layernorm(x, rows, cols, gamma, beta, 1e-5)
    finally:
        O.set_threads(0)
    assert np.array_equal(par.view(np.uint32), one.view(np.uint32))
    xr = x.reshape(rows, cols).astype(np.float64)
    mu = xr.mean(1, keepdims=True)
    ref = (xr - mu) / np.sqrt(((xr - mu) ** 2).mean(1, keepdims=True) + 1e-5) * gamma + beta
    assert np.abs(par.reshape(rows, cols) - ref).max() < 2e-6


def test_parallel_rowwise_epilogues_are_bitwise():
    rows, cols = 67, 64
    bias = f32([i * 0.01 - 0.2 for i in range(cols)])
    gamma = f32([i * 0.02 + 0.3 for i in range(cols)])
    x = f32([(i - 1000.0) * 0.03125 for i in range(rows * cols)])
    got = O.layerscale(O.add_bias_rows(x, rows, cols, bias), rows, cols, gamma)
    exp = ((x.reshape(rows, cols) + bias) * gamma).reshape(-1)  # IEEE f32 ops
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


# ---- erf / GELU / Cephes exp ---------------------------------------------------

def test_erf_within_abramowitz_stegun_bound():
    """A&S 7.1.26: |error| < 1.5e-7 (plus f32 rounding of ~10 ops)."""
    xs = np.linspace(-6, 6, 4001, dtype=np.float32)
    err = max(abs(O.erf(float(v)) - math.erf(float(v))) for v in xs)
    assert err < 1.5e-7 + 6e-7
    # The A&S polynomial sums to 1 + O(ulp) at t = 1, so erf(0) is ~6e-8, not 0.
    assert abs(O.erf(0.0)) < 1.5e-7
    assert O.erf(1.0) == -O.erf(-1.0) and O.erf(0.0) == -O.erf(-0.0)  # odd via signum


def test_cephes_exp_accuracy():
    xs = np.concatenate([np.linspace(-87, 88, 20001), [0.0, -1e-8, 1e-8, 88.7, -100.0]])
    for v in xs.astype(np.float32):
        got = O.cephes_exp(float(v))
        clamped = min(max(float(v), -88.37626), 88.37626)
        exact = math.exp(float(np.float32(clamped)))
        assert abs(got - exact) <= 3e-7 * exact + 1e-38, (v, got, exact)
    assert O.cephes_exp(0.0) == 1.0


def test_gelu_vs_exact_erf_gelu():
    xs = np.linspace(-8, 8, 3001, dtype=np.float32)
    got = O.gelu(xs)
    exact = np.array([0.5 * float(v) * (1 + math.erf(float(v) / math.sqrt(2))) for v in xs])
    assert np.abs(got - exact).max() < 2e-6


def test_gelu_simd_matches_scalar():
    """tests/simd_matches_scalar.rs:9-22: ramp 0.017i - 3, n = 1000, < 1e-4."""
    x = (np.arange(1000, dtype=np.float32) * np.float32(0.017) - np.float32(3.0)).astype(np.float32)
    assert np.abs(O.kernels_gelu(x) - O.gelu(x)).max() < 1e-4
    assert np.abs(O.gelu_avx512_lanes(x) - O.gelu(x)).max() < 1e-6


def test_add_simd_matches_scalar():
    """tests/simd_matches_scalar.rs:24-33 (exact)."""
    x = (np.arange(1000, dtype=np.float32) * np.float32(0.017) - np.float32(3.0)).astype(np.float32)
    assert np.array_equal(O.kernels_add(x, x), O.add(x, x))


@pytest.mark.skipif(not O.has_avx512(), reason="host without AVX-512")
def test_gelu_lane_restatement_is_bitwise_avx512():
    x = np.random.default_rng(5).standard_normal(100_003).astype(np.float32) * 4
    a, b = O.gelu_avx512_lanes(x), O.gelu_avx512(x)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    tail = x[-(x.size % 16):]
    assert np.array_equal(a[-tail.size:], O.gelu(tail))  # n % 16 tail is scalar::gelu


# ---- the host libm's expf, restated for the device's scalar GELU tail -----------

def test_exp2f_table_is_the_correctly_rounded_powers_of_two():
    """Entry i is the bits of 2^(i/32) rounded to double, minus i << 47: 2^(i/32)
    from 60-digit decimal arithmetic, rounded by float()."""
    from decimal import Decimal, getcontext
    import struct
    getcontext().prec = 60
    ln2 = Decimal(2).ln()
    for i in range(32):
        d = float((Decimal(i) / 32 * ln2).exp())
        bits = struct.unpack("<Q", struct.pack("<d", d))[0]
        assert O.exp2f_table_entry(i) == bits - (i << 47), i


def test_expf_restatement_equals_host_expf_for_every_input():
    """All 2^32 bit patterns (NaN results compared as NaN): the restated
    algorithm is the host's expf (glibc, which f32::exp calls on Linux), so
    the device's transcription of it gives the crate's bits in the GELU tail."""
    assert O.expf_form_mismatches(1) == 0


def test_device_gelu_tail_uses_the_restated_expf():
    """The device's glibc_expf (common.h) carries the oracle's table and
    constants digit for digit."""
    import re
    from pathlib import Path
    src = (Path(__file__).resolve().parents[1] / "vestra-kernels_amd/csrc/common.h").read_text()
    body = src[src.index("float glibc_expf(float x)"):src.index("float gelu_scalar_form(float v)")]
    tab = [int(t, 16) for t in re.findall(r"0x([0-9a-f]{16})ull", body)]
    assert tab == [O.exp2f_table_entry(i) for i in range(32)]
    for c in ("0x1.71547652b82fep+0", "0x1.8p+52", "0x1.c6af84b912394p-5", "0x1.ebfce50fac4f3p-3",
              "0x1.62e42ff0c52d6p-1", "0x1.62e42ep6f", "-0x1.9fe368p6f"):
        assert c in body, c
    assert "glibc_expf(mul_rn(-ax, ax))" in src
