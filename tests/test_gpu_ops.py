"""GPU parity of the C-ABI device operators against the reference's device
KATs (src/cuda.rs:1370-1607) and the CPU oracle.

Bars: bit-exact for layout, copies, residual adds, RoPE with host tables,
CPU-order LayerNorm and Q8_0; the reference's own tolerances elsewhere.
"""
import numpy as np
import pytest

import oracle as O
import vestra_hip as vh
from conftest import assert_bits_equal, max_rel
from vestra_hip import da3, seeded

pytestmark = pytest.mark.gpu


def deterministic_values(n, seed):
    """src/cuda.rs:1363-1367: sin(i*0.017578125 + seed)*0.75 + 0.1 in f32."""
    i = np.arange(n, dtype=np.float32)
    return ((np.sin((i * np.float32(0.017578125) + np.float32(seed)).astype(np.float32))
             .astype(np.float32) * np.float32(0.75)) + np.float32(0.1)).astype(np.float32)


# ---- src/cuda.rs:1370-1607 driver round trip and KATs ----------------------

def test_round_trip_add_copy_segments(rt):
    t = rt.upload_f32([1.0, -2.0, 3.5])
    add = rt.upload_f32([0.5, 2.0, -1.0])
    assert len(t) == 3 and not t.is_empty()
    rt.add_f32_in_place(t, add)
    assert rt.download_f32(t).tolist() == [1.5, 0.0, 2.5]
    src = rt.upload_f32([9.0, 8.0, 7.0, 6.0])
    copied = rt.copy_f32(src)
    rt.overwrite_prefix_f32(copied, rt.upload_f32([-1.0, -2.0]), 2)
    assert rt.download_f32(copied).tolist() == [-1.0, -2.0, 7.0, 6.0]
    seg = rt.copy_segment_f32(src, 1, 2)
    assert rt.download_f32(seg).tolist() == [8.0, 7.0]
    rt.copy_segment_into_f32(copied, 2, seg, 0, 2)
    assert rt.download_f32(copied).tolist() == [-1.0, -2.0, 8.0, 7.0]


def test_gemm_bias_scale_linear_chain_kats(rt):
    left = rt.upload_f32([1, 2, 3, 4, 5, 6])
    right = rt.upload_f32([7, 8, 9, 10, 11, 12])
    prod = rt.gemm_row_major_f32(left, right, 2, 3, 2)
    assert rt.download_f32(prod).tolist() == [58.0, 64.0, 139.0, 154.0]
    rt.bias_scale_f32_in_place(prod, rt.upload_f32([1.0, -4.0]), rt.upload_f32([0.5, 2.0]), 2, 2)
    assert rt.download_f32(prod).tolist() == [29.5, 120.0, 70.0, 300.0]
    first = rt.prepare_linear_f32(3, 2, [7, 8, 9, 10, 11, 12], [1.0, -4.0], [0.5, 2.0])
    second = rt.prepare_linear_f32(2, 1, [2.0, -1.0], [3.0])
    chained = second.run(first.run(left, 2), 2)
    assert rt.download_f32(chained).tolist() == [-58.0, -157.0]
    assert rt.download_f32(first.run_chw(left, 2)).tolist() == [29.5, 70.0, 120.0, 300.0]
    assert first.input_features() == 3 and first.output_features() == 2


def test_gelu_kat_within_2e6_of_scalar(rt):
    x = np.array([-3.0, -1.0, 0.0, 1.0, 3.0], np.float32)
    t = rt.upload_f32(x)
    rt.gelu_f32_in_place(t)
    assert np.abs(rt.download_f32(t) - O.gelu(x)).max() <= 2e-6


def test_layernorm_kats(rt):
    x = [1.0, 2.0, 5.0, -2.0, 3.0, 4.0]
    g, b = [1.5, 0.5, 2.0], [-1.0, 0.25, 2.0]
    exp = O.layernorm(x, 2, 3, g, b, 1e-5)
    xt, gt, bt = rt.upload_f32(x), rt.upload_f32(g), rt.upload_f32(b)
    assert np.abs(rt.download_f32(rt.layernorm_f32(xt, gt, bt, 2, 3, 1e-5)) - exp).max() <= 2e-5
    cpu = rt.download_f32(rt.layernorm_f32_cpu_order(xt, gt, bt, 2, 3, 1e-5))
    assert np.abs(cpu - exp).max() <= 2e-6
    assert_bits_equal(cpu, exp, "cpu-order LayerNorm")


def test_small_online_attention_vs_naive(rt):
    heads, tokens, hd = 2, 5, 4
    idx = np.arange(heads * tokens * hd, dtype=np.float32)

    def vals(seed):
        return np.sin(idx * np.float32(0.03125) + np.float32(seed)).astype(np.float32)

    q, k, v = vals(0.1), vals(-0.2), vals(0.7)
    exp = O.attention_naive(q, k, v, heads, tokens, hd)
    out = rt.attention_online_f32(rt.upload_f32(q), rt.upload_f32(k), rt.upload_f32(v), heads,
                                  tokens, hd)
    assert np.abs(rt.download_f32(out) - exp).max() <= 5e-5


def test_layout_split_unpack_chw(rt):
    T, H, Dh = 3, 2, 4
    E = H * Dh
    qkv = deterministic_values(T * 3 * E, -0.4)
    q, k, v = rt.split_qkv_hnd_f32(rt.upload_f32(qkv), T, H, Dh)
    eq, ek, ev = O.split_qkv_hnd(qkv, T, H, Dh)
    assert_bits_equal(rt.download_f32(q), eq, "split q")
    assert_bits_equal(rt.download_f32(k), ek, "split k")
    assert_bits_equal(rt.download_f32(v), ev, "split v")
    tm = rt.hnd_to_token_f32(q, T, H, Dh)
    etm = O.hnd_to_token(eq, T, H, Dh)
    assert_bits_equal(rt.download_f32(tm), etm, "hnd_to_token")
    chw = rt.download_f32(rt.token_to_chw_f32(tm, T, E))
    assert_bits_equal(chw, etm.reshape(T, E).T.reshape(-1), "token_to_chw")


def test_patchify_and_token_assembly_kats(rt):
    image = rt.upload_f32(np.arange(48, dtype=np.float32))
    patches = rt.download_f32(rt.patchify_nchw_f32(image, 4, 4, 2, 3))
    assert patches.tolist() == [
        0, 1, 4, 5, 16, 17, 20, 21, 32, 33, 36, 37, 2, 3, 6, 7, 18, 19, 22, 23, 34, 35, 38, 39,
        8, 9, 12, 13, 24, 25, 28, 29, 40, 41, 44, 45, 10, 11, 14, 15, 26, 27, 30, 31, 42, 43, 46,
        47]
    toks = rt.prepend_cls_add_pos_f32(rt.upload_f32([10, 20, 30, 40]), rt.upload_f32([1, 2]),
                                      rt.upload_f32([0.5, -0.5, 1.0, 2.0, -1.0, 3.0]), 2, 2)
    assert rt.download_f32(toks).tolist() == [1.5, 1.5, 11.0, 22.0, 29.0, 43.0]


# ---- error contract (CudaError variants, validation before launch) ---------

def test_errors_before_launch(rt):
    a = rt.upload_f32([1.0, 2.0, 3.0])
    b = rt.upload_f32([1.0, 2.0])
    with pytest.raises(vh.LengthMismatch) as e:
        rt.add_f32_in_place(a, b)
    assert (e.value.destination, e.value.source_len) == (3, 2)
    with pytest.raises(vh.BlasError):
        rt.gemm_row_major_f32(a, b, 2, 2, 2)
    with pytest.raises(vh.KernelError):
        rt.attention_online_f32(a, a, a, 1, 1, 65)
    with pytest.raises(vh.KernelError):
        rt.patchify_nchw_f32(a, 3, 1, 2, 1)
    with pytest.raises(vh.LengthMismatch):
        rt.copy_segment_f32(a, 2, 2)
    lin = rt.prepare_linear_f32(2, 1, [1.0, 2.0], [0.0])
    with pytest.raises(vh.BlasError):
        lin.run(a, 2)
    assert rt.download_f32(a).tolist() == [1.0, 2.0, 3.0]  # untouched


# ---- GEMM (fp32 MFMA) -------------------------------------------------------

# (70, 100, 2304) and (70, 3000, 768) take the 64 x 128 x 64 tile with K not a
# multiple of 64 (the masked slice path of the BK = 64 swizzled layout);
# (70, 2112, 768) whole 64-wide slices in an odd count per split (the slice
# loop runs two slices per iteration plus one).
@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (7, 5, 3), (865, 768, 768), (33, 96, 130),
                                   (64, 32, 64), (129, 67, 257), (70, 100, 2304), (70, 3000, 768),
                                   (70, 2112, 768)])
def test_gemm_row_major_matches_float64(rt, m, k, n):
    a = seeded.normal(101 + m, m * k)
    b = seeded.normal(202 + n, k * n)
    c = rt.download_f32(rt.gemm_row_major_f32(rt.upload_f32(a), rt.upload_f32(b), m, k, n))
    ref = a.reshape(m, k).astype(np.float64) @ b.reshape(k, n).astype(np.float64)
    # fp32 accumulation of K products: |err| <= K * eps * sum|a||b| bounds it.
    bound = k * 6e-8 * (np.abs(a.reshape(m, k)).astype(np.float64) @ np.abs(b.reshape(k, n)))
    assert np.all(np.abs(c.reshape(m, n) - ref) <= bound + 1e-30)


@pytest.mark.parametrize("rows, k, n, gamma", [(865, 768, 96, False), (864, 768, 768, False),
                                               (37, 64, 40, False), (865, 768, 96, True),
                                               (10, 20, 6, False)])
def test_linear_run_chw_equals_token_to_chw_of_run(rt, monkeypatch, rows, k, n, gamma):
    """CudaLinearF32::run_chw (src/cuda.rs:1340-1344) is token_to_chw of run.
    A linear without LayerScale and with K % 32 == 0 computes the transposed
    product in one GEMM (weight rows as A, input rows as Bt, channel-major
    store); the others run, then transpose.  Against float64 within the f32
    accumulation bound, and, with whole tiles on both routes (no balanced
    tail), bit for bit against the composition."""
    w = seeded.normal(7100 + n, k * n, 0.05)
    b = seeded.normal(7200 + n, n, 0.1)
    g = (0.5 + seeded.uniform01(7300 + n, n)).astype(np.float32) if gamma else None
    lin = rt.prepare_linear_f32(k, n, w, b, g)
    x = seeded.normal(7400 + rows, rows * k)
    xt = rt.upload_f32(x)
    got = rt.download_f32(lin.run_chw(xt, rows)).reshape(n, rows)
    ref = x.reshape(rows, k).astype(np.float64) @ w.reshape(k, n).astype(np.float64) + b
    if gamma:
        ref = ref * g
    bound = (k + 2) * 6e-8 * (np.abs(x.reshape(rows, k)).astype(np.float64) @ np.abs(w.reshape(k, n)) + np.abs(b))
    if gamma:
        bound = bound * np.abs(g) + 6e-8 * np.abs(ref)
    assert np.all(np.abs(got.T - ref) <= bound + 1e-30)
    monkeypatch.setenv("VESTRA_HIP_GEMM_TAIL", "0")
    a = rt.download_f32(lin.run_chw(xt, rows))
    e = rt.download_f32(rt.token_to_chw_f32(lin.run(xt, rows), rows, n))
    assert_bits_equal(a, e, f"run_chw vs token_to_chw(run) {rows}x{k}->{n}")


@pytest.mark.parametrize("m,k,n", [(865, 768, 3072), (33, 96, 130), (1, 768, 3072), (70, 64, 257)])
def test_gemm_row_major_b_in_place_equals_transposed_copy(rt, monkeypatch, m, k, n):
    """gemm_row_major_f32 reads B [K][N] in place (the default at M, K <=
    1024 with K % 32 == 0) or multiplies by a transposed copy
    (VESTRA_HIP_GEMM_RM_DIRECT=0): with whole tiles on both routes they take
    the same products in the same k order, so the same bits."""
    a = rt.upload_f32(seeded.normal(7500 + m, m * k))
    b = rt.upload_f32(seeded.normal(7600 + n, k * n, 0.05))
    monkeypatch.setenv("VESTRA_HIP_GEMM_TAIL", "0")
    outs = []
    for route in ("1", "0"):
        monkeypatch.setenv("VESTRA_HIP_GEMM_RM_DIRECT", route)
        outs.append(rt.download_f32(rt.gemm_row_major_f32(a, b, m, k, n)))
    assert_bits_equal(outs[0], outs[1], f"row-major GEMM {m}x{k}x{n}: B in place vs transposed")


# M = 865 is one 504x336 image; 3460 = the batch of 4 (BASELINE config 5a) and
# 3457 = one 1008x672 image (config 5b).  Past M = 1024 the GEMM takes other
# tiles, an XCD-ordered tile walk and other split-K choices, so those paths
# are compared with the oracle at those sizes too.
PROJ_M = [865, 3460, 3457]
PROJ_KN = [(768, 2304), (768, 768), (768, 3072), (3072, 768)]


@pytest.mark.parametrize("m", PROJ_M)
@pytest.mark.parametrize("k,n", PROJ_KN)
def test_da3_projection_shapes_vs_oracle(rt, m, k, n):
    a = seeded.normal(11, m * k)
    w = seeded.normal(12, k * n, 0.02)
    bias = seeded.normal(13, n, 0.01)
    scale = (0.75 + np.cos(np.arange(n) * 0.011)).astype(np.float32)
    exp = O.linear_bias_scale(a, w, bias, scale, m, n, k)
    lin = rt.prepare_linear_f32(k, n, w, bias, scale)
    got = rt.download_f32(lin.run(rt.upload_f32(a), m))
    assert max_rel(got, exp) <= 1e-5
    # a transposed weight (a plausible packing mistake) misses by far more
    if k == n:
        wt = np.ascontiguousarray(w.reshape(k, n).T).reshape(-1)
        assert max_rel(O.linear_bias_scale(a, wt, bias, scale, m, n, k), exp) >= 1e-3


@pytest.mark.parametrize("m", PROJ_M)
def test_fc1_gelu_epilogue_vs_oracle(rt, m):
    k, n = 768, 3072
    a = seeded.normal(21, m * k)
    w = seeded.normal(22, k * n, 0.02)
    bias = seeded.normal(23, n, 0.02)
    f = O.linear(a, w, m, n, k)
    f = O.add_bias_rows(f, m, n, bias)
    exp = O.gelu_avx512_lanes(f)
    lin = rt.prepare_linear_f32(k, n, w, bias)
    got = rt.download_f32(lin.run_gelu(rt.upload_f32(a), m))
    assert max_rel(got, exp) <= 1e-5


def test_fused_gelu_epilogue_form(rt):
    """The f32 GEMM's GELU epilogue evaluates the A&S 7.1.26 erf of
    Kernels::gelu with the hardware reciprocal and exp2.  Through an identity
    weight (every product but one is an exact zero, so the GEMM returns its
    input) it is compared with the oracle's exact GELU over [-12, 12], the
    edges of the erf polynomial and signed zeros: within 1e-6 * max(1, |v|)
    absolutely, against 0.47 for a GELU that dropped the 1/sqrt(2) (a
    plausible slip; computed with the oracle)."""
    k = n = 256
    v = np.concatenate([np.linspace(-12.0, 12.0, 256 * 250), [0.0, -0.0, 1e-30, -1e-30, 4.0, -4.0]])
    v = np.concatenate([v, np.zeros((-v.size) % k)]).astype(np.float32)
    m = v.size // k
    lin = rt.prepare_linear_f32(k, n, np.eye(k, dtype=np.float32).reshape(-1), np.zeros(n, np.float32))
    got = rt.download_f32(lin.run_gelu(rt.upload_f32(v), m))
    exp = O.kernels_gelu(v)
    err = np.abs(got.astype(np.float64) - exp) / np.maximum(1.0, np.abs(v))
    assert err.max() <= 1e-6
    slip = np.abs(O.kernels_gelu((v * np.float32(np.sqrt(2.0))).astype(np.float32)) - exp)
    assert (slip / np.maximum(1.0, np.abs(v))).max() >= 0.1


@pytest.mark.parametrize("m,k,n", [(865, 768, 3072), (400, 768, 3072), (865, 768, 3136),
                                   (300, 256, 4096), (3460, 768, 3072), (865, 480, 3072)])
def test_gemm_balanced_tail(rt, monkeypatch, m, k, n):
    """The tiles past the last whole round over the CUs run as K pieces that
    the last piece to finish sums in piece order (64 x 64 tile, GELU
    epilogue).  Shapes: fc1 (672 tiles, 3 pieces), 336 tiles (3 pieces), 686
    tiles (4 pieces, tail padded to a multiple of 8), K = 256 (2 pieces), the
    batched fc1 (2640 tiles, XCD-ordered), K = 480 (3 pieces of 5 slices: an
    odd slice count per piece).  Bars: identical run to run, and
    within 1e-5 of the one-workgroup-per-tile grid, from which the tail's
    K-split sums must differ in some bits (the tail ran)."""
    a = rt.upload_f32(seeded.normal(41 + m, m * k))
    lin = rt.prepare_linear_f32(k, n, seeded.normal(42, k * n, 0.02), seeded.normal(43, n, 0.02))
    monkeypatch.setenv("VESTRA_HIP_GEMM_TAIL", "1")
    got = rt.download_f32(lin.run_gelu(a, m))
    again = rt.download_f32(lin.run_gelu(a, m))
    assert_bits_equal(again, got, "balanced tail rerun")
    monkeypatch.setenv("VESTRA_HIP_GEMM_TAIL", "0")
    whole = rt.download_f32(lin.run_gelu(a, m))
    assert max_rel(got, whole) <= 1e-5
    assert (got.view(np.uint32) != whole.view(np.uint32)).any()


@pytest.mark.parametrize("m", [865, 194])
def test_fc2_tail_equals_split_k(rt, monkeypatch, m):
    """A long-K projection whose 64 x 64 grid has fewer tiles than CUs (fc2:
    K = 3072, N = 768; 168 and 48 tiles) runs as the balanced tail over the
    split table's K ranges, so each output is the same sum of the same
    partials as split-K 3 with its reduction kernel: bit for bit, residual
    epilogue included."""
    k, n = 3072, 768
    a = rt.upload_f32(seeded.normal(61 + m, m * k))
    ls = (0.1 + 0.9 * seeded.uniform01(64, n)).astype(np.float32)
    lin = rt.prepare_linear_f32(k, n, seeded.normal(62, k * n, 0.02), seeded.normal(63, n, 0.02), ls)
    x = seeded.normal(65, m * n)
    xt = rt.upload_f32(x)
    lin.run_residual(a, m, xt)
    tail = rt.download_f32(xt)
    monkeypatch.setenv("VESTRA_HIP_GEMM_TILE", "64x128x64x2x4x3")
    xs = rt.upload_f32(x)
    lin.run_residual(a, m, xs)
    assert_bits_equal(tail, rt.download_f32(xs), "balanced tail against split-K 3")


def test_gemm_balanced_tail_store_matches_float64(rt):
    """Store epilogue through the row-major GEMM: 336 tiles, K = 512 in two
    pieces; the fp32 error bound of test_gemm_row_major_matches_float64."""
    m, k, n = 400, 512, 3072
    a = seeded.normal(51, m * k)
    b = seeded.normal(52, k * n)
    c = rt.download_f32(rt.gemm_row_major_f32(rt.upload_f32(a), rt.upload_f32(b), m, k, n))
    ref = a.reshape(m, k).astype(np.float64) @ b.reshape(k, n).astype(np.float64)
    bound = k * 6e-8 * (np.abs(a.reshape(m, k)).astype(np.float64) @ np.abs(b.reshape(k, n)))
    assert np.all(np.abs(c.reshape(m, n) - ref) <= bound + 1e-30)


@pytest.mark.parametrize("m", PROJ_M)
@pytest.mark.parametrize("k", [768, 3072], ids=["proj", "fc2"])
def test_residual_epilogue_vs_oracle(rt, m, k):
    n = 768
    a = seeded.normal(31, m * k)
    w = seeded.normal(32, k * n, 0.02)
    bias = seeded.normal(33, n, 0.02)
    ls = (0.1 + 0.9 * seeded.uniform01(35, n)).astype(np.float32)
    x = seeded.normal(34, m * n)
    y = O.linear_bias_scale(a, w, bias, ls, m, n, k)
    exp = O.kernels_add(x, y)
    lin = rt.prepare_linear_f32(k, n, w, bias, ls)
    xt = rt.upload_f32(x)
    lin.run_residual(rt.upload_f32(a), m, xt)
    assert max_rel(rt.download_f32(xt) - x, y) <= 1e-5
    assert max_rel(rt.download_f32(xt), exp) <= 1e-5


@pytest.mark.parametrize("m,k,mode", [(865, 768, "default"), (97, 768, "default"),
                                      (1000, 256, "default"), (3460, 768, "forced"),
                                      (865, 3072, "forced"), (200, 384, "forced")])
def test_kgroup_residual_gemm(rt, monkeypatch, m, k, mode):
    """The Residual GEMM with K split over two wave groups of one workgroup
    and summed through LDS (32 x 96 tiles; the out-projection's default at
    M <= 1024, K <= 1024, forced with VESTRA_HIP_GEMM_KGROUP=1 elsewhere).
    Bars: within 1e-5 of the oracle, the GEMM part inside the fp32 error
    bound of a float64 product, identical run to run, and different in some
    bits from unsplit 64 x 64 tiles (so the kernel ran), with LayerScale and
    ragged row tiles (97, 865, 1000 rows)."""
    n = 768
    a = seeded.normal(71 + m, m * k)
    w = seeded.normal(72, k * n, 0.02)
    bias = seeded.normal(73, n, 0.02)
    ls = (0.1 + 0.9 * seeded.uniform01(75, n)).astype(np.float32)
    x = seeded.normal(74 + m, m * n)
    lin = rt.prepare_linear_f32(k, n, w, bias, ls)
    at = rt.upload_f32(a)
    monkeypatch.setenv("VESTRA_HIP_GEMM_KGROUP", "1" if mode == "forced" else "")
    xt = rt.upload_f32(x)
    lin.run_residual(at, m, xt)
    got = rt.download_f32(xt)
    again = rt.upload_f32(x)
    lin.run_residual(at, m, again)
    assert_bits_equal(rt.download_f32(again), got, "kgroup rerun")
    y = O.linear_bias_scale(a, w, bias, ls, m, n, k)
    assert max_rel(got, O.kernels_add(x, y)) <= 1e-5
    ref = a.reshape(m, k).astype(np.float64) @ w.reshape(k, n).astype(np.float64)
    bound = k * 6e-8 * (np.abs(a.reshape(m, k)).astype(np.float64) @ np.abs(w.reshape(k, n)))
    acc = ((got.reshape(m, n).astype(np.float64) - x.reshape(m, n)) / ls - bias)
    # acc carries the rounding of the bias add, the LayerScale and the
    # residual add too: a few ulps of |x| and |y| on top of the GEMM bound.
    slack = 4e-7 * (np.abs(x.reshape(m, n)) / ls + np.abs(ref) + np.abs(bias))
    assert np.all(np.abs(acc - ref) <= bound + slack)
    monkeypatch.setenv("VESTRA_HIP_GEMM_KGROUP", "0")
    monkeypatch.setenv("VESTRA_HIP_GEMM_TAIL", "0")
    monkeypatch.setenv("VESTRA_HIP_GEMM_TILE", "64x64x32x2x2x1")
    other = rt.upload_f32(x)
    lin.run_residual(at, m, other)
    other = rt.download_f32(other)
    assert max_rel(got - x, other - x) <= 1e-5
    assert (got.view(np.uint32) != other.view(np.uint32)).any()


@pytest.mark.parametrize("m,k,mode", [(865, 768, "default"), (97, 768, "default"),
                                      (865, 3072, "forced")])
def test_kgroup_store_gemm(rt, monkeypatch, m, k, mode):
    """The Store epilogue ((acc + b) * LayerScale, CudaLinearF32::run) on the
    K-group GEMM, the default for the out-projection's shape: within 1e-5 of
    the oracle, identical run to run, and different in some bits from
    unsplit 64 x 64 tiles (so the kernel ran)."""
    n = 768
    a = seeded.normal(81 + m, m * k)
    w = seeded.normal(82, k * n, 0.02)
    bias = seeded.normal(83, n, 0.02)
    ls = (0.1 + 0.9 * seeded.uniform01(85, n)).astype(np.float32)
    lin = rt.prepare_linear_f32(k, n, w, bias, ls)
    at = rt.upload_f32(a)
    monkeypatch.setenv("VESTRA_HIP_GEMM_KGROUP", "1" if mode == "forced" else "")
    got = rt.download_f32(lin.run(at, m))
    assert_bits_equal(rt.download_f32(lin.run(at, m)), got, "kgroup store rerun")
    assert max_rel(got, O.linear_bias_scale(a, w, bias, ls, m, n, k)) <= 1e-5
    monkeypatch.setenv("VESTRA_HIP_GEMM_KGROUP", "0")
    monkeypatch.setenv("VESTRA_HIP_GEMM_TAIL", "0")
    monkeypatch.setenv("VESTRA_HIP_GEMM_TILE", "64x64x32x2x2x1")
    other = rt.download_f32(lin.run(at, m))
    assert max_rel(got, other) <= 1e-5
    assert (got.view(np.uint32) != other.view(np.uint32)).any()


@pytest.mark.parametrize("images, rows, cols, rope", [
    (1, 24, 36, False), (1, 24, 36, True), (4, 24, 36, True), (1, 48, 72, True)],
    ids=["865", "865-rope", "4x865-rope", "3457-rope"])
def test_qkv_head_major_rope_vs_oracle(rt, images, rows, cols, rope):
    """Q/K/V head-major [images][12][tokens][64] with bias, and the 2-D RoPE on
    the 24 x 36 grid (one image and the batch of 4, M = 3460) and on the
    48 x 72 grid of a 1008x672 image (M = 3457)."""
    T = rows * cols + 1
    a = seeded.normal(41, images * T * 768)
    w = seeded.normal(42, 768 * 2304, 0.02)
    bias = seeded.normal(43, 2304, 0.02)
    pos = da3.positions_yx(rows, cols)
    exp = {"q": [], "k": [], "v": []}
    for img in range(images):
        eq, ek, ev = O.qkv(a[img * T * 768:(img + 1) * T * 768], w, bias, T)
        if rope:
            eq = O.rope2d(eq, 12, T, 64, pos, 100.0)
            ek = O.rope2d(ek, 12, T, 64, pos, 100.0)
        for name, e in (("q", eq), ("k", ek), ("v", ev)):
            exp[name].append(e)
    lin = rt.prepare_linear_f32(768, 2304, w, bias)
    q, k, v = lin.run_qkv_hnd(rt.upload_f32(a), images, T, 12, pos if rope else None, 100.0)
    for got, name in ((q, "q"), (k, "k"), (v, "v")):
        e = np.concatenate(exp[name])
        g = rt.download_f32(got)
        assert max_rel(g, e) <= 1e-5, name
        for img in range(images):  # every image in its own slot, not just overall
            sl = slice(img * T * 768, (img + 1) * T * 768)
            assert max_rel(g[sl], e[sl]) <= 1e-5, (name, img)


# ---- attention ---------------------------------------------------------------

@pytest.mark.parametrize("heads,n,hd,seed", [(2, 8, 16, 0x12345678), (4, 37, 32, 0xDEADBEEF),
                                             (1, 130, 8, 0x0BADF00D), (3, 71, 64, 0xA7710001)])
def test_online_attention_matches_naive_cases(rt, heads, n, hd, seed):
    """tests/attention_matches_naive.rs:21-58 cases, |diff| < 1e-4."""
    vals = seeded.xorshift32_values(3 * heads * n * hd, seed)
    q, k, v = np.split(vals, 3)
    exp = O.attention_naive(q, k, v, heads, n, hd)
    got = rt.download_f32(rt.attention_online_f32(rt.upload_f32(q), rt.upload_f32(k),
                                                  rt.upload_f32(v), heads, n, hd))
    assert np.abs(got - exp).max() < 1e-4


@pytest.mark.parametrize("heads,n,hd", [(3, 1, 5), (2, 300, 7), (5, 865, 40), (1, 1000, 63),
                                        (12, 200, 1)])
def test_online_attention_small_head_dims_vs_naive(rt, heads, n, hd):
    """Head dims below 64 run the MFMA flash kernel on rows zero-padded to 64
    with a 1/sqrt(hd) scale: odd widths (the pad and unpad handle a partial
    float4), one token, and sequences long enough for key splits.  N(0,1)
    inputs; bar 1e-4 max-relative against attention_naive, which a scale of
    1/8 instead of 1/sqrt(hd) misses."""
    q, k, v = (seeded.normal(600 + i, heads * n * hd) for i in range(3))
    exp = O.attention_naive(q, k, v, heads, n, hd)
    got = rt.download_f32(rt.attention_online_f32(rt.upload_f32(q), rt.upload_f32(k),
                                                  rt.upload_f32(v), heads, n, hd))
    assert got.shape == exp.shape
    assert max_rel(got, exp) <= 1e-4
    if n > 1 and hd != 64:
        wrong = O.attention_naive(q * np.float32(np.sqrt(hd) / 8.0), k, v, heads, n, hd)
        assert max_rel(wrong, exp) >= 1e-2


def test_flash_da3_production_shape_vs_oracle(rt):
    """src/cuda.rs:1612-1650: 12 x 865 x 64, MAE <= 5e-5 and max <= 5e-4 against
    attention(); the parity bar here is the tighter max-relative 1e-4."""
    H, T = 12, 865
    n = H * T * 64
    q, k, v = deterministic_values(n, 0.1), deterministic_values(n, -0.3), deterministic_values(n, 0.7)
    exp = O.attention(q, k, v, H, T, 64)
    got = rt.download_f32(rt.flash_attention_f32_da3_base(rt.upload_f32(q), rt.upload_f32(k),
                                                          rt.upload_f32(v), H, T))
    err = np.abs(got - exp)
    assert err.mean() <= 5e-5 and err.max() <= 5e-4
    assert max_rel(got, exp) <= 1e-4


def test_flash_config1_normal_inputs_token_major(rt):
    """Q, K, V ~ N(0,1), 12 heads x 865 x 64, out [865, 768]."""
    H, T = 12, 865
    n = H * T * 64
    q, k, v = seeded.normal(1, n), seeded.normal(2, n), seeded.normal(3, n)
    exp = O.hnd_to_token(O.attention(q, k, v, H, T, 64), T, H, 64)
    got = rt.download_f32(rt.flash_attention_f32_da3_base(rt.upload_f32(q), rt.upload_f32(k),
                                                          rt.upload_f32(v), H, T, True))
    assert max_rel(got, exp) <= 1e-4


def test_flash_two_view_window_vs_serial(rt):
    """src/specialized.rs:2871-2910: 1 head x 2*865 tokens, MAE <= 2e-5, max <= 2e-4."""
    T = 2 * 865
    i = np.arange(T * 64, dtype=np.float32)
    q = np.sin(i * np.float32(0.013)).astype(np.float32)
    k = np.cos(i * np.float32(0.007)).astype(np.float32)
    v = np.sin(i * np.float32(0.017)).astype(np.float32)
    exp = O.attention_serial(q, k, v, 1, T, 64)
    got = rt.download_f32(rt.flash_attention_f32_da3_base(rt.upload_f32(q), rt.upload_f32(k),
                                                          rt.upload_f32(v), 1, T))
    err = np.abs(got - exp)
    assert err.mean() <= 2e-5 and err.max() <= 2e-4


@pytest.mark.parametrize("T", [1, 63, 64, 65, 3457])
def test_flash_ragged_token_counts(rt, T):
    H = 2
    n = H * T * 64
    q, k, v = seeded.normal(5 + T, n), seeded.normal(6 + T, n), seeded.normal(7 + T, n)
    exp = O.attention_naive(q, k, v, H, T, 64)
    got = rt.download_f32(rt.flash_attention_f32_da3_base(rt.upload_f32(q), rt.upload_f32(k),
                                                          rt.upload_f32(v), H, T))
    assert max_rel(got, exp) <= 1e-4


# ---- LayerNorm / GELU / RoPE ---------------------------------------------------

def test_layernorm_da3_shape(rt):
    rows, cols = 865, 768
    x = seeded.normal(51, rows * cols)
    g = seeded.normal(52, cols, 0.1, 1.0)
    b = seeded.normal(53, cols, 0.1)
    exp = O.layernorm(x, rows, cols, g, b, 1e-6)
    xt, gt, bt = rt.upload_f32(x), rt.upload_f32(g), rt.upload_f32(b)
    assert max_rel(rt.download_f32(rt.layernorm_f32(xt, gt, bt, rows, cols, 1e-6)), exp) <= 1e-5
    cpu = rt.download_f32(rt.layernorm_f32_cpu_order(xt, gt, bt, rows, cols, 1e-6))
    assert_bits_equal(cpu, exp, "cpu-order LayerNorm at 865x768")


@pytest.mark.parametrize("n", [1000, 2657280, 17])
def test_gelu_vs_kernels_gelu(rt, n):
    """tests/simd_matches_scalar.rs ramp plus the fc1 size; AVX-512 form on
    the n - n%16 prefix, scalar form (with the host libm's expf) on the
    tail, both bit for bit."""
    x = (np.arange(n, dtype=np.float32) * np.float32(0.017) - np.float32(3.0)) if n == 1000 \
        else seeded.normal(60 + n, n, 2.0)
    exp = O.gelu_avx512_lanes(x)
    t = rt.upload_f32(x)
    rt.gelu_f32_in_place(t)
    got = rt.download_f32(t)
    main = n - n % 16
    assert_bits_equal(got[:main], exp[:main], "AVX-512-form GELU")
    assert_bits_equal(got[main:], exp[main:], "scalar-form GELU tail")


def test_gelu_scalar_tail_bit_exact(rt):
    """Arrays shorter than 16 run wholly in Kernels::gelu's scalar tail
    (scalar::gelu, src/scalar.rs:116-134, whose exp is the host libm's expf,
    which the device restates): 4000 arrays of 15 values, uniform over
    [-15, 15] (exp's argument down past its underflow) and N(0, 2^2), bit for
    bit against the oracle."""
    rng = np.random.default_rng(0x6E1)
    vals = np.concatenate([rng.uniform(-15, 15, 30000),
                           rng.standard_normal(30000) * 2]).astype(np.float32)
    got = np.empty_like(vals)
    for i in range(0, vals.size, 15):
        t = rt.upload_f32(vals[i:i + 15])
        rt.gelu_f32_in_place(t)
        got[i:i + 15] = rt.download_f32(t)
    exp = np.concatenate([O.kernels_gelu(vals[i:i + 15]) for i in range(0, vals.size, 15)])
    assert_bits_equal(got, exp, "scalar GELU")


def test_rope2d_bit_exact_with_host_table(rt):
    H, T = 12, 865
    x = seeded.normal(71, H * T * 64)
    pos = da3.positions_yx(24, 36)
    exp = O.rope2d(x, H, T, 64, pos, 100.0)
    t = rt.upload_f32(x)
    rt.rope2d_f32_in_place(t, H, T, 64, pos, 100.0)
    assert_bits_equal(rt.download_f32(t), exp, "rope2d")
    # src/rope.rs:133-154 small case: positions (i, 3i), head_dim 16
    x2 = ((np.arange(3 * 7 * 16, dtype=np.float32) - 43.0) * 0.0625).astype(np.float32)
    pos2 = np.array([[i, 3 * i] for i in range(7)], np.int64).reshape(-1)
    t2 = rt.upload_f32(x2)
    rt.rope2d_f32_in_place(t2, 3, 7, 16, pos2, 100.0)
    assert_bits_equal(rt.download_f32(t2), O.rope2d(x2, 3, 7, 16, pos2, 100.0), "rope2d small")
    # head_dim 64 with a row count that leaves idle lanes in the last workgroup
    x3 = seeded.normal(72, 3 * 97 * 64)
    pos3 = np.array([[i % 5, i // 5] for i in range(97)], np.int64).reshape(-1)
    t3 = rt.upload_f32(x3)
    rt.rope2d_f32_in_place(t3, 3, 97, 64, pos3, 100.0)
    assert_bits_equal(rt.download_f32(t3), O.rope2d(x3, 3, 97, 64, pos3, 100.0), "rope2d ragged")


def test_qk_norm_rope_production_shape(rt):
    """src/cuda.rs:1652-1733: MAE <= 5e-5, max <= 5e-4 for Q and K."""
    H, T, Dm = 12, 865, 64
    n = H * T * Dm
    src = deterministic_values(n, 0.21)
    ksrc = deterministic_values(n, -0.37)
    qg, qb = deterministic_values(Dm, 0.11), deterministic_values(Dm, -0.15)
    kg, kb = deterministic_values(Dm, 0.31), deterministic_values(Dm, -0.23)
    pos = da3.positions_yx(24, 36)
    eq, ek = O.qk_norm_rope(src, ksrc, H, T, qg, qb, kg, kb, pos, 100.0, 1e-5)
    q, k = rt.upload_f32(src), rt.upload_f32(ksrc)
    rt.qk_norm_rope_f32_da3_base(q, k, rt.upload_f32(qg), rt.upload_f32(qb), rt.upload_f32(kg),
                                 rt.upload_f32(kb), rt.upload_f32(pos.astype(np.float32)), H, T,
                                 100.0, 1e-5)
    for got, exp in ((rt.download_f32(q), eq), (rt.download_f32(k), ek)):
        err = np.abs(got - exp)
        assert err.mean() <= 5e-5 and err.max() <= 5e-4


# ---- Q8_0 (bit-exact) -------------------------------------------------------------

# 4096 and 2048 rows take the 8-row tiles with one 16-byte store per block
# column of scales; 4100 rows end on a partial tile (2-byte scale stores).
@pytest.mark.parametrize("rows,k", [(865, 768), (3, 32), (8, 64), (4096, 768), (4100, 768), (2048, 96)])
def test_quantize_q8_0_bit_exact(rt, rows, k):
    x = seeded.normal(81 + rows, rows * k)
    x[:32] = 0.0  # an all-zero block: d = 0, inv = 0
    x[32:64] *= 1e-6  # tiny scales: f16 subnormal d
    exp = O.quantize_rows_q8_0(x, rows, k)
    got = rt.q8_0_download(rt.quantize_q8_0(rt.upload_f32(x), rows, k))
    assert np.array_equal(got["d"], exp["d"])
    assert np.array_equal(got["qs"], exp["qs"])


def test_quantize_into_an_existing_tensor(rt):
    """quantize_row_q8_0(x, out) writes the caller's blocks: equal to the
    allocating entry point and to the oracle, twice into the same tensor (the
    second call overwrites every block); a tensor of another shape is the
    reference's length assert."""
    rows, k = 4096, 768
    out = rt.quantize_q8_0(rt.upload_f32(np.ones(rows * k, np.float32)), rows, k)
    for seed in (4701, 4702):
        x = seeded.normal(seed, rows * k)
        xt = rt.upload_f32(x)
        rt.quantize_q8_0_into(xt, rows, k, out)
        got = rt.q8_0_download(out)
        assert np.array_equal(got, rt.q8_0_download(rt.quantize_q8_0(xt, rows, k)))
        exp = O.quantize_rows_q8_0(x, rows, k)
        assert np.array_equal(got["d"], exp["d"]) and np.array_equal(got["qs"], exp["qs"])
    with pytest.raises(vh.LengthMismatch):
        rt.quantize_q8_0_into(xt, rows - 1, k, out)
    small = rt.quantize_q8_0(rt.upload_f32(np.ones(64, np.float32)), 2, 32)
    with pytest.raises(vh.LengthMismatch):
        rt.quantize_q8_0_into(xt, rows, k, small)


def test_q8_0_upload_download_every_int8_value(rt):
    """Every int8 value (-128 included, as GGUF files may hold it) and
    arbitrary scale bits survive the device's block-major repack."""
    rows, k = 3, 256
    blocks = np.zeros(rows * k // 32, vh.BLOCK_Q8_0)
    blocks["qs"] = np.arange(rows * k, dtype=np.int64).reshape(-1, 32) % 256 - 128
    blocks["d"] = np.arange(blocks.size, dtype=np.uint16) * 2477 + 1
    got = rt.q8_0_download(rt.q8_0_upload(blocks, rows, k))
    assert np.array_equal(got["qs"], blocks["qs"]) and np.array_equal(got["d"], blocks["d"])
    # -128 operands: |isum| = 32 * 128^2 still exact
    a = np.zeros(1, vh.BLOCK_Q8_0)
    a["qs"], a["d"] = -128, 0x3C00  # d = 1.0
    c = rt.download_f32(rt.gemm_q8_0(rt.q8_0_upload(a, 1, 32), rt.q8_0_upload(a, 1, 32), 1, 1, 32))
    assert c[0] == 32 * 128 * 128


@pytest.mark.parametrize("m,n,k", [(865, 3072, 768), (8, 8, 64), (5, 17, 96), (64, 96, 3072),
                                   (33, 70, 1056), (1024, 1920, 2112), (1024, 1920, 1120)])
def test_gemm_q8_0_bit_exact(rt, m, n, k):
    """BASELINE config 4 (fc1 weights N(0, 0.02^2), activations N(0,1) quantised
    on the device), the tests/q8_0_dot_matches_f32.rs shape, and the scale
    chunking and prefetch grouping: the 32x32 tile with 96 blocks in one
    chunk (3072) and an odd block count (1056: one block per prefetch
    group), the 64x64 tile with 66 blocks in chunks of 32, 32 and 2 (2112)
    and with 35 blocks, odd, in chunks of 32 and 3 (1120)."""
    x = seeded.normal(91, m * k)
    w = seeded.normal(92, k * n, 0.02)
    wt = np.ascontiguousarray(w.reshape(k, n).T).reshape(-1)
    bq = O.quantize_rows_q8_0(wt, n, k)
    aq = O.quantize_rows_q8_0(x, m, k)
    exp = O.gemm_q8_0(aq, bq, m, n, k, impl="kernels")
    a_dev = rt.quantize_q8_0(rt.upload_f32(x), m, k)
    b_dev = rt.q8_0_upload(bq, n, k)
    got = rt.download_f32(rt.gemm_q8_0(a_dev, b_dev, m, n, k))
    assert_bits_equal(got, exp, "Q8_0 GEMM")


def test_gemm_q8_0_into_an_existing_tensor(rt):
    """Kernels::gemm_q8_0(m, n, k, a_q, b_q, c) writes the caller's c: equal
    bit for bit to the allocating entry point and to the oracle, twice into
    the same tensor (the second product overwrites every element, as a
    NaN-filled c shows); a c of another length is the reference's length
    assert (src/scalar.rs:37)."""
    m, n, k = 865, 3072, 768
    bq = O.quantize_rows_q8_0(seeded.normal(4802, n * k, 0.02), n, k)
    b_dev = rt.q8_0_upload(bq, n, k)
    c = rt.upload_f32(np.full(m * n, np.nan, np.float32))
    for seed in (4803, 4804):
        x = seeded.normal(seed, m * k)
        a_dev = rt.quantize_q8_0(rt.upload_f32(x), m, k)
        rt.gemm_q8_0_into(a_dev, b_dev, m, n, k, c)
        got = rt.download_f32(c)
        assert_bits_equal(got, rt.download_f32(rt.gemm_q8_0(a_dev, b_dev, m, n, k)), "into vs allocating")
        exp = O.gemm_q8_0(O.quantize_rows_q8_0(x, m, k), bq, m, n, k, impl="kernels")
        assert_bits_equal(got, exp, "into vs oracle")
    with pytest.raises(vh.LengthMismatch):
        rt.gemm_q8_0_into(a_dev, b_dev, m, n, k, rt.upload_f32(np.zeros(m * n - 1, np.float32)))
    with pytest.raises(vh.LengthMismatch):
        rt.gemm_q8_0_into(a_dev, b_dev, m - 1, n, k, c)


def test_flash_key_layouts_deterministic_and_consistent(rt, monkeypatch):
    """Every key layout -- one key stream per workgroup (direct-to-LDS panels,
    or register-staged panels with DIRECT=0), two streams per workgroup
    (merged in stream order through LDS), or keys split over 2-4 workgroups
    (merged in split order by a second kernel) -- gives run-to-run identical
    results, and all agree to rounding.  1-, 64- and 65-token shapes leave
    the second stream without valid keys; 130 tokens gives a split of one
    short panel."""
    layouts = (("1", "1", "1"), ("1", "1", "0"), ("1", "2", "1"), ("2", "1", "1"),
               ("3", "1", "1"), ("3", "1", "0"), ("4", "1", "1"))
    for H, T in ((12, 865), (2, 1), (2, 64), (2, 65), (1, 130)):
        n = H * T * 64
        q, k, v = (rt.upload_f32(seeded.normal(s + T, n)) for s in (31, 32, 33))
        outs = {}
        for splits, streams, direct in layouts:
            monkeypatch.setenv("VESTRA_HIP_FLASH_SPLITS", splits)
            monkeypatch.setenv("VESTRA_HIP_FLASH_STREAMS", streams)
            monkeypatch.setenv("VESTRA_HIP_FLASH_DIRECT", direct)
            a = rt.download_f32(rt.flash_attention_f32_da3_base(q, k, v, H, T))
            b = rt.download_f32(rt.flash_attention_f32_da3_base(q, k, v, H, T))
            assert_bits_equal(a, b, f"flash splits={splits} streams={streams} direct={direct} rerun")
            assert np.isfinite(a).all()
            outs[(splits, streams, direct)] = a
        for key, a in outs.items():
            assert max_rel(a, outs[("1", "1", "1")]) <= 2e-6, (H, T, key)


@pytest.mark.parametrize("xcd", ["1", "0"], ids=["xcd_grouped", "launch_order"])
@pytest.mark.parametrize("token_major", [False, True], ids=["head_major", "token_major"])
def test_flash_in_kernel_merge_equals_merge_launch(rt, monkeypatch, token_major, xcd):
    """Key splits merged by the split that finishes last in each 64-query
    group (VESTRA_HIP_FLASH_FUSED=1; the default when the grid is one round
    of workgroups) equal, bit for bit, the same splits merged by the separate
    merge launch (=0), at 2, 3 and 4 splits, for full and partial last query
    tiles and for grids of one round (12 x 865 at 2 and 3 splits) and of
    several (48 x 865).  In launch order (VESTRA_HIP_FLASH_XCD=0) the splits
    of a query group sit on different XCDs, whose L2s do not see each
    other's writes: the publication must go through the agent-scope path.  Each shape runs three times,
    every output kept alive so that no run lands in an earlier run's memory:
    the arrival counters must be back at zero after every run, or a later
    run would merge early or leave rows unwritten."""
    monkeypatch.setenv("VESTRA_HIP_FLASH_XCD", xcd)
    for H, T in ((12, 865), (48, 865), (1, 130), (3, 200), (2, 257)):
        n = H * T * 64
        q, k, v = (rt.upload_f32(seeded.normal(s + 7 * T + H, n)) for s in (41, 42, 43))
        for splits in ("2", "3", "4"):
            monkeypatch.setenv("VESTRA_HIP_FLASH_SPLITS", splits)
            monkeypatch.setenv("VESTRA_HIP_FLASH_FUSED", "0")
            exp = rt.download_f32(rt.flash_attention_f32_da3_base(q, k, v, H, T, token_major))
            assert np.isfinite(exp).all()
            monkeypatch.setenv("VESTRA_HIP_FLASH_FUSED", "1")
            kept = []
            for run in range(3):
                kept.append(rt.flash_attention_f32_da3_base(q, k, v, H, T, token_major))
                assert_bits_equal(rt.download_f32(kept[-1]), exp,
                                  f"in-kernel merge {H}x{T} splits={splits} run {run}")


# ---- streaming forms (launches that move >= 128 MiB) --------------------------
# Past 128 MiB of traffic the elementwise kernels switch to non-temporal
# loads and stores with more bytes in flight per thread.  Only the access
# flavour changes, so each large launch must equal, bit for bit, the same op
# run as smaller launches that take the regular form (or the oracle).

def _big(seed, n):
    base = seeded.normal(seed, 1 << 22)
    return np.tile(base, (n + base.size - 1) // base.size)[:n] * np.float32(1.0 + (seed % 7) / 8)


def test_streaming_copy_and_add_bit_exact(rt):
    n = (64 << 20) + 12  # 256 MiB + a tail; the add also takes the streaming form
    a, b = _big(61, n), _big(62, n)
    ta, tb = rt.upload_f32(a), rt.upload_f32(b)
    assert_bits_equal(rt.download_f32(rt.copy_f32(ta)), a, "streaming copy")
    rt.add_f32_in_place(ta, tb)
    assert_bits_equal(rt.download_f32(ta), (a + b).astype(np.float32), "streaming add")


def test_streaming_gelu_matches_oracle(rt):
    n = 40 << 20  # 160 MiB in place
    x = _big(63, n)
    t = rt.upload_f32(x)
    rt.gelu_f32_in_place(t)
    assert_bits_equal(rt.download_f32(t), O.kernels_gelu(x), "streaming GELU")


def test_streaming_layernorm_equals_regular_slices(rt):
    rows, cols, parts = 24576, 768, 4  # 144 MiB moved; each slice 36 MiB
    x = _big(64, rows * cols)
    g = (1.0 + 0.1 * seeded.normal(65, cols)).astype(np.float32)
    b = seeded.normal(66, cols, 0.1)
    gt, bt = rt.upload_f32(g), rt.upload_f32(b)
    big = rt.download_f32(rt.layernorm_f32(rt.upload_f32(x), gt, bt, rows, cols, 1e-6))
    r = rows // parts
    small = np.concatenate([rt.download_f32(rt.layernorm_f32(
        rt.upload_f32(x[i * r * cols:(i + 1) * r * cols]), gt, bt, r, cols, 1e-6)) for i in range(parts)])
    assert_bits_equal(big, small, "streaming LayerNorm")
    assert max_rel(big[:cols * 4], O.layernorm(x[:cols * 4], 4, cols, g, b, 1e-6)) <= 1e-5


def test_streaming_quantize_equals_regular_slices(rt):
    rows, k, parts = 49152, 768, 4  # 144 MiB read; each slice 36 MiB
    x = _big(67, rows * k)
    big = rt.q8_0_download(rt.quantize_q8_0(rt.upload_f32(x), rows, k))
    r = rows // parts
    small = np.concatenate([rt.q8_0_download(rt.quantize_q8_0(
        rt.upload_f32(x[i * r * k:(i + 1) * r * k]), r, k)) for i in range(parts)])
    assert np.array_equal(big.view(np.uint8), small.view(np.uint8))
    exp = O.quantize_rows_q8_0(x[:64 * k], 64, k)
    assert np.array_equal(big[:64 * k // 32].view(np.uint8), np.asarray(exp).view(np.uint8))


def test_streaming_rope_equals_regular_slices(rt):
    heads, n = 96, 3457  # 331872 rows of 64: 162 MiB moved; 8 heads per slice
    pos = da3.positions_yx(48, 72)
    x = _big(68, heads * n * 64)
    t = rt.upload_f32(x)
    rt.rope2d_f32_in_place(t, heads, n, 64, pos, 100.0)
    big = rt.download_f32(t)
    per = 8
    for h0 in range(0, heads, per):
        sl = slice(h0 * n * 64, (h0 + per) * n * 64)
        s = rt.upload_f32(x[sl])
        rt.rope2d_f32_in_place(s, per, n, 64, pos, 100.0)
        assert_bits_equal(big[sl], rt.download_f32(s), f"streaming RoPE heads {h0}..")


def test_gelu_bit_exact_over_a_float32_sweep(rt):
    """Every 7th float32 bit pattern (all exponents, both signs, 614M values
    in chunks), device GELU against the oracle's Kernels::gelu bit for bit.
    This covers the whole range of the erf reciprocal t = 1/(1 + 0.3275911
    |x| / sqrt 2), fast path [1, 2^64) and the division past it included;
    NaN inputs give NaN on both sides."""
    chunk = 7 << 22  # a multiple of 16 and of 7: every value takes the AVX-512 form
    step = 7
    for start in range(0, 1 << 32, chunk * step):
        bits = np.arange(start, min(start + chunk * step, 1 << 32), step, dtype=np.uint64)
        bits = bits[:bits.size - bits.size % 16].astype(np.uint32)
        x = bits.view(np.float32)
        t = rt.upload_f32(x)
        rt.gelu_f32_in_place(t)
        got = rt.download_f32(t)
        exp = O.kernels_gelu(x)
        same = (got.view(np.uint32) == exp.view(np.uint32)) | (np.isnan(got) & np.isnan(exp))
        assert same.all(), (start, x[~same][:4], got[~same][:4], exp[~same][:4])


def test_quantize_bit_exact_over_a_float32_sweep(rt):
    """Every 7th float32 bit pattern (614M values, both signs, every
    exponent, subnormals, infinities and NaN patterns) as rows of 768:
    quantize_row_q8_0 on the device against the oracle, every block's bytes.
    Each block's amax then sweeps the float range, so the scale d = amax / 127
    and 1 / d are checked well past the values activations take."""
    chunk = 7 << 22  # 768 * 38229 values
    step, k = 7, 768
    for start in range(0, 1 << 32, chunk * step):
        bits = np.arange(start, min(start + chunk * step, 1 << 32), step, dtype=np.uint64)
        rows = bits.size // k
        x = bits[:rows * k].astype(np.uint32).view(np.float32)
        got = rt.q8_0_download(rt.quantize_q8_0(rt.upload_f32(x), rows, k))
        exp = O.quantize_rows_q8_0(x, rows, k)
        ok = got.view(np.uint8).reshape(-1, 34) == np.asarray(exp).view(np.uint8).reshape(-1, 34)
        assert ok.all(), (start, np.nonzero(~ok.all(1))[0][:4])
