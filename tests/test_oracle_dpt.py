"""CPU pins of the DPT-head oracle (convolution, transposed convolution,
bilinear resize): the reference's own hand-checked cases and variant claims
(src/conv.rs and src/resample.rs test modules), plus float64 restatements of
the definitions, so that a wrong tap index, a transposed weight or a shifted
sampling grid fails."""
import numpy as np
import pytest

import oracle as O


def conv_f64(x, in_c, ih, iw, w, out_c, k, stride, pad, bias=None):
    """Direct convolution in float64 (independent of the oracle's loops)."""
    x = np.asarray(x, np.float64).reshape(in_c, ih, iw)
    w = np.asarray(w, np.float64).reshape(out_c, in_c, k, k)
    xp = np.zeros((in_c, ih + 2 * pad, iw + 2 * pad))
    xp[:, pad:pad + ih, pad:pad + iw] = x
    oh, ow = (ih + 2 * pad - k) // stride + 1, (iw + 2 * pad - k) // stride + 1
    out = np.zeros((out_c, oh, ow))
    for ky in range(k):
        for kx in range(k):
            patch = xp[:, ky:ky + stride * oh:stride, kx:kx + stride * ow:stride]
            out += np.einsum("oc,chw->ohw", w[:, :, ky, kx], patch)
    if bias is not None:
        out += np.asarray(bias, np.float64)[:, None, None]
    return out.reshape(-1)


def conv_t_f64(x, in_c, ih, iw, w, out_c, k, stride, bias=None):
    x = np.asarray(x, np.float64).reshape(in_c, ih, iw)
    w = np.asarray(w, np.float64).reshape(in_c, out_c, k, k)
    oh, ow = (ih - 1) * stride + k, (iw - 1) * stride + k
    out = np.zeros((out_c, oh, ow))
    for iy in range(ih):
        for ix in range(iw):
            out[:, iy * stride:iy * stride + k, ix * stride:ix * stride + k] += np.einsum(
                "c,cokl->okl", x[:, iy, ix], w)
    if bias is not None:
        out += np.asarray(bias, np.float64)[:, None, None]
    return out.reshape(-1)


def f32_bound(k_terms, absval):
    return (k_terms + 2) * 6e-8 * absval + 1e-30


# ---- the reference's hand-checked cases -----------------------------------------

def test_conv2d_1x1_hand_checked():
    """src/conv.rs:1107-1155."""
    x = np.arange(1, 13, dtype=np.float32)
    got = O.conv2d_naive(x, 3, 2, 2, [1, 0, 0, 0, 0, 1], 2, 1, 1, 1, 0, [10, -1])
    assert got.tolist() == [11, 12, 13, 14, 8, 9, 10, 11]


def test_conv_transpose2d_k4s4_hand_checked():
    """src/conv.rs:1248-1296: one input pixel, the output is the kernel."""
    w = np.zeros(2 * 2 * 16, np.float32)
    w[:16] = 1.0
    w[48:] = 5.0
    for fn in (O.conv_transpose2d, O.conv_transpose2d_naive):
        got = fn([2.0, 3.0], 2, 1, 1, w, 2, 4, 4, 4, [1.0, -2.0])
        assert got[:16].tolist() == [3.0] * 16 and got[16:].tolist() == [13.0] * 16


def test_bilinear_hand_checked():
    """src/resample.rs:250-287, 355-402."""
    ident = np.arange(1, 10, dtype=np.float32)
    assert np.array_equal(O.bilinear_resize(ident, 1, 3, 3, 3, 3), ident)
    assert np.array_equal(O.bilinear_resize_align_corners(ident, 1, 3, 3, 3, 3), ident)
    up = O.bilinear_resize([10.0, 20.0], 1, 1, 2, 1, 4)
    assert np.abs(up - [10.0, 12.5, 17.5, 20.0]).max() < 1e-6
    ac = O.bilinear_resize_align_corners([10.0, 20.0], 1, 1, 2, 1, 5)
    assert ac[0] == 10.0 and ac[4] == 20.0
    assert np.abs(ac - [10.0, 12.5, 15.0, 17.5, 20.0]).max() < 1e-6
    assert O.bilinear_resize_align_corners([5.0, 7.0, 9.0], 1, 1, 3, 1, 1).tolist() == [5.0]


def test_xorshift_generator_matches_definition():
    """The reference tests' data generator, against a direct u32 restatement."""
    x, vals = 0xABCD1234, []
    for _ in range(3):
        x ^= (x << 13) % 2**32
        x ^= x >> 17
        x ^= (x << 5) % 2**32
        vals.append(float(np.float32(np.float32(np.float32(x) / np.float32(2**32)) * 2) - 1))
    assert O.xorshift32_vec(0xABCD1234, 3).tolist() == [np.float32(v) for v in vals]


# ---- variant claims of the reference ---------------------------------------------

@pytest.mark.parametrize("c, ih, iw, oh, ow, seed", [(3, 5, 7, 9, 4, 0xABCD1234),
                                                     (2, 16, 16, 5, 5, 0x13579BDF),
                                                     (4, 24, 36, 96, 144, 7)])
def test_bilinear_tables_equal_per_element_form(c, ih, iw, oh, ow, seed):
    """src/resample.rs:289-328 claim 1e-5; both forms round the same ops, so
    they agree bit for bit."""
    x = O.xorshift32_vec(seed, c * ih * iw)
    a = O.bilinear_resize(x, c, ih, iw, oh, ow)
    b = O.bilinear_resize_naive(x, c, ih, iw, oh, ow)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_align_corners_differs_from_half_pixel():
    """src/resample.rs:404-424."""
    x = O.xorshift32_vec(0x2222AAAA, 2 * 16)
    a = O.bilinear_resize_align_corners(x, 2, 4, 4, 7, 5)
    b = O.bilinear_resize(x, 2, 4, 4, 7, 5)
    assert np.abs(a - b).max() > 1e-4


def test_nonoverlap_transpose_is_bitwise_serial_scatter():
    """src/conv.rs:1345-1388 (in_c = 3: the generic kernel == stride route)."""
    in_c, out_c, ih, iw, k = 3, 4, 3, 2, 2
    rng = O.xorshift32_vec(0x7A4E0001, in_c * ih * iw + in_c * out_c * k * k + out_c)
    x, w, b = rng[:18], rng[18:18 + 48], rng[66:]
    fast = O.conv_transpose2d(x, in_c, ih, iw, w, out_c, k, k, k, b)
    oh, ow = ih * k, iw * k
    serial = np.zeros(out_c * oh * ow, np.float32)
    for ic in range(in_c):
        for iy in range(ih):
            for ix in range(iw):
                iv = x[(ic * ih + iy) * iw + ix]
                for oc in range(out_c):
                    for ky in range(k):
                        for kx in range(k):
                            i = (oc * oh + iy * k + ky) * ow + ix * k + kx
                            serial[i] = np.float32(serial[i] + np.float32(
                                iv * w[((ic * out_c + oc) * k + ky) * k + kx]))
    for oc in range(out_c):
        serial[oc * oh * ow:(oc + 1) * oh * ow] += b[oc]
    assert np.array_equal(fast.view(np.uint32), serial.view(np.uint32))


@pytest.mark.parametrize("in_c, out_c, ih, iw, k, s", [(3, 2, 2, 3, 4, 4), (16, 8, 3, 5, 4, 4),
                                                        (5, 3, 4, 3, 3, 2)])
def test_conv_transpose_routes_match_naive(in_c, out_c, ih, iw, k, s):
    """src/conv.rs:1298-1343 (1e-4), for the generic, the AVX-512 non-overlap
    (in_c % 16 == 0) and the scatter routes."""
    n = in_c * ih * iw + in_c * out_c * k * k + out_c
    r = O.xorshift32_vec(0xFEED1234 + in_c, n)
    x, w, b = r[:in_c * ih * iw], r[in_c * ih * iw:n - out_c], r[n - out_c:]
    got = O.conv_transpose2d(x, in_c, ih, iw, w, out_c, k, k, s, b)
    nv = O.conv_transpose2d_naive(x, in_c, ih, iw, w, out_c, k, k, s, b)
    assert np.abs(got - nv).max() < 1e-4
    exact = conv_t_f64(x, in_c, ih, iw, w, out_c, k, s, b)
    absb = conv_t_f64(np.abs(x), in_c, ih, iw, np.abs(w), out_c, k, s, np.abs(b))
    assert np.all(np.abs(nv - exact) <= f32_bound(in_c * k * k, absb))


# ---- closed forms ----------------------------------------------------------------

@pytest.mark.parametrize("in_c, out_c, ih, iw, k, s, p", [(2, 3, 7, 5, 3, 2, 1), (5, 7, 4, 3, 1, 1, 0),
                                                          (3, 5, 7, 9, 3, 1, 1), (4, 2, 9, 6, 4, 4, 0)])
def test_conv2d_naive_is_the_definition(in_c, out_c, ih, iw, k, s, p):
    n = in_c * ih * iw + out_c * in_c * k * k + out_c
    r = O.xorshift32_vec(0xC0FFEE01 + k, n)
    x, w, b = r[:in_c * ih * iw], r[in_c * ih * iw:n - out_c], r[n - out_c:]
    got = O.conv2d_naive(x, in_c, ih, iw, w, out_c, k, k, s, p, b)
    exact = conv_f64(x, in_c, ih, iw, w, out_c, k, s, p, b)
    absb = conv_f64(np.abs(x), in_c, ih, iw, np.abs(w), out_c, k, s, p, np.abs(b))
    assert np.all(np.abs(got - exact) <= f32_bound(in_c * k * k, absb))
    # a transposed kernel (kx <-> ky) gives another result when k > 1
    if k > 1:
        wt = np.ascontiguousarray(w.reshape(out_c, in_c, k, k).transpose(0, 1, 3, 2)).reshape(-1)
        assert np.abs(O.conv2d_naive(x, in_c, ih, iw, wt, out_c, k, k, s, p, b) - got).max() > 1e-3


# ---- Winograd F(2x2, 3x3): the crate's CPU route for 3x3 stride-1 pad-1 -----------

def test_winograd_f2_matches_direct_oracle_reference_case():
    """src/conv.rs:1438-1477: in_c 3, out_c 5, 7 x 9, Xorshift32(0xF2F2_0001)
    drawing input, weight and bias in that order; |winograd - naive| < 2e-5."""
    in_c, out_c, h, w = 3, 5, 7, 9
    r = O.xorshift32_vec(0xF2F20001, in_c * h * w + out_c * in_c * 9 + out_c)
    x, wt, b = r[:in_c * h * w], r[in_c * h * w:-out_c], r[-out_c:]
    got = O.conv3x3_winograd_f2(x, in_c, h, w, wt, out_c, b)
    direct = O.conv2d_naive(x, in_c, h, w, wt, out_c, 3, 3, 1, 1, b)
    assert np.abs(got - direct).max() < 2e-5


@pytest.mark.parametrize("in_c, out_c, ih, iw", [(3, 5, 7, 9), (16, 32, 13, 11), (64, 32, 5, 4),
                                                 (96, 128, 24, 36), (1, 16, 1, 1)])
def test_winograd_f2_is_the_convolution(in_c, out_c, ih, iw):
    """Against the float64 definition within the f32 accumulation bound, at odd
    sizes (edge tiles half outside the image) and DPT shapes; the transposed
    kernel (kx <-> ky) must miss, so a swapped transform index cannot pass."""
    n = in_c * ih * iw + out_c * in_c * 9 + out_c
    r = O.xorshift32_vec(0xF2F2 + in_c + ih, n)
    x, w, b = r[:in_c * ih * iw], r[in_c * ih * iw:n - out_c], r[n - out_c:]
    w = w * np.float32(1.0 / np.sqrt(in_c * 9))
    got = O.conv3x3_winograd_f2(x, in_c, ih, iw, w, out_c, b)
    exact = conv_f64(x, in_c, ih, iw, w, out_c, 3, 1, 1, b)
    absb = conv_f64(np.abs(x), in_c, ih, iw, np.abs(w), out_c, 3, 1, 1, np.abs(b))
    assert np.all(np.abs(got - exact) <= f32_bound(in_c * 9 + 16, absb))
    wt = np.ascontiguousarray(w.reshape(out_c, in_c, 3, 3).transpose(0, 1, 3, 2)).reshape(-1)
    if ih > 1 and iw > 1:
        assert np.abs(O.conv3x3_winograd_f2(x, in_c, ih, iw, wt, out_c, b) - got).max() > 1e-3


def test_winograd_f2_filter_is_g_g_gt():
    """U = G g G^T per (oc, ic), stored [position][ic][oc]."""
    in_c, out_c = 3, 2
    w = O.xorshift32_vec(0xF117, out_c * in_c * 9)
    u = O.winograd_f2_filter(w, in_c, out_c).reshape(16, in_c, out_c)
    G = np.array([[1, 0, 0], [0.5, 0.5, 0.5], [0.5, -0.5, 0.5], [0, 0, 1]])
    g = np.asarray(w, np.float64).reshape(out_c, in_c, 3, 3)
    for oc in range(out_c):
        for ic in range(in_c):
            exp = (G @ g[oc, ic] @ G.T).reshape(16)
            assert np.abs(u[:, ic, oc] - exp).max() <= 4e-7 * (np.abs(g[oc, ic]).sum() + 1e-30)


@pytest.mark.skipif(not O.has_avx512(), reason="host without AVX-512")
def test_winograd_f2_avx512_product_is_its_lane_restatement():
    """The AVX-512 product (one FMA chain per lane over the input channels)
    equals its fmaf restatement bit for bit, edge tiles and a partial last
    tile block included."""
    in_c, out_c, ih, iw = 48, 32, 9, 13
    x = O.xorshift32_vec(0xA5, in_c * ih * iw)
    w = O.xorshift32_vec(0xA6, out_c * in_c * 9)
    b = O.xorshift32_vec(0xA7, out_c)
    u = O.winograd_f2_filter(w, in_c, out_c)
    a = O.conv3x3_winograd_f2(x, in_c, ih, iw, None, out_c, b, u=u)
    lanes = O.conv3x3_winograd_f2(x, in_c, ih, iw, None, out_c, b, u=u, lanes=True)
    assert np.array_equal(a.view(np.uint32), lanes.view(np.uint32))


def test_winograd_f2_scalar_tier_is_the_convolution():
    """The crate's scalar product (unfused sums, src/conv.rs:775-788), taken
    on hosts without AVX-512 and for out_c % 16 != 0."""
    in_c, out_c, ih, iw = 8, 16, 6, 7
    n = in_c * ih * iw + out_c * in_c * 9 + out_c
    r = O.xorshift32_vec(0x5CA1, n)
    x, w, b = r[:in_c * ih * iw], r[in_c * ih * iw:n - out_c], r[n - out_c:]
    O.force_scalar(True)
    try:
        got = O.conv3x3_winograd_f2(x, in_c, ih, iw, w, out_c, b)
    finally:
        O.force_scalar(False)
    exact = conv_f64(x, in_c, ih, iw, w, out_c, 3, 1, 1, b)
    absb = conv_f64(np.abs(x), in_c, ih, iw, np.abs(w), out_c, 3, 1, 1, np.abs(b))
    assert np.all(np.abs(got - exact) <= f32_bound(in_c * 9 + 16, absb))


def test_winograd_relu_input_equals_materialised_relu_bitwise():
    """src/conv.rs:1479-1519: ReLU applied while loading the patches gives the
    bits of the convolution of the materialised ReLU."""
    in_c, out_c, h, w = 3, 5, 7, 9
    i = np.arange(in_c * h * w, dtype=np.float32)
    x = ((np.sin(i * np.float32(0.17)) - np.float32(0.4)) * np.float32(1.3)).astype(np.float32)
    wt = (np.cos(np.arange(out_c * in_c * 9, dtype=np.float32) * np.float32(0.11))
          * np.float32(0.2)).astype(np.float32)
    b = (np.arange(out_c, dtype=np.float32) * np.float32(0.03) - np.float32(0.05)).astype(np.float32)
    expected = O.conv3x3_winograd_f2(np.maximum(x, 0), in_c, h, w, wt, out_c, b)
    actual = O.conv3x3_winograd_f2(x, in_c, h, w, wt, out_c, b, relu_input=True)
    assert np.array_equal(actual.view(np.uint32), expected.view(np.uint32))


def bilinear_f64(x, c, ih, iw, oh, ow, align):
    """The sampling definitions in float64: half-pixel src = (d+0.5)*in/out - 0.5
    clamped to the edge; align-corners src = d*(in-1)/(out-1)."""
    x = np.asarray(x, np.float64).reshape(c, ih, iw)

    def taps(n_in, n_out):
        d = np.arange(n_out, dtype=np.float64)
        if align:
            src = d * (n_in - 1) / (n_out - 1) if n_out > 1 else np.zeros(n_out)
        else:
            src = np.maximum((d + 0.5) * n_in / n_out - 0.5, 0.0)
        i0 = np.minimum(np.floor(src).astype(int), n_in - 1)
        i1 = np.minimum(i0 + 1, n_in - 1)
        f = np.where(i1 == i0, 0.0, np.clip(src - i0, 0, 1))
        return i0, i1, f
    y0, y1, fy = taps(ih, oh)
    x0, x1, fx = taps(iw, ow)
    top = x[:, y0][:, :, x0] * (1 - fx) + x[:, y0][:, :, x1] * fx
    bot = x[:, y1][:, :, x0] * (1 - fx) + x[:, y1][:, :, x1] * fx
    return (top * (1 - fy)[None, :, None] + bot * fy[None, :, None]).reshape(-1)


@pytest.mark.parametrize("align", [False, True])
@pytest.mark.parametrize("c, ih, iw, oh, ow", [(3, 5, 7, 9, 4), (2, 12, 18, 48, 72), (1, 7, 3, 2, 11)])
def test_bilinear_is_the_sampling_definition(align, c, ih, iw, oh, ow):
    x = O.xorshift32_vec(99 + ih, c * ih * iw)
    fn = O.bilinear_resize_align_corners if align else O.bilinear_resize
    got = fn(x, c, ih, iw, oh, ow)
    # The f32 source coordinate carries a few ulps of max(ih, iw); its error
    # times the neighbour difference (|x| <= 1) bounds the deviation.  A
    # wrong formula (no -0.5, a swapped axis) moves values by ~0.1.
    tol = 4 * 2.0**-23 * max(ih, iw) * 2 + 1e-6
    assert np.abs(got - bilinear_f64(x, c, ih, iw, oh, ow, align)).max() <= tol
