"""GPU parity of the DPT-head operations (convolution, transposed
convolution, bilinear resize) through the C ABI.

Convolutions run as fp32-MFMA GEMMs, so they are held to the f32
accumulation bound against the crate's direct oracle: |gpu - naive| <=
(K + 2) * 6e-8 * sum|x||w| per output (K taps).  The gather-form transposed
convolution and the resizes restate the reference's op order and are
bit-exact.  3x3 stride-1 convolutions are also compared with the crate's own
CPU route for them, Winograd F(2x2, 3x3).  The fused variants (ReLU input,
resize + add + conv) are checked bit for bit against their materialised
routes, as the crate's own tests do (src/conv.rs:1479-1600)."""
import numpy as np
import pytest

import oracle as O
import vestra_hip as vh
from conftest import assert_bits_equal, max_rel

pytestmark = pytest.mark.gpu


def _data(seed, *sizes):
    r = O.xorshift32_vec(seed, sum(sizes))
    out, o = [], 0
    for n in sizes:
        out.append(r[o:o + n])
        o += n
    return out


def _conv_bound(x, in_c, ih, iw, w, out_c, k, s, p, b):
    absb = O.conv2d_naive(np.abs(x), in_c, ih, iw, np.abs(w), out_c, k, k, s, p,
                          None if b is None else np.abs(b))
    return (in_c * k * k + 2) * 6e-8 * absb.astype(np.float64) + 1e-30


CONV_CASES = [
    # in_c, out_c, ih, iw, k, stride, pad
    (3, 2, 2, 2, 1, 1, 0),
    (5, 7, 4, 3, 1, 1, 0),
    (2, 3, 7, 5, 3, 2, 1),
    (16, 16, 7, 9, 3, 1, 1),
    (96, 128, 24, 36, 3, 1, 1),      # DPT layer_rn at the 24 x 36 grid
    (768, 96, 24, 36, 1, 1, 0),      # DPT projection
    (768, 768, 24, 36, 3, 2, 1),     # DPT resize layer 4 (3x3, stride 2)
    (768, 128, 12, 18, 3, 1, 1),     # DPT layer_rn at 12 x 18: 8 tiles, K split 27 ways
    (384, 128, 24, 36, 3, 1, 1),     # DPT layer_rn at 24 x 36: 28 tiles, K split 9 ways
    (64, 32, 48, 72, 3, 1, 1),       # head convolution
    (3, 4, 10, 11, 5, 3, 2),
    (32, 16, 9, 11, 5, 1, 2),        # implicit GEMM, 5x5 taps, 4 junk columns per row
    (64, 8, 7, 7, 3, 1, 0),          # implicit GEMM without padding
    (96, 40, 13, 5, 1, 1, 1),        # implicit GEMM, 1x1 with padding
]


@pytest.mark.parametrize("in_c, out_c, ih, iw, k, s, p", CONV_CASES)
def test_conv2d_vs_naive(rt, in_c, out_c, ih, iw, k, s, p):
    x, w, b = _data(0xC0FFEE01 + in_c + k, in_c * ih * iw, out_c * in_c * k * k, out_c)
    w = w * np.float32(1.0 / np.sqrt(in_c * k * k))
    conv = rt.prepare_conv2d_f32(in_c, out_c, k, k, s, p, w, b)
    oh, ow = conv.output_hw(ih, iw)
    assert (oh, ow) == O.conv_out_hw(ih, iw, k, k, s, p)
    got = rt.download_f32(conv.run(rt.upload_f32(x), ih, iw))
    exp = O.conv2d_naive(x, in_c, ih, iw, w, out_c, k, k, s, p, b)
    assert np.all(np.abs(got.astype(np.float64) - exp) <= _conv_bound(x, in_c, ih, iw, w, out_c, k, s, p, b))


@pytest.mark.parametrize("in_c, out_c, ih, iw", [(96, 128, 24, 36), (64, 32, 48, 72),
                                                 (128, 128, 96, 144), (16, 16, 7, 9)])
def test_conv3x3_vs_crate_winograd(rt, in_c, out_c, ih, iw):
    """The crate computes 3x3 stride-1 pad-1 convolutions with Winograd F(2x2,
    3x3) (conv::conv2d, src/conv.rs:897-900), not with the direct sum.  The
    device's direct convolution and that route each hold the f32 accumulation
    bound of the exact convolution (the oracle's Winograd is pinned to it on
    the CPU), so they agree within twice the bound."""
    x, w, b = _data(0xF2F2A000 + in_c + ih, in_c * ih * iw, out_c * in_c * 9, out_c)
    w = w * np.float32(1.0 / np.sqrt(in_c * 9))
    conv = rt.prepare_conv2d_f32(in_c, out_c, 3, 3, 1, 1, w, b)
    got = rt.download_f32(conv.run(rt.upload_f32(x), ih, iw))
    wino = O.conv3x3_winograd_f2(x, in_c, ih, iw, w, out_c, b)
    bound = 2 * _conv_bound(x, in_c, ih, iw, w, out_c, 3, 1, 1, b)
    assert np.all(np.abs(got.astype(np.float64) - wino) <= bound)


def test_conv2d_hand_checked_and_one_shot(rt):
    """src/conv.rs:1107-1155; the one-call form equals the prepared form."""
    x = rt.upload_f32(np.arange(1, 13, dtype=np.float32))
    got = rt.download_f32(rt.conv2d_f32(x, 3, 2, 2, [1, 0, 0, 0, 0, 1], 2, 1, 1, 1, 0, [10, -1]))
    assert got.tolist() == [11, 12, 13, 14, 8, 9, 10, 11]
    xs, w = _data(5, 4 * 9 * 9, 6 * 4 * 9)
    a = rt.download_f32(rt.conv2d_f32(rt.upload_f32(xs), 4, 9, 9, w, 6, 3, 3, 1, 1))
    c = rt.prepare_conv2d_f32(4, 6, 3, 3, 1, 1, w)
    assert_bits_equal(a, rt.download_f32(c.run(rt.upload_f32(xs), 9, 9)), "one-shot vs prepared")


@pytest.mark.parametrize("in_c, out_c, ih, iw, k, s, p", [c for c in CONV_CASES if c[0] % 32 == 0])
def test_conv2d_direct_matches_staged(rt, monkeypatch, in_c, out_c, ih, iw, k, s, p):
    """The direct implicit GEMM (CHW image read in place) against the staged
    forms (padded channel-last copy, patch matrix, transposes): with whole
    tiles (the GEMM's balanced tail off) they take the same products in the
    same k order, so stride-1 shapes agree bit for bit; the staged stride-2
    form splits K and agrees to rounding.  By default a staged GEMM with
    fewer tiles than CUs runs its tiles as K pieces (the 1x1 768 -> 96
    convolution: 28 tiles), which also agrees to rounding."""
    x, w, b = _data(0xD1EC7 + in_c + k, in_c * ih * iw, out_c * in_c * k * k, out_c)
    w = w * np.float32(1.0 / np.sqrt(in_c * k * k))
    conv = rt.prepare_conv2d_f32(in_c, out_c, k, k, s, p, w, b)
    xt = rt.upload_f32(x)
    outs = {}
    for direct, tail in (("1", "0"), ("0", "0"), ("0", None)):
        monkeypatch.setenv("VESTRA_HIP_CONV_DIRECT", direct)
        if tail is None:
            monkeypatch.delenv("VESTRA_HIP_GEMM_TAIL", raising=False)
        else:
            monkeypatch.setenv("VESTRA_HIP_GEMM_TAIL", tail)
        outs[(direct, tail)] = (rt.download_f32(conv.run(xt, ih, iw)),
                                rt.download_f32(conv.run_relu_input(xt, ih, iw)))
    for a, b_, t in zip(outs[("1", "0")], outs[("0", "0")], outs[("0", None)]):
        if s == 1:
            assert_bits_equal(a, b_, "direct vs staged convolution")
        else:
            assert max_rel(a, b_) <= 1e-5
        assert max_rel(a, t) <= 1e-5


# direct implicit GEMM (256: its 8 tiles split K 18 ways) / channel-last patch copy
@pytest.mark.parametrize("in_c", [32, 256, 12])
def test_conv2d_relu_input_equals_materialised_relu(rt, in_c):
    """src/conv.rs:1479-1520, on the device."""
    out_c, h, w_ = 24, 18, 27
    x, w, b = _data(11, in_c * h * w_, out_c * in_c * 9, out_c)
    conv = rt.prepare_conv2d_f32(in_c, out_c, 3, 3, 1, 1, w, b)
    fused = rt.download_f32(conv.run_relu_input(rt.upload_f32(x), h, w_))
    mat = rt.download_f32(conv.run(rt.upload_f32(np.maximum(x, 0)), h, w_))
    assert_bits_equal(fused, mat, "relu input")


def test_conv2d_resize_add_equals_materialised_route(rt):
    """src/conv.rs:1522-1580: resize (align corners), + add, then the conv."""
    in_c, out_c, ih, iw, oh, ow = 16, 16, 7, 5, 11, 9
    x, add, w, b = _data(0xF05E0001, in_c * ih * iw, in_c * oh * ow, out_c * in_c * 9, out_c)
    conv = rt.prepare_conv2d_f32(in_c, out_c, 3, 3, 1, 1, w, b)
    fused = rt.download_f32(conv.run_resize_align_corners(rt.upload_f32(x), ih, iw, oh, ow,
                                                          rt.upload_f32(add)))
    resized = rt.bilinear_resize_align_corners_f32(rt.upload_f32(x), in_c, ih, iw, oh, ow,
                                                   rt.upload_f32(add))
    assert_bits_equal(rt.download_f32(resized),
                      O.bilinear_resize_align_corners(x, in_c, ih, iw, oh, ow) + add, "resize + add")
    mat = rt.download_f32(conv.run(resized, oh, ow))
    assert_bits_equal(fused, mat, "fused resize route")


@pytest.mark.parametrize("in_c, out_c, ih, iw, k", [
    (96, 96, 24, 36, 4),    # DA3 k4s4: patch-scatter GEMM, 16-byte stores
    (192, 192, 24, 36, 2),  # k2s2: patch-scatter GEMM, element stores
    (32, 5, 7, 9, 4),       # 80 weight rows: a partial row tile, 63 pixels
    (64, 3, 5, 6, 2),       # 12 weight rows
    (32, 7, 4, 5, 3),       # k3s3: rows do not align to (oc, ky) groups of 4
    (3, 4, 3, 2, 2),        # in_c % 32 != 0: GEMM into a staging buffer, then the scatter
    (16, 8, 3, 5, 4)])
def test_conv_transpose_nonoverlap_vs_naive(rt, in_c, out_c, ih, iw, k):
    x, w, b = _data(0xFEED1234 + in_c, in_c * ih * iw, in_c * out_c * k * k, out_c)
    ct = rt.prepare_conv_transpose2d_f32(in_c, out_c, k, k, k, w, b)
    got = rt.download_f32(ct.run(rt.upload_f32(x), ih, iw))
    exp = O.conv_transpose2d_naive(x, in_c, ih, iw, w, out_c, k, k, k, b)
    absb = O.conv_transpose2d_naive(np.abs(x), in_c, ih, iw, np.abs(w), out_c, k, k, k, np.abs(b))
    assert np.all(np.abs(got.astype(np.float64) - exp) <= (in_c + 2) * 6e-8 * absb + 1e-30)
    ref_main = O.conv_transpose2d(x, in_c, ih, iw, w, out_c, k, k, k, b)
    assert np.abs(got - ref_main).max() < 1e-4


@pytest.mark.parametrize("in_c, out_c, ih, iw, k", [
    (96, 96, 24, 36, 4), (192, 192, 24, 36, 2), (32, 5, 7, 9, 4), (32, 7, 4, 5, 3)])
def test_conv_transpose_chw_read_equals_channel_last_copy(rt, monkeypatch, in_c, out_c, ih, iw, k):
    """The patch-scatter GEMM reading the CHW input in place (the default)
    against the same GEMM over a channel-last copy (VESTRA_HIP_CONV_DIRECT=0):
    the same products in the same k order, so the same bits, including the
    partial last pixel tile (63 and 20 pixels)."""
    x, w, b = _data(0xC7A0 + in_c + k, in_c * ih * iw, in_c * out_c * k * k, out_c)
    ct = rt.prepare_conv_transpose2d_f32(in_c, out_c, k, k, k, w, b)
    xt = rt.upload_f32(x)
    monkeypatch.setenv("VESTRA_HIP_CONV_DIRECT", "0")
    staged = rt.download_f32(ct.run(xt, ih, iw))
    monkeypatch.setenv("VESTRA_HIP_CONV_DIRECT", "1")
    direct = rt.download_f32(ct.run(xt, ih, iw))
    assert_bits_equal(direct, staged, f"transposed conv {in_c}->{out_c} k{k} from CHW")


def test_conv_transpose_k4s4_hand_checked(rt):
    """src/conv.rs:1248-1296."""
    w = np.zeros(64, np.float32)
    w[:16] = 1.0
    w[48:] = 5.0
    got = rt.download_f32(rt.conv_transpose2d_f32(rt.upload_f32([2.0, 3.0]), 2, 1, 1, w, 2, 4, 4,
                                                  4, [1.0, -2.0]))
    assert got[:16].tolist() == [3.0] * 16 and got[16:].tolist() == [13.0] * 16


@pytest.mark.parametrize("in_c, out_c, ih, iw, k, s, bias", [(5, 3, 4, 3, 3, 2, True),
                                                              (8, 6, 9, 7, 5, 2, False),
                                                              (4, 4, 6, 6, 2, 3, True)])
def test_conv_transpose_general_bit_exact_with_gather_oracle(rt, in_c, out_c, ih, iw, k, s, bias):
    x, w, b = _data(77 + k, in_c * ih * iw, in_c * out_c * k * k, out_c)
    b = b if bias else None
    got = rt.download_f32(rt.conv_transpose2d_f32(rt.upload_f32(x), in_c, ih, iw, w, out_c, k, k,
                                                  s, b))
    assert_bits_equal(got, O.conv_transpose2d_naive(x, in_c, ih, iw, w, out_c, k, k, s, b),
                      "gather transposed conv")


RESIZE_CASES = [(3, 5, 7, 9, 4), (2, 16, 16, 5, 5), (1, 1, 2, 1, 4), (1, 1, 2, 1, 5),
                (1, 1, 3, 1, 1), (4, 24, 36, 96, 144), (128, 48, 72, 96, 144), (1, 3, 3, 3, 3),
                (2, 1, 1, 4, 6)]


@pytest.mark.parametrize("c, ih, iw, oh, ow", RESIZE_CASES)
def test_bilinear_bit_exact(rt, c, ih, iw, oh, ow):
    x = O.xorshift32_vec(0xABCD1234 + oh, c * ih * iw)
    xt = rt.upload_f32(x)
    assert_bits_equal(rt.download_f32(rt.bilinear_resize_f32(xt, c, ih, iw, oh, ow)),
                      O.bilinear_resize(x, c, ih, iw, oh, ow), "half-pixel")
    assert_bits_equal(rt.download_f32(rt.bilinear_resize_align_corners_f32(xt, c, ih, iw, oh, ow)),
                      O.bilinear_resize_align_corners(x, c, ih, iw, oh, ow), "align corners")


def test_dpt_errors_before_launch(rt):
    x = rt.upload_f32(np.zeros(12, np.float32))
    with pytest.raises(vh.KernelError):
        rt.prepare_conv2d_f32(3, 2, 1, 1, 0, 0, np.zeros(6, np.float32))
    conv = rt.prepare_conv2d_f32(3, 2, 3, 3, 1, 0, np.zeros(54, np.float32))
    with pytest.raises(vh.LengthMismatch):
        conv.run(x, 3, 3)
    with pytest.raises(vh.KernelError):
        conv.run(x, 2, 2)  # 3x3 kernel on an unpadded 2x2 input
    with pytest.raises(vh.LengthMismatch):
        rt.bilinear_resize_f32(x, 3, 2, 3, 4, 4)
    empty = rt.bilinear_resize_f32(rt.upload_f32(np.zeros(0, np.float32)), 2, 0, 3, 2, 2)
    assert rt.download_f32(empty).tolist() == [0.0] * 8
