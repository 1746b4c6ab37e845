"""TEST INFRASTRUCTURE ONLY: numpy/ctypes front end of the CPU oracle.

The oracle (``oracle/vk_oracle.c``) restates hoppworks/vestra-kernels'
scalar and AVX-512 kernels op for op; every wrapper names the reference
function it stands for.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module; the HIP product
path never does.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
# VKO_ORACLE_LIB selects another build of the same sources (the sanitizer
# build of `make -C oracle asan`); the default is the plain build.
_LIB_PATH = Path(os.environ.get("VKO_ORACLE_LIB") or _HERE / "libvk_oracle.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_i64p = ctypes.POINTER(ctypes.c_int64)
_sz = ctypes.c_size_t

# numpy dtype identical to the reference's #[repr(C)] BlockQ8_0 (src/lib.rs:33-38).
BLOCK_Q8_0 = np.dtype([("d", "<u2"), ("qs", "i1", (32,))], align=False)
assert BLOCK_Q8_0.itemsize == 34

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run __graft_entry__.build())")
        _lib = ctypes.CDLL(str(_LIB_PATH))
        _declare(_lib)
    return _lib


def _declare(L):
    def sig(name, res, *args):
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = list(args)

    vp = ctypes.c_void_p
    sig("vko_has_avx512", ctypes.c_int)
    sig("vko_set_threads", None, ctypes.c_int)
    sig("vko_force_scalar", None, ctypes.c_int)
    sig("vko_f16_sweep", ctypes.c_uint64, ctypes.c_uint32)
    sig("vko_get_threads", ctypes.c_int)
    sig("vko_rust_max", ctypes.c_float, ctypes.c_float, ctypes.c_float)
    sig("vko_f32_to_f16", ctypes.c_uint16, ctypes.c_float)
    sig("vko_f16_to_f32", ctypes.c_float, ctypes.c_uint16)
    sig("vko_f32_to_f16_hw", ctypes.c_uint16, ctypes.c_float)
    sig("vko_gemm_f32", None, _sz, _sz, _sz, _f32p, _f32p, _f32p)
    sig("vko_gemm_q8_0", None, _sz, _sz, _sz, vp, vp, _f32p)
    sig("vko_gemm_q8_0_avx512", None, _sz, _sz, _sz, vp, vp, _f32p)
    sig("vko_kernels_gemm_q8_0", None, _sz, _sz, _sz, vp, vp, _f32p)
    sig("vko_add", None, _f32p, _f32p, _sz)
    sig("vko_add_bias_rows", None, _f32p, _sz, _sz, _f32p)
    sig("vko_layernorm", None, _f32p, _sz, _sz, _f32p, _f32p, ctypes.c_float)
    sig("vko_erf", ctypes.c_float, ctypes.c_float)
    sig("vko_cephes_exp", ctypes.c_float, ctypes.c_float)
    sig("vko_gelu", None, _f32p, _sz)
    sig("vko_gelu_avx512", None, _f32p, _sz)
    sig("vko_gelu_avx512_lanes", None, _f32p, _sz)
    sig("vko_kernels_gelu", None, _f32p, _sz)
    sig("vko_kernels_add", None, _f32p, _f32p, _sz)
    sig("vko_layerscale", None, _f32p, _sz, _sz, _f32p)
    sig("vko_softmax_rows", None, _f32p, _sz, _sz)
    sig("vko_quantize_row_q8_0", None, _f32p, _sz, vp)
    sig("vko_dequantize_q8_0", None, vp, _sz, _f32p)
    sig("vko_rope2d", None, _f32p, _sz, _sz, _sz, _i64p, ctypes.c_float)
    sig("vko_rope_rotations", None, _i64p, _sz, ctypes.c_float, _f32p)
    sig("vko_qk_norm_rope", None, _f32p, _f32p, _sz, _sz, _f32p, _f32p, _f32p, _f32p, _i64p,
        ctypes.c_float, ctypes.c_float)
    for name in ("vko_attention_naive", "vko_attention_serial", "vko_attention"):
        sig(name, None, _f32p, _f32p, _f32p, _sz, _sz, _sz, _f32p)
    sig("vko_flash_attention_scalar", None, _f32p, _f32p, _f32p, _sz, _sz, _f32p)
    sig("vko_flash_attention_avx512", ctypes.c_int, _f32p, _f32p, _f32p, _sz, _sz, _f32p)
    sig("vko_linear_fma_scalar", None, _sz, _sz, _sz, _f32p, _f32p, _f32p)
    sig("vko_linear", None, _sz, _sz, _sz, _f32p, _f32p, _f32p)
    sig("vko_linear_bias_scale", None, _sz, _sz, _sz, _f32p, _f32p, _f32p, _f32p, _f32p)
    sig("vko_qkv", None, _sz, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p)
    sig("vko_split_qkv_hnd", None, _f32p, _sz, _sz, _sz, _f32p, _f32p, _f32p)
    sig("vko_hnd_to_token", None, _f32p, _sz, _sz, _sz, _f32p)
    sig("vko_conv2d_naive", None, _f32p, _sz, _sz, _sz, _f32p, _sz, _sz, _sz, _sz, _sz, _f32p,
        _f32p)
    sig("vko_expf_glibc_form", ctypes.c_float, ctypes.c_float)
    sig("vko_exp2f_table_entry", ctypes.c_uint64, ctypes.c_int)
    sig("vko_expf_form_mismatches", ctypes.c_uint64, ctypes.c_uint32)
    sig("vko_winograd_f2_filter", None, _f32p, _sz, _sz, _f32p)
    sig("vko_conv3x3_winograd_f2", None, _f32p, _sz, _sz, _sz, _f32p, _sz, _f32p, ctypes.c_int,
        _f32p)
    sig("vko_winograd_use_lanes", None, ctypes.c_int)
    for name in ("vko_conv_transpose2d", "vko_conv_transpose2d_naive"):
        sig(name, None, _f32p, _sz, _sz, _sz, _f32p, _sz, _sz, _sz, _sz, _f32p, _f32p)
    for name in ("vko_bilinear_resize", "vko_bilinear_resize_naive",
                 "vko_bilinear_resize_align_corners"):
        sig(name, None, _f32p, _sz, _sz, _sz, _sz, _sz, _f32p)
    for name in ("vko_vit_block", "vko_vit_block_q8_0"):
        sig(name, None, _f32p, _sz, _sz, ctypes.POINTER(BlockWeights), _i64p,
            ctypes.c_float, ctypes.c_float, _f32p, _f32p, _f32p)


class BlockWeights(ctypes.Structure):
    _fields_ = [(n, _f32p) for n in (
        "ln1_gamma", "ln1_beta", "w_qkv", "b_qkv", "w_proj", "b_proj", "ls1",
        "ln2_gamma", "ln2_beta", "w_fc1", "b_fc1", "w_fc2", "b_fc2", "ls2",
        "q_norm_gamma", "q_norm_beta", "k_norm_gamma", "k_norm_beta")]


# DA3 late-block Q/K LayerNorm parameters: optional (absent -> plain block).
QK_NORM_FIELDS = ["q_norm_gamma", "q_norm_beta", "k_norm_gamma", "k_norm_beta"]


def _f(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_f32p)


def _i(a: np.ndarray):
    assert a.dtype == np.int64 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_i64p)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def has_avx512() -> bool:
    return bool(lib().vko_has_avx512())


def force_scalar(on: bool) -> None:
    """Take the reference's scalar (non-AVX-512) dispatch arms."""
    lib().vko_force_scalar(1 if on else 0)


def f16_sweep(step: int = 1) -> int:
    """Mismatches of the software f16 conversions against F16C."""
    return int(lib().vko_f16_sweep(step))


def rust_max(a: float, b: float) -> float:
    """f32::max as the oracle restates it (any NaN operand is ignored)."""
    return float(lib().vko_rust_max(ctypes.c_float(a), ctypes.c_float(b)))


def set_threads(n: int) -> None:
    lib().vko_set_threads(int(n))


def threads() -> int:
    return int(lib().vko_get_threads())


# ---- f16 -----------------------------------------------------------------
def f32_to_f16(x: float) -> int:
    return int(lib().vko_f32_to_f16(ctypes.c_float(x)))


def f16_to_f32(h: int) -> float:
    return float(lib().vko_f16_to_f32(ctypes.c_uint16(h)))


# ---- scalar.rs -------------------------------------------------------------
def gemm_f32(a, b, m, n, k):
    """scalar::gemm_f32 (src/scalar.rs:3-18)."""
    a, b = f32(a), f32(b)
    c = np.empty(m * n, np.float32)
    lib().vko_gemm_f32(m, n, k, _f(a), _f(b), _f(c))
    return c


def add(dst, src):
    """scalar::add (src/scalar.rs:58-63); returns the updated copy."""
    d = f32(dst).copy()
    lib().vko_add(_f(d), _f(f32(src)), d.size)
    return d


def add_bias_rows(x, rows, cols, bias):
    d = f32(x).copy()
    lib().vko_add_bias_rows(_f(d), rows, cols, _f(f32(bias)))
    return d


def layernorm(x, rows, cols, gamma, beta, eps):
    """scalar::layernorm (src/scalar.rs:83-114)."""
    d = f32(x).copy()
    lib().vko_layernorm(_f(d), rows, cols, _f(f32(gamma)), _f(f32(beta)), eps)
    return d


def erf(x: float) -> float:
    return float(lib().vko_erf(ctypes.c_float(x)))


def cephes_exp(x: float) -> float:
    """The AVX-512 Cephes exp (src/simd_avx512.rs:22-69), one lane."""
    return float(lib().vko_cephes_exp(ctypes.c_float(x)))


def gelu(x):
    """scalar::gelu (src/scalar.rs:116-134)."""
    d = f32(x).copy()
    lib().vko_gelu(_f(d), d.size)
    return d


def gelu_avx512(x):
    d = f32(x).copy()
    lib().vko_gelu_avx512(_f(d), d.size)
    return d


def gelu_avx512_lanes(x):
    """gelu_avx512 arithmetic in scalar code (any host); n%16 tail scalar::gelu."""
    d = f32(x).copy()
    lib().vko_gelu_avx512_lanes(_f(d), d.size)
    return d


def kernels_gelu(x):
    """Kernels::gelu (src/dispatch.rs:56-73)."""
    d = f32(x).copy()
    lib().vko_kernels_gelu(_f(d), d.size)
    return d


def kernels_add(dst, src):
    d = f32(dst).copy()
    lib().vko_kernels_add(_f(d), _f(f32(src)), d.size)
    return d


def layerscale(x, rows, cols, gamma):
    d = f32(x).copy()
    lib().vko_layerscale(_f(d), rows, cols, _f(f32(gamma)))
    return d


def softmax_rows(x, rows, cols):
    d = f32(x).copy()
    lib().vko_softmax_rows(_f(d), rows, cols)
    return d


# ---- Q8_0 ------------------------------------------------------------------
def quantize_rows_q8_0(x, rows, k):
    """quantize_row_q8_0 (src/q8_0_dot.rs:27-46) applied to each row."""
    x = f32(x).reshape(rows, k)
    out = np.zeros(rows * (k // 32), BLOCK_Q8_0)
    lib().vko_quantize_row_q8_0(_f(np.ascontiguousarray(x)), out.size, out.ctypes.data)
    return out


def dequantize_q8_0(blocks):
    blocks = np.ascontiguousarray(blocks, BLOCK_Q8_0)
    out = np.empty(blocks.size * 32, np.float32)
    lib().vko_dequantize_q8_0(blocks.ctypes.data, blocks.size, _f(out))
    return out


def gemm_q8_0(a_q, b_q, m, n, k, impl="scalar"):
    """scalar::gemm_q8_0 (src/scalar.rs:25-56) / gemm_q8_0_avx512 (src/simd_avx512.rs:295)."""
    a_q = np.ascontiguousarray(a_q, BLOCK_Q8_0)
    b_q = np.ascontiguousarray(b_q, BLOCK_Q8_0)
    c = np.empty(m * n, np.float32)
    fn = {"scalar": lib().vko_gemm_q8_0, "avx512": lib().vko_gemm_q8_0_avx512,
          "kernels": lib().vko_kernels_gemm_q8_0}[impl]
    fn(m, n, k, a_q.ctypes.data, b_q.ctypes.data, _f(c))
    return c


# ---- RoPE ------------------------------------------------------------------
def rope2d(x, heads, n, head_dim, pos_yx, freq):
    """rope::rope2d (src/rope.rs:30-80)."""
    d = f32(x).copy()
    pos = np.ascontiguousarray(pos_yx, np.int64)
    lib().vko_rope2d(_f(d), heads, n, head_dim, _i(pos), freq)
    return d


def rope_rotations(pos_yx, tokens, freq):
    """rope_rotations (src/specialized.rs:389-410): [tokens, 2, 16, (sin, cos)]."""
    pos = np.ascontiguousarray(pos_yx, np.int64)
    rot = np.empty(tokens * 64, np.float32)
    lib().vko_rope_rotations(_i(pos), tokens, freq, _f(rot))
    return rot


def qk_norm_rope(q, k, heads, tokens, qg, qb, kg, kb, pos_yx, freq, eps):
    """qk_norm_rope_f32_da3_base arithmetic (src/specialized.rs:278-454)."""
    q2, k2 = f32(q).copy(), f32(k).copy()
    pos = np.ascontiguousarray(pos_yx, np.int64)
    lib().vko_qk_norm_rope(_f(q2), _f(k2), heads, tokens, _f(f32(qg)), _f(f32(qb)), _f(f32(kg)),
                           _f(f32(kb)), _i(pos), freq, eps)
    return q2, k2


# ---- attention -------------------------------------------------------------
def _attn(fn, q, k, v, heads, n, hd):
    q, k, v = f32(q), f32(k), f32(v)
    out = np.empty(heads * n * hd, np.float32)
    fn(_f(q), _f(k), _f(v), heads, n, hd, _f(out))
    return out


def attention_naive(q, k, v, heads, n, hd):
    """attention::attention_naive (src/attention.rs:10-59)."""
    return _attn(lib().vko_attention_naive, q, k, v, heads, n, hd)


def attention_serial(q, k, v, heads, n, hd):
    """attention::attention_serial (src/attention.rs:204-233)."""
    return _attn(lib().vko_attention_serial, q, k, v, heads, n, hd)


def attention(q, k, v, heads, n, hd):
    """attention::attention (src/attention.rs:66-108), DA3 flash gate included."""
    return _attn(lib().vko_attention, q, k, v, heads, n, hd)


def flash_attention_scalar(q, k, v, heads, tokens):
    q, k, v = f32(q), f32(k), f32(v)
    out = np.empty(heads * tokens * 64, np.float32)
    lib().vko_flash_attention_scalar(_f(q), _f(k), _f(v), heads, tokens, _f(out))
    return out


def flash_attention_avx512(q, k, v, heads, tokens):
    """flash_attention_f32_da3_base (src/specialized.rs:730-765); None if gated off."""
    q, k, v = f32(q), f32(k), f32(v)
    out = np.empty(heads * tokens * 64, np.float32)
    ok = lib().vko_flash_attention_avx512(_f(q), _f(k), _f(v), heads, tokens, _f(out))
    return out if ok else None


# ---- projections -----------------------------------------------------------
def linear_fma_scalar(a, b, m, n, k):
    a, b = f32(a), f32(b)
    c = np.empty(m * n, np.float32)
    lib().vko_linear_fma_scalar(m, n, k, _f(a), _f(b), _f(c))
    return c


def linear(a, b, m, n, k):
    """linear_f32_da3_base arithmetic (src/specialized.rs:770-806, 1252-1300)."""
    a, b = f32(a), f32(b)
    c = np.empty(m * n, np.float32)
    lib().vko_linear(m, n, k, _f(a), _f(b), _f(c))
    return c


def linear_bias_scale(a, b, bias, scale, m, n, k):
    """linear_bias_scale_f32_da3_base (src/specialized.rs:811-929)."""
    a, b = f32(a), f32(b)
    c = np.empty(m * n, np.float32)
    lib().vko_linear_bias_scale(m, n, k, _f(a), _f(b), _f(f32(bias)), _f(f32(scale)), _f(c))
    return c


def qkv(a, w, bias, m):
    """qkv_f32_da3_base (src/specialized.rs:996-1167): head-major Q, K, V."""
    a, w = f32(a), f32(w)
    q = np.empty(m * 768, np.float32)
    k = np.empty(m * 768, np.float32)
    v = np.empty(m * 768, np.float32)
    lib().vko_qkv(m, _f(a), _f(w), _f(f32(bias)), _f(q), _f(k), _f(v))
    return q, k, v


def split_qkv_hnd(qkv_tm, tokens, heads, hd):
    x = f32(qkv_tm)
    n = tokens * heads * hd
    q, k, v = (np.empty(n, np.float32) for _ in range(3))
    lib().vko_split_qkv_hnd(_f(x), tokens, heads, hd, _f(q), _f(k), _f(v))
    return q, k, v


def hnd_to_token(hnd, tokens, heads, hd):
    x = f32(hnd)
    out = np.empty(tokens * heads * hd, np.float32)
    lib().vko_hnd_to_token(_f(x), tokens, heads, hd, _f(out))
    return out


# ---- DPT head ----------------------------------------------------------------
def _opt(a):
    return None if a is None else f32(a)


def conv_out_hw(ih, iw, kh, kw, stride, pad):
    return (ih + 2 * pad - kh) // stride + 1, (iw + 2 * pad - kw) // stride + 1


def conv2d_naive(x, in_c, ih, iw, w, out_c, kh, kw, stride, pad, bias=None):
    """conv::conv2d_naive (src/conv.rs:950-998), CHW, weight OIHW."""
    oh, ow = conv_out_hw(ih, iw, kh, kw, stride, pad)
    out = np.empty(out_c * oh * ow, np.float32)
    b = _opt(bias)
    lib().vko_conv2d_naive(_f(f32(x)), in_c, ih, iw, _f(f32(w)), out_c, kh, kw, stride, pad,
                           _f(b) if b is not None else None, _f(out))
    return out


def expf_glibc_form(x: float) -> float:
    """glibc 2.35's expf algorithm restated (the device GELU tail's expf)."""
    return float(lib().vko_expf_glibc_form(ctypes.c_float(x)))


def exp2f_table_entry(i: int) -> int:
    return int(lib().vko_exp2f_table_entry(i))


def expf_form_mismatches(step: int = 1) -> int:
    """Bit patterns (every step-th) where the restatement differs from the host's expf."""
    return int(lib().vko_expf_form_mismatches(step))


def winograd_f2_filter(w, in_c, out_c):
    """conv::transformed_winograd_filter (src/conv.rs:121-173): OIHW 3x3
    weights -> U [16][in_c][out_c]."""
    u = np.empty(16 * in_c * out_c, np.float32)
    lib().vko_winograd_f2_filter(_f(f32(w)), in_c, out_c, _f(u))
    return u


def conv3x3_winograd_f2(x, in_c, ih, iw, w, out_c, bias=None, relu_input=False, u=None,
                        lanes=False):
    """The crate's 3x3 stride-1 pad-1 convolution, Winograd F(2x2, 3x3)
    (src/conv.rs:681-829 with src/specialized.rs:597-633), CHW.  u: a
    prepared filter (winograd_f2_filter), else w (OIHW) is transformed
    first.  lanes: the AVX-512 product restated with fmaf."""
    if u is None:
        u = winograd_f2_filter(w, in_c, out_c)
    out = np.empty(out_c * ih * iw, np.float32)
    b = _opt(bias)
    lib().vko_winograd_use_lanes(1 if lanes else 0)
    try:
        lib().vko_conv3x3_winograd_f2(_f(f32(x)), in_c, ih, iw, _f(u), out_c,
                                      _f(b) if b is not None else None, 1 if relu_input else 0,
                                      _f(out))
    finally:
        lib().vko_winograd_use_lanes(0)
    return out


def _conv_t(fn, x, in_c, ih, iw, w, out_c, kh, kw, stride, bias):
    oh, ow = (ih - 1) * stride + kh, (iw - 1) * stride + kw
    out = np.empty(out_c * oh * ow, np.float32)
    b = _opt(bias)
    fn(_f(f32(x)), in_c, ih, iw, _f(f32(w)), out_c, kh, kw, stride,
       _f(b) if b is not None else None, _f(out))
    return out


def conv_transpose2d(x, in_c, ih, iw, w, out_c, kh, kw, stride, bias=None):
    """conv::conv_transpose2d (src/conv.rs:1009-1098), weight IOHW."""
    return _conv_t(lib().vko_conv_transpose2d, x, in_c, ih, iw, w, out_c, kh, kw, stride, bias)


def conv_transpose2d_naive(x, in_c, ih, iw, w, out_c, kh, kw, stride, bias=None):
    """The crate's gather-form test oracle (src/conv.rs:1646-1704)."""
    return _conv_t(lib().vko_conv_transpose2d_naive, x, in_c, ih, iw, w, out_c, kh, kw, stride,
                   bias)


def _resize(fn, x, c, ih, iw, oh, ow):
    out = np.zeros(c * oh * ow, np.float32)
    fn(_f(f32(x)), c, ih, iw, oh, ow, _f(out))
    return out


def bilinear_resize(x, c, ih, iw, oh, ow):
    """resample::bilinear_resize (src/resample.rs:10-77), half-pixel centres."""
    return _resize(lib().vko_bilinear_resize, x, c, ih, iw, oh, ow)


def bilinear_resize_naive(x, c, ih, iw, oh, ow):
    """resample::bilinear_resize_naive (src/resample.rs:101-149)."""
    return _resize(lib().vko_bilinear_resize_naive, x, c, ih, iw, oh, ow)


def bilinear_resize_align_corners(x, c, ih, iw, oh, ow):
    """resample::bilinear_resize_align_corners (src/resample.rs:184-245)."""
    return _resize(lib().vko_bilinear_resize_align_corners, x, c, ih, iw, oh, ow)


def xorshift32_vec(seed, n):
    """The reference tests' Xorshift32 data generator (src/conv.rs:1626-1640,
    src/resample.rs:330-345): x ^= x<<13, x ^= x>>17, x ^= x<<5 (u32), then
    (x as f32 / u32::MAX as f32) * 2 - 1, rounded as f32 at every step."""
    x = seed & 0xFFFFFFFF
    out = np.empty(n, np.float32)
    umax = np.float32(4294967295.0)
    for i in range(n):
        x ^= (x << 13) & 0xFFFFFFFF
        x ^= x >> 17
        x ^= (x << 5) & 0xFFFFFFFF
        v = np.float32(np.float32(x) / umax)
        out[i] = np.float32(np.float32(v * np.float32(2.0)) - np.float32(1.0))
    return out


# ---- block -----------------------------------------------------------------
BLOCK_FIELDS = [f for f, _ in BlockWeights._fields_ if f not in QK_NORM_FIELDS]


def vit_block(x, weights: dict, images, tokens, pos_yx=None, rope_freq=100.0, eps=1e-6,
              taps=False, q8_0=False):
    """One DA3-BASE encoder block per image (engine composition of the crate's kernels).

    q8_0=True runs the four projections as Q8_0: quantize_row_q8_0 of the
    input rows and of the rows of W^T, Kernels::gemm_q8_0, then bias /
    LayerScale / GELU as separate f32 passes (vko_vit_block_q8_0)."""
    xs = f32(x).copy()
    keep = {n: f32(weights[n]) for n in BLOCK_FIELDS + QK_NORM_FIELDS if weights.get(n) is not None}
    bw = BlockWeights(**{n: _f(a) for n, a in keep.items()})
    pos = None if pos_yx is None else np.ascontiguousarray(pos_yx, np.int64)
    t_ln = t_att = t_gelu = None
    null = ctypes.cast(None, _f32p)
    if taps:
        t_ln = np.empty(images * tokens * 768, np.float32)
        t_att = np.empty(images * tokens * 768, np.float32)
        t_gelu = np.empty(images * tokens * 3072, np.float32)
    fn = lib().vko_vit_block_q8_0 if q8_0 else lib().vko_vit_block
    fn(_f(xs), images, tokens, ctypes.byref(bw),
       _i(pos) if pos is not None else ctypes.cast(None, _i64p), rope_freq, eps,
       _f(t_ln) if taps else null, _f(t_att) if taps else null, _f(t_gelu) if taps else null)
    if taps:
        return xs, {"ln1": t_ln, "attn": t_att, "gelu": t_gelu}
    return xs


def encoder(x, layers: list, images, tokens, pos_yx=None, rope_freq=100.0, eps=1e-6,
            q8_0=False):
    """Blocks in order; q8_0 is one flag for all or a list with one per block."""
    flags = q8_0 if isinstance(q8_0, (list, tuple)) else [q8_0] * len(layers)
    for w, q in zip(layers, flags):
        x = vit_block(x, w, images, tokens, pos_yx, rope_freq, eps, q8_0=q)
    return x
