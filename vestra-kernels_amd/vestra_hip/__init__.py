"""Python front end of the MI355X HIP backend (``libvestra_hip.so``).

Mirrors the reference crate's device API (``src/cuda.rs``): ``Runtime`` is
``CudaRuntime``, ``Tensor`` is ``CudaTensorF32``, ``Linear`` is
``CudaLinearF32`` and the ``VhError`` subclasses are the ``CudaError``
variants.  Every call goes through the C ABI declared in
``include/vestra_hip.h``; there is no host fallback: if the shared library is
missing, importing ``lib()`` raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

from . import da3, seeded  # noqa: F401  (re-exported helpers)

_HERE = Path(__file__).resolve().parent
# VESTRA_HIP_LIB selects another build of the same sources (the host-side
# sanitizer build of `make -C vestra-kernels_amd asan`, for CPU-only runs).
LIB_PATH = Path(os.environ.get("VESTRA_HIP_LIB") or _HERE / "libvestra_hip.so")

_p = ctypes.c_void_p
_sz = ctypes.c_size_t
_f32p = ctypes.POINTER(ctypes.c_float)
_i64p = ctypes.POINTER(ctypes.c_int64)
_pp = ctypes.POINTER(ctypes.c_void_p)

# numpy twin of the reference's #[repr(C)] BlockQ8_0 (src/lib.rs:33-38).
BLOCK_Q8_0 = np.dtype([("d", "<u2"), ("qs", "i1", (32,))], align=False)

# ---- errors: CudaError (src/cuda.rs:337-354) --------------------------------


class VhError(RuntimeError):
    status = -1


class InitializeError(VhError):
    status = 1


class UploadError(VhError):
    status = 2


class DownloadError(VhError):
    status = 3


class LengthMismatch(VhError):
    status = 4

    def __init__(self, msg, destination=0, source_len=0):
        super().__init__(msg)
        self.destination = destination
        self.source_len = source_len


class KernelError(VhError):
    status = 5


class BlasError(VhError):
    status = 6


class InvalidArgument(VhError):
    status = 7


_ERRORS = {c.status: c for c in (InitializeError, UploadError, DownloadError, LengthMismatch,
                                  KernelError, BlasError, InvalidArgument)}

# ---- library ---------------------------------------------------------------

_lib = None

# (name, restype, argtypes) of every exported symbol of include/vestra_hip.h.
_S = ctypes.c_int  # vh_status
SIGNATURES = [
    ("vh_last_error", ctypes.c_char_p, []),
    ("vh_last_length_mismatch", None, [ctypes.POINTER(_sz), ctypes.POINTER(_sz)]),
    ("vh_runtime_new", _S, [_sz, _pp]),
    ("vh_runtime_clone", _S, [_p, _pp]),
    ("vh_runtime_free", None, [_p]),
    ("vh_runtime_device", _sz, [_p]),
    ("vh_runtime_stream", _p, [_p]),
    ("vh_runtime_synchronize", _S, [_p]),
    ("vh_upload_f32", _S, [_p, _f32p, _sz, _pp]),
    ("vh_download_f32", _S, [_p, _p, _f32p, _sz]),
    ("vh_tensor_alloc", _S, [_p, _sz, _pp]),
    ("vh_tensor_free", None, [_p]),
    ("vh_tensor_len", _sz, [_p]),
    ("vh_tensor_is_empty", ctypes.c_int, [_p]),
    ("vh_tensor_device_ptr", _p, [_p]),
    ("vh_copy_f32", _S, [_p, _p, _pp]),
    ("vh_copy_segment_f32", _S, [_p, _p, _sz, _sz, _pp]),
    ("vh_copy_segment_into_f32", _S, [_p, _p, _sz, _p, _sz, _sz]),
    ("vh_overwrite_prefix_f32", _S, [_p, _p, _p, _sz]),
    ("vh_add_f32_in_place", _S, [_p, _p, _p]),
    ("vh_gemm_row_major_f32", _S, [_p, _p, _p, _sz, _sz, _sz, _pp]),
    ("vh_bias_scale_f32_in_place", _S, [_p, _p, _p, _p, _sz, _sz]),
    ("vh_gelu_f32_in_place", _S, [_p, _p]),
    ("vh_layernorm_f32", _S, [_p, _p, _p, _p, _sz, _sz, ctypes.c_float, _pp]),
    ("vh_layernorm_f32_cpu_order", _S, [_p, _p, _p, _p, _sz, _sz, ctypes.c_float, _pp]),
    ("vh_attention_online_f32", _S, [_p, _p, _p, _p, _sz, _sz, _sz, _pp]),
    ("vh_flash_attention_f32_da3_base", _S, [_p, _p, _p, _p, _sz, _sz, ctypes.c_int, _pp]),
    ("vh_flash_attention_f32_da3_base_into", _S, [_p, _p, _p, _p, _sz, _sz, ctypes.c_int, _p]),
    ("vh_split_qkv_hnd_f32", _S, [_p, _p, _sz, _sz, _sz, _pp, _pp, _pp]),
    ("vh_hnd_to_token_f32", _S, [_p, _p, _sz, _sz, _sz, _pp]),
    ("vh_token_to_chw_f32", _S, [_p, _p, _sz, _sz, _pp]),
    ("vh_patchify_nchw_f32", _S, [_p, _p, _sz, _sz, _sz, _sz, _pp]),
    ("vh_prepend_cls_add_pos_f32", _S, [_p, _p, _p, _p, _sz, _sz, _pp]),
    ("vh_rope2d_f32_in_place", _S, [_p, _p, _sz, _sz, _sz, _i64p, ctypes.c_float]),
    ("vh_qk_norm_rope_f32_da3_base", _S, [_p, _p, _p, _p, _p, _p, _p, _p, _sz, _sz,
                                          ctypes.c_float, ctypes.c_float]),
    ("vh_prepare_linear_f32", _S, [_p, _sz, _sz, _f32p, _f32p, _f32p, _pp]),
    ("vh_linear_free", None, [_p]),
    ("vh_linear_input_features", _sz, [_p]),
    ("vh_linear_output_features", _sz, [_p]),
    ("vh_linear_run", _S, [_p, _p, _sz, _pp]),
    ("vh_linear_run_chw", _S, [_p, _p, _sz, _pp]),
    ("vh_linear_run_gelu", _S, [_p, _p, _sz, _pp]),
    ("vh_linear_run_residual", _S, [_p, _p, _sz, _p]),
    ("vh_linear_run_qkv_hnd", _S, [_p, _p, _sz, _sz, _sz, _i64p, ctypes.c_float, _pp, _pp, _pp]),
    ("vh_q8_0_upload", _S, [_p, _p, _sz, _sz, _pp]),
    ("vh_q8_0_download", _S, [_p, _p, _p, _sz]),
    ("vh_q8_tensor_free", None, [_p]),
    ("vh_q8_tensor_rows", _sz, [_p]),
    ("vh_q8_tensor_k", _sz, [_p]),
    ("vh_quantize_q8_0", _S, [_p, _p, _sz, _sz, _pp]),
    ("vh_quantize_q8_0_into", _S, [_p, _p, _sz, _sz, _p]),
    ("vh_gemm_q8_0", _S, [_p, _p, _p, _sz, _sz, _sz, _pp]),
    ("vh_gemm_q8_0_into", _S, [_p, _p, _p, _sz, _sz, _sz, _p]),
    ("vh_prepare_linear_q8_0", _S, [_p, _sz, _sz, _p, _f32p, _f32p, _pp]),
    ("vh_linear_q8_0_free", None, [_p]),
    ("vh_linear_q8_0_input_features", _sz, [_p]),
    ("vh_linear_q8_0_output_features", _sz, [_p]),
    ("vh_linear_q8_0_run", _S, [_p, _p, _sz, _pp]),
    ("vh_linear_q8_0_run_gelu", _S, [_p, _p, _sz, _pp]),
    ("vh_linear_q8_0_run_residual", _S, [_p, _p, _sz, _p]),
    ("vh_prepare_conv2d_f32", _S, [_p, _sz, _sz, _sz, _sz, _sz, _sz, _f32p, _f32p, _pp]),
    ("vh_conv2d_free", None, [_p]),
    ("vh_conv2d_output_height", _sz, [_p, _sz]),
    ("vh_conv2d_output_width", _sz, [_p, _sz]),
    ("vh_conv2d_run", _S, [_p, _p, _sz, _sz, _pp]),
    ("vh_conv2d_run_relu_input", _S, [_p, _p, _sz, _sz, _pp]),
    ("vh_conv2d_run_resize_align_corners", _S, [_p, _p, _sz, _sz, _sz, _sz, _p, _pp]),
    ("vh_conv2d_f32", _S, [_p, _p, _sz, _sz, _sz, _f32p, _sz, _sz, _sz, _sz, _sz, _f32p, _pp]),
    ("vh_prepare_conv_transpose2d_f32", _S, [_p, _sz, _sz, _sz, _sz, _sz, _f32p, _f32p, _pp]),
    ("vh_conv_transpose2d_free", None, [_p]),
    ("vh_conv_transpose2d_run", _S, [_p, _p, _sz, _sz, _pp]),
    ("vh_conv_transpose2d_f32", _S, [_p, _p, _sz, _sz, _sz, _f32p, _sz, _sz, _sz, _sz, _f32p,
                                     _pp]),
    ("vh_bilinear_resize_f32", _S, [_p, _p, _sz, _sz, _sz, _sz, _sz, _pp]),
    ("vh_bilinear_resize_align_corners_f32", _S, [_p, _p, _sz, _sz, _sz, _sz, _sz, _p, _pp]),
    ("vh_block_prepare", _S, [_p, _p, _pp]),
    ("vh_block_prepare_q8_0", _S, [_p, _p, _pp]),
    ("vh_block_is_q8_0", ctypes.c_int, [_p]),
    ("vh_block_free", None, [_p]),
    ("vh_vit_block_run", _S, [_p, _p, _p, _sz, _sz, _i64p, ctypes.c_float, ctypes.c_float]),
    ("vh_encoder_run", _S, [_p, _pp, _sz, _p, _sz, _sz, _i64p, ctypes.c_float,
                            ctypes.c_float]),
    ("vh_profile_enable", _S, [_p, ctypes.c_int]),
    ("vh_profile_reset", _S, [_p]),
    ("vh_profile_report", _S, [_p, ctypes.c_char_p, _sz]),
    ("vh_timer_start", _S, [_p]),
    ("vh_timer_stop", _S, [_p, ctypes.POINTER(ctypes.c_float)]),
]


def lib() -> ctypes.CDLL:
    """Loads libvestra_hip.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"HIP backend not built: {LIB_PATH} is missing (run __graft_entry__.build())")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, res, args in SIGNATURES:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(status: int) -> None:
    if status == 0:
        return
    L = lib()
    msg = (L.vh_last_error() or b"").decode(errors="replace")
    cls = _ERRORS.get(status, VhError)
    if cls is LengthMismatch:
        d, s = _sz(), _sz()
        L.vh_last_length_mismatch(ctypes.byref(d), ctypes.byref(s))
        raise LengthMismatch(msg, d.value, s.value)
    raise cls(msg)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _fp(a: np.ndarray):
    return a.ctypes.data_as(_f32p)


def _ip(a):
    if a is None:
        return ctypes.cast(None, _i64p)
    return np.ascontiguousarray(a, np.int64).ctypes.data_as(_i64p)


# ---- handles -----------------------------------------------------------------


class Tensor:
    """CudaTensorF32 (src/cuda.rs:1283-1286): an opaque device f32 buffer."""

    def __init__(self, runtime: "Runtime", handle: int):
        self._rt = runtime
        self._h = ctypes.c_void_p(handle)

    def __len__(self) -> int:
        return int(lib().vh_tensor_len(self._h))

    def is_empty(self) -> bool:
        return bool(lib().vh_tensor_is_empty(self._h))

    @property
    def handle(self):
        return self._h

    @property
    def device_ptr(self) -> int:
        return int(lib().vh_tensor_device_ptr(self._h) or 0)

    def free(self) -> None:
        if self._h and self._h.value:
            lib().vh_tensor_free(self._h)
            self._h = ctypes.c_void_p(None)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Linear:
    """CudaLinearF32 (src/cuda.rs:1291-1345)."""

    def __init__(self, runtime: "Runtime", handle: int):
        self._rt = runtime
        self._h = ctypes.c_void_p(handle)

    def input_features(self) -> int:
        return int(lib().vh_linear_input_features(self._h))

    def output_features(self) -> int:
        return int(lib().vh_linear_output_features(self._h))

    def run(self, x: Tensor, rows: int) -> Tensor:
        out = ctypes.c_void_p()
        _check(lib().vh_linear_run(self._h, x.handle, rows, ctypes.byref(out)))
        return Tensor(self._rt, out.value)

    def run_chw(self, x: Tensor, rows: int) -> Tensor:
        out = ctypes.c_void_p()
        _check(lib().vh_linear_run_chw(self._h, x.handle, rows, ctypes.byref(out)))
        return Tensor(self._rt, out.value)

    def run_gelu(self, x: Tensor, rows: int) -> Tensor:
        out = ctypes.c_void_p()
        _check(lib().vh_linear_run_gelu(self._h, x.handle, rows, ctypes.byref(out)))
        return Tensor(self._rt, out.value)

    def run_residual(self, x: Tensor, rows: int, residual: Tensor) -> None:
        _check(lib().vh_linear_run_residual(self._h, x.handle, rows, residual.handle))

    def run_qkv_hnd(self, x: Tensor, images: int, tokens: int, heads: int, pos_yx=None,
                    frequency: float = 100.0):
        q, k, v = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        pos = None if pos_yx is None else np.ascontiguousarray(pos_yx, np.int64)
        _check(lib().vh_linear_run_qkv_hnd(self._h, x.handle, images, tokens, heads, _ip(pos),
                                           frequency, ctypes.byref(q), ctypes.byref(k),
                                           ctypes.byref(v)))
        return Tensor(self._rt, q.value), Tensor(self._rt, k.value), Tensor(self._rt, v.value)

    def __del__(self):
        try:
            if self._h and self._h.value:
                lib().vh_linear_free(self._h)
                self._h = ctypes.c_void_p(None)
        except Exception:
            pass


class Q8Tensor:
    """Device rows of BlockQ8_0 (src/lib.rs:33-38)."""

    def __init__(self, runtime: "Runtime", handle: int):
        self._rt = runtime
        self._h = ctypes.c_void_p(handle)

    @property
    def handle(self):
        return self._h

    @property
    def rows(self) -> int:
        return int(lib().vh_q8_tensor_rows(self._h))

    @property
    def k(self) -> int:
        return int(lib().vh_q8_tensor_k(self._h))

    def __del__(self):
        try:
            if self._h and self._h.value:
                lib().vh_q8_tensor_free(self._h)
                self._h = ctypes.c_void_p(None)
        except Exception:
            pass


class LinearQ8:
    """A projection with BlockQ8_0 weights; input rows are quantised per run."""

    def __init__(self, runtime: "Runtime", handle: int):
        self._rt = runtime
        self._h = ctypes.c_void_p(handle)

    def input_features(self) -> int:
        return int(lib().vh_linear_q8_0_input_features(self._h))

    def output_features(self) -> int:
        return int(lib().vh_linear_q8_0_output_features(self._h))

    def _new(self, fn, x: Tensor, rows: int) -> Tensor:
        out = ctypes.c_void_p()
        _check(fn(self._h, x.handle, rows, ctypes.byref(out)))
        return Tensor(self._rt, out.value)

    def run(self, x: Tensor, rows: int) -> Tensor:
        return self._new(lib().vh_linear_q8_0_run, x, rows)

    def run_gelu(self, x: Tensor, rows: int) -> Tensor:
        return self._new(lib().vh_linear_q8_0_run_gelu, x, rows)

    def run_residual(self, x: Tensor, rows: int, residual: Tensor) -> None:
        _check(lib().vh_linear_q8_0_run_residual(self._h, x.handle, rows, residual.handle))

    def __del__(self):
        try:
            if self._h and self._h.value:
                lib().vh_linear_q8_0_free(self._h)
                self._h = ctypes.c_void_p(None)
        except Exception:
            pass


class Conv2d:
    """A prepared 2-D convolution (conv2d with a model-owned weight)."""

    def __init__(self, runtime: "Runtime", handle: int):
        self._rt = runtime
        self._h = ctypes.c_void_p(handle)

    def output_hw(self, ih: int, iw: int):
        return (int(lib().vh_conv2d_output_height(self._h, ih)),
                int(lib().vh_conv2d_output_width(self._h, iw)))

    def _new(self, fn, *args) -> Tensor:
        out = ctypes.c_void_p()
        _check(fn(self._h, *args, ctypes.byref(out)))
        return Tensor(self._rt, out.value)

    def run(self, x: Tensor, ih: int, iw: int) -> Tensor:
        return self._new(lib().vh_conv2d_run, x.handle, ih, iw)

    def run_relu_input(self, x: Tensor, ih: int, iw: int) -> Tensor:
        return self._new(lib().vh_conv2d_run_relu_input, x.handle, ih, iw)

    def run_resize_align_corners(self, x: Tensor, ih: int, iw: int, oh: int, ow: int,
                                 add: Tensor | None = None) -> Tensor:
        return self._new(lib().vh_conv2d_run_resize_align_corners, x.handle, ih, iw, oh, ow,
                         add.handle if add is not None else None)

    def __del__(self):
        try:
            if self._h and self._h.value:
                lib().vh_conv2d_free(self._h)
                self._h = ctypes.c_void_p(None)
        except Exception:
            pass


class ConvTranspose2d:
    """A prepared transposed convolution (IOHW weight)."""

    def __init__(self, runtime: "Runtime", handle: int):
        self._rt = runtime
        self._h = ctypes.c_void_p(handle)

    def run(self, x: Tensor, ih: int, iw: int) -> Tensor:
        out = ctypes.c_void_p()
        _check(lib().vh_conv_transpose2d_run(self._h, x.handle, ih, iw, ctypes.byref(out)))
        return Tensor(self._rt, out.value)

    def __del__(self):
        try:
            if self._h and self._h.value:
                lib().vh_conv_transpose2d_free(self._h)
                self._h = ctypes.c_void_p(None)
        except Exception:
            pass


class BlockParams(ctypes.Structure):
    _fields_ = [(n, _f32p) for n in da3.BLOCK_FIELDS + da3.QK_NORM_FIELDS]


class Block:
    """A prepared DA3-BASE encoder block (weights resident and repacked)."""

    def __init__(self, runtime: "Runtime", handle: int):
        self._rt = runtime
        self._h = ctypes.c_void_p(handle)

    @property
    def handle(self):
        return self._h

    @property
    def is_q8_0(self) -> bool:
        return bool(lib().vh_block_is_q8_0(self._h))

    def __del__(self):
        try:
            if self._h and self._h.value:
                lib().vh_block_free(self._h)
                self._h = ctypes.c_void_p(None)
        except Exception:
            pass


class Runtime:
    """CudaRuntime (src/cuda.rs:357-1279) over one HIP device and stream."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        _check(lib().vh_runtime_new(device, ctypes.byref(h)))
        self._h = h

    def __del__(self):
        try:
            if self._h and self._h.value:
                lib().vh_runtime_free(self._h)
                self._h = ctypes.c_void_p(None)
        except Exception:
            pass

    @property
    def handle(self):
        return self._h

    def device(self) -> int:
        return int(lib().vh_runtime_device(self._h))

    def stream(self) -> int:
        return int(lib().vh_runtime_stream(self._h) or 0)

    def synchronize(self) -> None:
        _check(lib().vh_runtime_synchronize(self._h))

    def _out(self, fn, *args) -> Tensor:
        out = ctypes.c_void_p()
        _check(fn(self._h, *args, ctypes.byref(out)))
        return Tensor(self, out.value)

    # -- tensors
    def upload_f32(self, values) -> Tensor:
        a = _f32(values).reshape(-1)
        return self._out(lib().vh_upload_f32, _fp(a), a.size)

    def download_f32(self, t: Tensor) -> np.ndarray:
        out = np.empty(len(t), np.float32)
        _check(lib().vh_download_f32(self._h, t.handle, _fp(out), out.size))
        return out

    def alloc_f32(self, n: int) -> Tensor:
        return self._out(lib().vh_tensor_alloc, n)

    def copy_f32(self, src: Tensor) -> Tensor:
        return self._out(lib().vh_copy_f32, src.handle)

    def copy_segment_f32(self, src: Tensor, offset: int, n: int) -> Tensor:
        return self._out(lib().vh_copy_segment_f32, src.handle, offset, n)

    def copy_segment_into_f32(self, dst: Tensor, dst_offset: int, src: Tensor, src_offset: int,
                              n: int) -> None:
        _check(lib().vh_copy_segment_into_f32(self._h, dst.handle, dst_offset, src.handle,
                                              src_offset, n))

    def overwrite_prefix_f32(self, dst: Tensor, src: Tensor, n: int) -> None:
        _check(lib().vh_overwrite_prefix_f32(self._h, dst.handle, src.handle, n))

    def add_f32_in_place(self, dst: Tensor, src: Tensor) -> None:
        _check(lib().vh_add_f32_in_place(self._h, dst.handle, src.handle))

    # -- GEMM / epilogues
    def gemm_row_major_f32(self, a: Tensor, b: Tensor, m: int, k: int, n: int) -> Tensor:
        return self._out(lib().vh_gemm_row_major_f32, a.handle, b.handle, m, k, n)

    def bias_scale_f32_in_place(self, v: Tensor, bias: Tensor, gamma: Tensor, rows: int,
                                cols: int) -> None:
        _check(lib().vh_bias_scale_f32_in_place(self._h, v.handle, bias.handle, gamma.handle,
                                                rows, cols))

    def gelu_f32_in_place(self, v: Tensor) -> None:
        _check(lib().vh_gelu_f32_in_place(self._h, v.handle))

    def layernorm_f32(self, x, gamma, beta, rows, cols, eps) -> Tensor:
        return self._out(lib().vh_layernorm_f32, x.handle, gamma.handle, beta.handle, rows, cols,
                         eps)

    def layernorm_f32_cpu_order(self, x, gamma, beta, rows, cols, eps) -> Tensor:
        return self._out(lib().vh_layernorm_f32_cpu_order, x.handle, gamma.handle, beta.handle,
                         rows, cols, eps)

    # -- attention
    def attention_online_f32(self, q, k, v, heads, tokens, head_dim) -> Tensor:
        return self._out(lib().vh_attention_online_f32, q.handle, k.handle, v.handle, heads,
                         tokens, head_dim)

    def flash_attention_f32_da3_base(self, q, k, v, heads, tokens, token_major=False) -> Tensor:
        return self._out(lib().vh_flash_attention_f32_da3_base, q.handle, k.handle, v.handle,
                         heads, tokens, 1 if token_major else 0)

    def flash_attention_f32_da3_base_into(self, q, k, v, heads, tokens, token_major,
                                          out: Tensor) -> None:
        """The same attention into a caller-provided `out`, with no device
        allocation (key-split partials in the library's per-GPU scratch)."""
        _check(lib().vh_flash_attention_f32_da3_base_into(
            self._h, q.handle, k.handle, v.handle, heads, tokens, 1 if token_major else 0,
            out.handle))

    # -- layout
    def split_qkv_hnd_f32(self, qkv, tokens, heads, head_dim):
        q, k, v = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        _check(lib().vh_split_qkv_hnd_f32(self._h, qkv.handle, tokens, heads, head_dim,
                                          ctypes.byref(q), ctypes.byref(k), ctypes.byref(v)))
        return Tensor(self, q.value), Tensor(self, k.value), Tensor(self, v.value)

    def hnd_to_token_f32(self, hnd, tokens, heads, head_dim) -> Tensor:
        return self._out(lib().vh_hnd_to_token_f32, hnd.handle, tokens, heads, head_dim)

    def token_to_chw_f32(self, tm, tokens, channels) -> Tensor:
        return self._out(lib().vh_token_to_chw_f32, tm.handle, tokens, channels)

    def patchify_nchw_f32(self, image, height, width, patch, channels) -> Tensor:
        return self._out(lib().vh_patchify_nchw_f32, image.handle, height, width, patch, channels)

    def prepend_cls_add_pos_f32(self, patches, cls, position, patch_count, embed) -> Tensor:
        return self._out(lib().vh_prepend_cls_add_pos_f32, patches.handle, cls.handle,
                         position.handle, patch_count, embed)

    # -- RoPE
    def rope2d_f32_in_place(self, x, heads, n, head_dim, pos_yx, frequency) -> None:
        pos = np.ascontiguousarray(pos_yx, np.int64)
        _check(lib().vh_rope2d_f32_in_place(self._h, x.handle, heads, n, head_dim, _ip(pos),
                                            frequency))

    def qk_norm_rope_f32_da3_base(self, q, k, qg, qb, kg, kb, positions_yx, heads, tokens,
                                  frequency, epsilon) -> None:
        _check(lib().vh_qk_norm_rope_f32_da3_base(self._h, q.handle, k.handle, qg.handle,
                                                  qb.handle, kg.handle, kb.handle,
                                                  positions_yx.handle, heads, tokens, frequency,
                                                  epsilon))

    # -- prepared projections
    def prepare_linear_f32(self, input_features, output_features, weight, bias,
                           gamma=None) -> Linear:
        w, b = _f32(weight).reshape(-1), _f32(bias).reshape(-1)
        g = None if gamma is None else _f32(gamma).reshape(-1)
        out = ctypes.c_void_p()
        _check(lib().vh_prepare_linear_f32(self._h, input_features, output_features, _fp(w),
                                           _fp(b), _fp(g) if g is not None else None,
                                           ctypes.byref(out)))
        return Linear(self, out.value)

    # -- Q8_0
    def q8_0_upload(self, blocks, rows, k) -> Q8Tensor:
        b = np.ascontiguousarray(blocks, BLOCK_Q8_0)
        out = ctypes.c_void_p()
        _check(lib().vh_q8_0_upload(self._h, b.ctypes.data, rows, k, ctypes.byref(out)))
        return Q8Tensor(self, out.value)

    def q8_0_download(self, t: Q8Tensor) -> np.ndarray:
        nb = t.rows * t.k // 32
        out = np.zeros(nb, BLOCK_Q8_0)
        _check(lib().vh_q8_0_download(self._h, t.handle, out.ctypes.data, nb))
        return out

    def quantize_q8_0(self, x: Tensor, rows, k) -> Q8Tensor:
        out = ctypes.c_void_p()
        _check(lib().vh_quantize_q8_0(self._h, x.handle, rows, k, ctypes.byref(out)))
        return Q8Tensor(self, out.value)

    def quantize_q8_0_into(self, x: Tensor, rows, k, out: Q8Tensor) -> None:
        """quantize_row_q8_0(x, out) into an existing rows x k Q8_0 tensor."""
        _check(lib().vh_quantize_q8_0_into(self._h, x.handle, rows, k, out.handle))

    def gemm_q8_0(self, a_q: Q8Tensor, b_q: Q8Tensor, m, n, k) -> Tensor:
        return self._out(lib().vh_gemm_q8_0, a_q.handle, b_q.handle, m, n, k)

    def gemm_q8_0_into(self, a_q: Q8Tensor, b_q: Q8Tensor, m, n, k, c: Tensor) -> None:
        """Kernels::gemm_q8_0 into an existing [m, n] tensor (the reference's c)."""
        _check(lib().vh_gemm_q8_0_into(self._h, a_q.handle, b_q.handle, m, n, k, c.handle))

    def prepare_linear_q8_0(self, input_features, output_features, weight_blocks, bias=None,
                            gamma=None) -> LinearQ8:
        """weight_blocks: output_features x input_features/32 BlockQ8_0 rows (W^T)."""
        wb = np.ascontiguousarray(weight_blocks, BLOCK_Q8_0)
        b = None if bias is None else _f32(bias).reshape(-1)
        g = None if gamma is None else _f32(gamma).reshape(-1)
        out = ctypes.c_void_p()
        _check(lib().vh_prepare_linear_q8_0(self._h, input_features, output_features,
                                            wb.ctypes.data if wb.size else None,
                                            _fp(b) if b is not None else None,
                                            _fp(g) if g is not None else None,
                                            ctypes.byref(out)))
        return LinearQ8(self, out.value)

    # -- DPT head
    def prepare_conv2d_f32(self, in_c, out_c, kh, kw, stride, pad, weight, bias=None) -> Conv2d:
        w = _f32(weight).reshape(-1)
        b = None if bias is None else _f32(bias).reshape(-1)
        out = ctypes.c_void_p()
        _check(lib().vh_prepare_conv2d_f32(self._h, in_c, out_c, kh, kw, stride, pad, _fp(w),
                                           _fp(b) if b is not None else None, ctypes.byref(out)))
        return Conv2d(self, out.value)

    def conv2d_f32(self, x: Tensor, in_c, ih, iw, weight, out_c, kh, kw, stride, pad,
                   bias=None) -> Tensor:
        w = _f32(weight).reshape(-1)
        b = None if bias is None else _f32(bias).reshape(-1)
        return self._out(lib().vh_conv2d_f32, x.handle, in_c, ih, iw, _fp(w), out_c, kh, kw,
                         stride, pad, _fp(b) if b is not None else None)

    def prepare_conv_transpose2d_f32(self, in_c, out_c, kh, kw, stride, weight,
                                     bias=None) -> ConvTranspose2d:
        w = _f32(weight).reshape(-1)
        b = None if bias is None else _f32(bias).reshape(-1)
        out = ctypes.c_void_p()
        _check(lib().vh_prepare_conv_transpose2d_f32(self._h, in_c, out_c, kh, kw, stride, _fp(w),
                                                     _fp(b) if b is not None else None,
                                                     ctypes.byref(out)))
        return ConvTranspose2d(self, out.value)

    def conv_transpose2d_f32(self, x: Tensor, in_c, ih, iw, weight, out_c, kh, kw, stride,
                             bias=None) -> Tensor:
        w = _f32(weight).reshape(-1)
        b = None if bias is None else _f32(bias).reshape(-1)
        return self._out(lib().vh_conv_transpose2d_f32, x.handle, in_c, ih, iw, _fp(w), out_c,
                         kh, kw, stride, _fp(b) if b is not None else None)

    def bilinear_resize_f32(self, x: Tensor, c, ih, iw, oh, ow) -> Tensor:
        return self._out(lib().vh_bilinear_resize_f32, x.handle, c, ih, iw, oh, ow)

    def bilinear_resize_align_corners_f32(self, x: Tensor, c, ih, iw, oh, ow,
                                          add: Tensor | None = None) -> Tensor:
        return self._out(lib().vh_bilinear_resize_align_corners_f32, x.handle, c, ih, iw, oh, ow,
                         add.handle if add is not None else None)

    # -- DA3 block / encoder
    def prepare_block(self, weights: dict, q8_0: bool = False) -> Block:
        """q8_0=True quantises the four projection weights to Q8_0 on the device."""
        keep = {n: _f32(weights[n]).reshape(-1) for n in da3.BLOCK_FIELDS + da3.QK_NORM_FIELDS
                if weights.get(n) is not None}
        params = BlockParams(**{n: _fp(a) for n, a in keep.items()})
        out = ctypes.c_void_p()
        fn = lib().vh_block_prepare_q8_0 if q8_0 else lib().vh_block_prepare
        _check(fn(self._h, ctypes.byref(params), ctypes.byref(out)))
        return Block(self, out.value)

    def vit_block_run(self, block: Block, x: Tensor, images, tokens, pos_yx=None,
                      rope_frequency=da3.ROPE_FREQ, epsilon=da3.LN_EPS) -> None:
        pos = None if pos_yx is None else np.ascontiguousarray(pos_yx, np.int64)
        _check(lib().vh_vit_block_run(self._h, block.handle, x.handle, images, tokens, _ip(pos),
                                      rope_frequency, epsilon))

    def encoder_run(self, blocks, x: Tensor, images, tokens, pos_yx=None,
                    rope_frequency=da3.ROPE_FREQ, epsilon=da3.LN_EPS) -> None:
        arr = (ctypes.c_void_p * max(1, len(blocks)))(*[b.handle.value for b in blocks])
        pos = None if pos_yx is None else np.ascontiguousarray(pos_yx, np.int64)
        _check(lib().vh_encoder_run(self._h, ctypes.cast(arr, _pp), len(blocks), x.handle, images,
                                    tokens, _ip(pos), rope_frequency, epsilon))

    # -- profiling
    def profile_enable(self, on: bool = True) -> None:
        _check(lib().vh_profile_enable(self._h, 1 if on else 0))

    def profile_reset(self) -> None:
        _check(lib().vh_profile_reset(self._h))

    def profile_report(self) -> dict:
        buf = ctypes.create_string_buffer(1 << 16)
        _check(lib().vh_profile_report(self._h, buf, len(buf)))
        out = {}
        for line in buf.value.decode().splitlines():
            name, count, ms = line.split()
            out[name] = (int(count), float(ms))
        return out

    def timer_start(self) -> None:
        _check(lib().vh_timer_start(self._h))

    def timer_stop(self) -> float:
        ms = ctypes.c_float()
        _check(lib().vh_timer_stop(self._h, ctypes.byref(ms)))
        return float(ms.value)
