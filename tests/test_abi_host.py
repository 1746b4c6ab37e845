"""CPU checks of the C-ABI library and the host-side logic (no compute calls).

- libvestra_hip.so loads and exports every function declared in
  include/vestra_hip.h, and the Python binding declares each one;
- null handles and bad arguments fail with the documented status before any
  HIP call, and runtime creation without a device reports Initialize;
- the seeded generator, DA3 positions and bench.py's single-GPU contract.
"""
import ctypes
import re
import subprocess
import sys

import numpy as np

import vestra_hip as vh
from conftest import ROOT
from vestra_hip import da3, seeded

HEADER = ROOT / "include" / "vestra_hip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(vh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) > 50
    lib = vh.lib()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    bound = {n for n, _, _ in vh.SIGNATURES}
    assert set(names) == bound, (set(names) ^ bound)


RUST_BINDING = ROOT / "vestra-kernels_amd" / "rust" / "hip.rs"
# Not bound in Rust: clones share one runtime through Arc, and is_empty uses len.
RUST_UNBOUND = {"vh_runtime_clone", "vh_tensor_is_empty"}


C_BASE_TO_RUST = {"size_t": "usize", "int": "c_int", "float": "f32", "int64_t": "i64",
                  "void": "c_void", "char": "c_char", "vh_status": "Status"}


def _rust_name(c_base):
    """vh_q8_tensor -> VhQ8Tensor; the scalar types through C_BASE_TO_RUST."""
    if c_base in C_BASE_TO_RUST:
        return C_BASE_TO_RUST[c_base]
    assert c_base.startswith("vh_"), c_base
    return "".join(w[:1].upper() + w[1:] for w in c_base.split("_"))


def c_type_as_rust(decl, has_name=True):
    """The Rust FFI spelling of a C parameter or return type: `const T *p`
    -> `*const T`, `T **p` -> `*mut *mut T`, `const T *const *p` ->
    `*const *const T`, built from the innermost pointee outwards (each
    level's const qualifier decides the next pointer's mutability)."""
    decl = " ".join(decl.replace("*", " * ").split())
    tokens = decl.split()
    if has_name:
        tokens = tokens[:-1]  # the parameter name
    parts = " ".join(tokens).split("*")
    base_words = parts[0].split()
    const = "const" in base_words
    base = [w for w in base_words if w != "const"]
    assert len(base) == 1, decl
    rust = _rust_name(base[0])
    for qual in parts[1:]:
        rust = ("*const " if const else "*mut ") + rust
        const = "const" in qual.split()
    return rust


def test_rust_binding_declares_the_header():
    """The `hip` feature's FFI block (rust/hip.rs) declares every C-ABI
    function with the header's parameter and return types, in order
    (size_t -> usize, int -> c_int, float -> f32, int64_t -> i64,
    `const T *` -> `*const T`, `T *` / `T **` -> `*mut ...`).  The Rust file
    is compiled by the crate's build, not here: no Rust toolchain in this
    image."""
    text = RUST_BINDING.read_text()
    block = text[text.index('unsafe extern "C" {'):]
    block = block[:block.index("\n}\n")]
    rust = {m.group(1): (m.group(2), (m.group(3) or "").strip())
            for m in re.finditer(r"fn (vh_[a-z0-9_]+)\(([^)]*)\)\s*(?:->\s*([^;]+))?;", block, flags=re.S)}
    names = set(declared_functions())
    assert set(rust) == names - RUST_UNBOUND, set(rust) ^ (names - RUST_UNBOUND)
    header = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    checked = 0
    for name, (params, ret) in rust.items():
        m = re.search(r"([A-Za-z_][\w\s\*]*?)\b" + name + r"\s*\(([^)]*)\)", header)
        c_ret, c_params = m.group(1), m.group(2)
        c_list = [] if c_params.strip() in ("", "void") else [p.strip() for p in c_params.split(",")]
        r_list = [p.strip() for p in params.split(",") if p.strip()]
        assert len(c_list) == len(r_list), (name, c_list, r_list)
        for c_p, r_p in zip(c_list, r_list):
            r_type = " ".join(r_p.split(":", 1)[1].split())
            assert c_type_as_rust(c_p) == r_type, (name, c_p, r_p)
            checked += 1
        c_ret = c_ret.strip()
        want = "" if c_ret == "void" else c_type_as_rust(c_ret, has_name=False)
        assert " ".join(ret.split()) == want, (name, c_ret, ret)
    assert checked > 250
    assert 'compile_error!("features `cuda` and `hip` are exclusive' in text


def test_rust_type_mapping_catches_mismatches():
    """The mapping the binding test uses distinguishes what an FFI mistake
    would confuse."""
    assert c_type_as_rust("size_t n") == "usize"
    assert c_type_as_rust("int flag") == "c_int"
    assert c_type_as_rust("float eps") == "f32"
    assert c_type_as_rust("const float *x") == "*const f32"
    assert c_type_as_rust("float *x") == "*mut f32"
    assert c_type_as_rust("const int64_t *pos") == "*const i64"
    assert c_type_as_rust("vh_tensor **out") == "*mut *mut VhTensor"
    assert c_type_as_rust("const vh_block *const *blocks") == "*const *const VhBlock"
    assert c_type_as_rust("const vh_q8_tensor *q") == "*const VhQ8Tensor"
    assert c_type_as_rust("vh_status", has_name=False) == "Status"
    assert c_type_as_rust("const char *", has_name=False) == "*const c_char"


def test_null_handles_fail_before_any_device_call():
    L = vh.lib()
    out = ctypes.c_void_p()
    x = np.ones(4, np.float32)
    st = L.vh_upload_f32(None, x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), 4,
                         ctypes.byref(out))
    assert st == vh.InvalidArgument.status
    assert b"null" in L.vh_last_error()
    assert L.vh_tensor_len(None) == 0 and L.vh_tensor_is_empty(None) == 1
    assert L.vh_runtime_new(0, None) == vh.InvalidArgument.status
    assert L.vh_linear_run(None, None, 0, None) == vh.InvalidArgument.status
    assert L.vh_vit_block_run(None, None, None, 1, 865, None, 100.0, 1e-6) == vh.InvalidArgument.status


def test_runtime_without_device_reports_initialize():
    L = vh.lib()
    h = ctypes.c_void_p()
    st = L.vh_runtime_new(0, ctypes.byref(h))
    if st == 0:  # a device is visible: nothing to check here
        L.vh_runtime_free(h)
        return
    assert st == vh.InitializeError.status
    assert b"initialize" in L.vh_last_error()
    try:
        vh.Runtime(0)
    except vh.InitializeError:
        pass
    else:
        raise AssertionError("Runtime(0) must raise InitializeError without a device")
    assert L.vh_runtime_new(10 ** 6, ctypes.byref(h)) == vh.InitializeError.status


def test_seeded_normal_statistics_and_determinism():
    a = seeded.normal(42, 200_000)
    assert a.dtype == np.float32
    assert abs(float(a.mean())) < 0.01 and abs(float(a.std()) - 1.0) < 0.01
    assert np.array_equal(a, seeded.normal(42, 200_000))
    assert not np.array_equal(a[:100], seeded.normal(43, 100))
    b = seeded.normal(42, 1001, std=0.02)
    assert np.allclose(b, a[:1001] * 0.02, rtol=1e-6, atol=1e-9)
    # splitmix64 reference value (state 0 -> first output)
    assert int(seeded.splitmix64(0, 1)[0]) == 0xE220A8397B1DCDAF


def test_da3_shapes_and_positions():
    assert da3.grid(336, 504) == (24, 36) and da3.tokens_for(336, 504) == 865
    assert da3.grid(672, 1008) == (48, 72) and da3.tokens_for(672, 1008) == 3457
    pos = da3.positions_yx(24, 36).reshape(-1, 2)
    assert pos.shape == (865, 2) and pos[0].tolist() == [0, 0]
    assert pos[1 + 37].tolist() == [2, 2]  # patch 37 = row 1, col 1
    w = da3.block_weights(seed=1)
    assert w["w_qkv"].size == 768 * 2304 and w["w_fc2"].size == 3072 * 768
    assert float(w["ls1"][0]) == np.float32(1e-5)
    assert abs(float(w["w_fc1"].std()) - 0.02) < 0.001


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr
