// Device helpers shared by the gfx950 kernels: MFMA wrappers, wave64
// reductions and explicitly rounded float ops.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace vh {

// Raises a kernel's dynamic-LDS limit once per device: the attribute belongs
// to the device the call is made on, so each call site keeps one bit per
// device (atomically, as runtimes on different host threads may launch).
template <class Kernel>
inline hipError_t ensure_dynamic_lds(Kernel kernel, size_t bytes, std::atomic<uint64_t> &done) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = dev >= 0 && dev < 64 ? (uint64_t)1 << dev : 0;
    if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
    e = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_acq_rel);
    return e;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// v_mfma_f32_16x16x4_f32.  Lane l supplies A[l%16][l/16] and B[l/16][l%16];
// D[4*(l/16)+r][l%16] lands in register r of lane l.
__device__ __forceinline__ f32x4 mfma16x16x4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// v_mfma_i32_16x16x32_i8.  Lane l supplies 8 int8 of A row l%16 at
// k = 8*(l/16)..+7 and 8 int8 of B column l%16 at the same k;
// D[4*(l/16)+r][l%16] lands in register r of lane l.
__device__ __forceinline__ i32x4 mfma16x16x32_i8(long a, long b, i32x4 c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}

// Separately rounded float ops: the epilogues restate reference arithmetic
// that Rust never contracts into FMAs.  The operations are created under
// `fp contract(off)`, so they carry no contraction flag and the backend
// cannot fuse a multiply feeding an add even after inlining (HIP's own
// __fmul_rn/__fadd_rn are plain operators and do get fused).
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}
__device__ __forceinline__ float sub_rn(float a, float b) {
#pragma clang fp contract(off)
    return a - b;
}
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}
__device__ __forceinline__ float div_rn(float a, float b) {
#pragma clang fp contract(off)
    return __fdiv_rn(a, b);
}
// Correctly rounded square root.  The f32 sqrt of the device libm is only
// faithful (1 ulp); the f64 square root rounded to f32 is exact because
// 53 >= 2*24 + 2 makes double rounding innocuous for sqrt.
__device__ __forceinline__ float sqrt_rn(float x) { return (float)__builtin_sqrt((double)x); }

// p[i] when p is non-null, else `fallback`, with the load itself
// unconditional: it reads alt[i] (any valid address) when p is null, and the
// value is selected afterwards.  A load inside a branch leaves the compiler's
// wait insertion unsure at the join whether it is still pending, and it then
// waits for every load and store in flight there.
template <class T>
__device__ __forceinline__ T load_or(const T *p, const T *alt, size_t i, T fallback) {
    const T v = (p ? p : alt)[i];
    return p ? v : fallback;
}

// s_waitcnt vmcnt(0): every vector memory load and store of the wave done.
// Placed after a group of epilogue reads, it leaves nothing pending, so the
// stores that follow need no waits between them (vmcnt counts stores too).
__device__ __forceinline__ void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// Non-temporal store for the Store, GELU and Residual GEMM epilogues: the
// lines are not left dirty in the XCD's L2, so the end-of-kernel write-back
// that makes them visible to the next kernel has less to do (Q8_0 GEMM at
// the fc1 shape 15.5 -> 14.5 us, the f32 block's QKV-less GEMMs 0.4-0.5 us
// each).  Head-major Q/K/V stay cached: the attention re-reads each K and V
// panel from every query tile, and streamed Q/K/V cost it 0.5 us.
template <typename T>
__device__ __forceinline__ void stream_store(T *p, T v) {
    __builtin_nontemporal_store(v, p);
}

// One DPP lane permutation (a VALU modifier, no LDS round trip).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}

// Butterfly sum over the 64 lanes; every lane ends with the same total
// (each step adds two group sums, and a + b == b + a).  Within a 16-lane
// row by DPP: quad_perm [1,0,3,2] (lane ^ 1), quad_perm [2,3,0,1] (lane ^ 2),
// row_half_mirror (pairs the two quads of each 8), row_mirror (pairs the two
// 8s of each 16); across rows by two shuffles.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<0xb1>(v);
    v += dpp_f32<0x4e>(v);
    v += dpp_f32<0x141>(v);
    v += dpp_f32<0x140>(v);
    v += __shfl_xor(v, 16, kWave);
    v += __shfl_xor(v, 32, kWave);
    return v;
}

// Sum over each aligned group of G consecutive lanes (G = 2, 4, 8 or 16):
// the first log2(G) DPP steps of wave_sum; every lane of a group ends with
// the group's total.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(G == 2 || G == 4 || G == 8 || G == 16, "DPP lane groups within a row");
    v += dpp_f32<0xb1>(v);
    if constexpr (G >= 4) v += dpp_f32<0x4e>(v);
    if constexpr (G >= 8) v += dpp_f32<0x141>(v);
    if constexpr (G >= 16) v += dpp_f32<0x140>(v);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// LayerNorm of one row held by one wave in registers: r[j] = the float4
// chunk lane + 64 j of the row (n4 = cols / 4 <= 256 chunks; absent chunks
// are zero).  Mean, then the variance about the mean (two passes over the
// registers), inv = 1 / sqrt(var + eps) correctly rounded; every kernel that
// normalises rows this way shares these two functions and so produces the
// same bits.
__device__ __forceinline__ void ln_row_stats(const f32x4 (&r)[4], int lane, int n4, int cols,
                                             float eps, float &mean, float &inv) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) s += (r[j].x + r[j].y) + (r[j].z + r[j].w);
    mean = div_rn(wave_sum(s), (float)cols);
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        if (lane + j * 64 < n4) {
            const f32x4 d = r[j] - mean;
            q += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
        }
    }
    const float var = div_rn(wave_sum(q), (float)cols);
    inv = div_rn(1.0f, sqrt_rn(add_rn(var, eps)));
}
// ((x - mean) * inv) * g + b, each step separately rounded.
__device__ __forceinline__ f32x4 ln_apply(f32x4 x, float mean, float inv, f32x4 g, f32x4 b) {
    f32x4 o;
    o.x = add_rn(mul_rn(mul_rn(sub_rn(x.x, mean), inv), g.x), b.x);
    o.y = add_rn(mul_rn(mul_rn(sub_rn(x.y, mean), inv), g.y), b.y);
    o.z = add_rn(mul_rn(mul_rn(sub_rn(x.z, mean), inv), g.z), b.z);
    o.w = add_rn(mul_rn(mul_rn(sub_rn(x.w, mean), inv), g.w), b.w);
    return o;
}


// Cephes-style exp with the constants and FMA placement of the reference's
// AVX-512 exp (src/simd_avx512.rs:22-69).  x86 min/max select the second
// operand on NaN; cvttps truncates toward zero.
__device__ __forceinline__ float cephes_exp(float x) {
    x = (x < 88.37626f) ? x : 88.37626f;
    x = (x > -88.37626f) ? x : -88.37626f;
    // The reference truncates (cvttps) and subtracts one where truncation
    // rose; after the clamps fx0 lies in [-127, 128], where that is floor
    // (the same bits for all 2^32 inputs, checked on the host), one
    // instruction instead of five.
    const float fx = __builtin_floorf(__fmaf_rn(x, 1.44269504f, 0.5f));
    x = __fmaf_rn(-fx, 0.693359375f, x);
    x = __fmaf_rn(-fx, -2.1219444e-4f, x);
    float z = mul_rn(x, x);
    float y = 1.98756915e-4f;
    y = __fmaf_rn(y, x, 1.39819995e-3f);
    y = __fmaf_rn(y, x, 8.3334519e-3f);
    y = __fmaf_rn(y, x, 4.1665796e-2f);
    y = __fmaf_rn(y, x, 1.6666665e-1f);
    y = __fmaf_rn(y, x, 5.0000001e-1f);
    y = __fmaf_rn(y, z, x);
    y = add_rn(y, 1.0f);
    int e = ((int)fx + 0x7f) << 23;
    return mul_rn(y, __int_as_float(e));
}

// Correctly rounded 1/x for normal x in [2^-126, 2^126): one Newton step
// from v_rcp_f32 (r + r(1 - x r), two FMAs).  An exhaustive check of every
// float in that range on gfx950 found each result equal to the IEEE
// division; other x (zero, subnormal, huge, inf, NaN) take the division.
__device__ __forceinline__ float recip_rn(float x) {
    if (x >= 0x1p-126f && x < 0x1p126f) {
        const float r = __builtin_amdgcn_rcpf(x);
        return __builtin_fmaf(__builtin_fmaf(-x, r, 1.0f), r, r);
    }
    return div_rn(1.0f, x);
}

// Correctly rounded a / 127 for finite a >= 0 (the Q8_0 scale amax / 127):
// the product with the rounded reciprocal, corrected once by its FMA
// residual.  An exhaustive check of all 2^31 - 2^23 non-negative finite
// floats on gfx950 found every result equal to the IEEE division; inf and
// NaN take the division.
__device__ __forceinline__ float div127_rn(float a) {
    if (a < __builtin_inff()) {
        const float k = 1.0f / 127.0f;
        const float q = a * k;
        return __builtin_fmaf(__builtin_fmaf(-127.0f, q, a), k, q);
    }
    return div_rn(a, 127.0f);
}

// One step of quantize_row_q8_0's block max (src/q8_0_dot.rs:35): the fold
// starts at 0 and f32::max returns the other operand when one is NaN, so the
// max ignores every NaN (quiet or signalling) and an all-NaN block has
// amax 0.  A compare-select does exactly that (a NaN compares false) and, with
// NaNs ignored, the result does not depend on the order of the steps.
__device__ __forceinline__ float q8_absmax(float acc, float v) {
    const float a = fabsf(v);
    return a > acc ? a : acc;
}

// quantize_row_q8_0's scale and its reciprocal (src/q8_0_dot.rs:35-37):
// d = amax / 127, inv = d != 0 ? 1 / d : 0, both correctly rounded.
__device__ __forceinline__ void q8_scale(float amax, float &d, float &inv) {
    d = div127_rn(amax);
    inv = d != 0.0f ? recip_rn(d) : 0.0f;
}

// GELU with the AVX-512 erf of src/simd_avx512.rs:141-209:
// t = 1/fma(c,|a|,1); Horner by FMA; y = 1 - poly*exp(-a^2) fused.
__device__ __forceinline__ float gelu_avx512_form(float v) {
    float a = mul_rn(v, 0.70710678f);
    float xa = fabsf(a);
    float sign = (a < 0.0f) ? -1.0f : 1.0f;
    float t = recip_rn(__fmaf_rn(0.3275911f, xa, 1.0f));  // _mm512_div_ps(1, .)
    float poly = 1.0614054f;
    poly = __fmaf_rn(poly, t, -1.4531520f);
    poly = __fmaf_rn(poly, t, 1.4214137f);
    poly = __fmaf_rn(poly, t, -0.28449674f);
    poly = __fmaf_rn(poly, t, 0.25482959f);
    poly = mul_rn(poly, t);
    float e = cephes_exp(sub_rn(0.0f, mul_rn(xa, xa)));
    float y = __fmaf_rn(-poly, e, 1.0f);
    float erf = mul_rn(sign, y);
    return mul_rn(mul_rn(0.5f, v), add_rn(1.0f, erf));
}

// The same A&S 7.1.26 erf GELU with the hardware reciprocal and exp2 (each
// within 1 ulp) in place of the correctly rounded division and the Cephes
// exp: about half the VALU work of gelu_avx512_form, within a few ulp of it.
// For fused f32 GEMM epilogues, whose input already carries the GEMM's
// rounding; the standalone GELU and the Q8_0 paths keep the exact forms.
__device__ __forceinline__ float gelu_fast_form(float v) {
    const float a = v * 0.70710678f;
    const float xa = fabsf(a);
    const float t = __builtin_amdgcn_rcpf(__fmaf_rn(0.3275911f, xa, 1.0f));
    float p = __fmaf_rn(1.0614054f, t, -1.4531520f);
    p = __fmaf_rn(p, t, 1.4214137f);
    p = __fmaf_rn(p, t, -0.28449674f);
    p = __fmaf_rn(p, t, 0.25482959f);
    p = p * t;
    const float e = __builtin_amdgcn_exp2f(-(xa * xa) * 1.44269504f);
    const float erf = copysignf(__fmaf_rn(-p, e, 1.0f), a);
    return (0.5f * v) * (1.0f + erf);
}

// expf as glibc 2.35 computes it on x86-64 with FMA (the function the
// crate's f32::exp calls on Linux), so that the scalar GELU below gives the
// crate's bits.  The published design of that expf (ARM optimized-routines,
// taken into glibc 2.27): x * 32/ln2 = k + r with k rounded to an integer by
// the 1.5 * 2^52 shift, 2^(k/32) from a 32-entry table of the correctly
// rounded 2^(i/32) with i << 47 subtracted from each entry's bits (so that
// adding k << 47 puts k / 32 into the exponent), and 2^(r/32) by a degree-3
// polynomial, all in double, every multiply-add fused, then one rounding to
// float.  Reproduced exactly, this form equals the host libm's expf for all
// 2^32 inputs (an exhaustive host comparison of the same arithmetic in the
// test suite); the device's own expf is within 1 ulp but not always equal.
__device__ __forceinline__ float glibc_expf(float x) {
    constexpr uint64_t kTab[32] = {
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};
    const uint32_t bits = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (bits >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                            // |x| >= 88, inf or NaN
        if (bits == 0xff800000u) return 0.0f;          // exp(-inf)
        if (abstop >= 0x7f8) return x + x;             // +inf, NaN
        if (x > 0x1.62e42ep6f) return __builtin_inff(); // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;           // underflow
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    const double s = __builtin_bit_cast(double, kTab[ki % 32] + (ki << 47));
    const double z = __builtin_fma(c0, r, c1), r2 = r * r;
    const double y = __builtin_fma(z, r2, __builtin_fma(c2, r, 1.0));
    return (float)(y * s);
}

// Scalar GELU of src/scalar.rs:116-134 (used by the AVX-512 path's n%16
// tail), with the host libm's expf (glibc_expf above).
__device__ __forceinline__ float gelu_scalar_form(float v) {
    float x = mul_rn(v, 0.70710677f);
    float s = isnan(x) ? x : copysignf(1.0f, x);
    float ax = fabsf(x);
    float t = div_rn(1.0f, add_rn(1.0f, mul_rn(0.3275911f, ax)));
    float p = sub_rn(mul_rn(1.0614054f, t), 1.453152f);
    p = add_rn(mul_rn(p, t), 1.4214137f);
    p = sub_rn(mul_rn(p, t), 0.28449674f);
    p = add_rn(mul_rn(p, t), 0.2548296f);
    float y = sub_rn(1.0f, mul_rn(mul_rn(p, t), glibc_expf(mul_rn(-ax, ax))));
    return mul_rn(mul_rn(0.5f, v), add_rn(1.0f, mul_rn(s, y)));
}

}  // namespace vh
