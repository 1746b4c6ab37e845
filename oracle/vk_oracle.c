/*
 * vk_oracle.c -- TEST INFRASTRUCTURE ONLY (see vk_oracle.h).
 *
 * CPU restatement of hoppworks/vestra-kernels' scalar oracles and AVX-512
 * kernels for the DA3-BASE ViT encoder hot path.  Build flags (oracle/Makefile):
 *   -O2 -ffp-contract=off -fno-fast-math -fopenmp
 * AVX-512 functions carry their own target attributes and are only entered
 * after vko_has_avx512(); every one has a scalar restatement with identical
 * arithmetic that the tests compare bitwise, as the reference's own tests do.
 *
 * Threading: OpenMP replaces rayon.  Work splits mirror the reference's
 * (column panels, row tiles, head x query tiles); results never depend on
 * the split because each output keeps its own sequential accumulation.
 */
#include "vk_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#define DA3_TOKENS 865 /* src/specialized.rs:31 */

/* ------------------------------------------------------------------------ */
/* capability / threads                                                     */
/* ------------------------------------------------------------------------ */

/* 1 = behave as a host without AVX-512 (the reference's scalar tier). */
static int g_force_scalar = 0;
void vko_force_scalar(int on) { g_force_scalar = on ? 1 : 0; }

int vko_has_avx512(void) {
    /* src/dispatch.rs:34-48 gates the AVX-512 tier on F+BW+VNNI; the DA3
     * kernels additionally check fma (src/specialized.rs:759). */
    if (g_force_scalar) return 0;
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("fma");
}

/* src/specialized.rs:759 and src/attention.rs:83 gate on avx512f (+fma) only. */
static int has_avx512f_fma(void) {
    if (g_force_scalar) return 0;
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("fma");
}

static int g_threads = 0;
int vko_get_threads(void);
#define OMP_THREADS num_threads(vko_get_threads())
void vko_set_threads(int n) { g_threads = n > 0 ? n : 0; }
int vko_get_threads(void) { return g_threads > 0 ? g_threads : omp_get_max_threads(); }

/* Rust's `iter().sum::<f32>()` folds from -0.0 (core::iter::Sum for f32). */
#define RUST_SUM_INIT (-0.0f)

/* Rust f32::max (core f32::max): the larger operand, and "if one of the
 * arguments is NaN, then the other argument is returned" -- every NaN,
 * signalling ones included (IEEE maxNum would quiet a signalling NaN, and
 * glibc fmaxf does). */
static inline float rmax(float a, float b) {
    if (isnan(b)) return a;
    if (isnan(a)) return b;
    return fmaxf(a, b);
}

float vko_rust_max(float a, float b) { return rmax(a, b); }

/* ------------------------------------------------------------------------ */
/* f16: half 2.7.1 f16::from_f32 / to_f32 (IEEE binary16, RNE)              */
/* ------------------------------------------------------------------------ */

uint16_t vko_f32_to_f16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t exp = (u >> 23) & 0xffu;
    uint32_t man = u & 0x7fffffu;
    if (exp == 0xffu) { /* inf / nan: keep a quiet payload bit for nan */
        if (man == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | (man >> 13));
    }
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
    if (e <= 0) {                                   /* subnormal or zero */
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (half & 1u))) half++;
        return (uint16_t)(sign | half);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* may carry into exp: correct */
    return (uint16_t)h;
}

float vko_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t man = (uint32_t)h & 0x3ffu;
    uint32_t u;
    if (exp == 0) {
        if (man == 0) {
            u = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do {
                e++;
                man <<= 1;
            } while ((man & 0x400u) == 0);
            u = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (exp == 0x1fu) { /* inf stays inf; a NaN widens quiet (bit 22 set) */
        u = sign | 0x7f800000u | (man ? 0x400000u : 0u) | (man << 13);
    } else {
        u = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

__attribute__((target("f16c"))) uint16_t vko_f32_to_f16_hw(float x) {
    return (uint16_t)_cvtss_sh(x, 0);
}

/* Pins the software conversion against F16C (vcvtps2ph imm 0 = RNE) over
 * every `step`-th f32 bit pattern and every f16 -> f32 widening; returns the
 * number of mismatches (NaN results compare by NaN-ness and sign). */
__attribute__((target("f16c"))) uint64_t vko_f16_sweep(uint32_t step) {
    uint64_t bad = 0;
    if (step == 0) step = 1;
#pragma omp parallel for OMP_THREADS reduction(+ : bad) schedule(static)
    for (int64_t i = 0; i <= 0xffffffffLL; i += step) {
        uint32_t u = (uint32_t)i;
        float f;
        memcpy(&f, &u, 4);
        uint16_t sw = vko_f32_to_f16(f), hw = (uint16_t)_cvtss_sh(f, 0);
        if (sw != hw) bad++;
    }
    for (uint32_t h = 0; h < 65536; h++) {
        float a = vko_f16_to_f32((uint16_t)h), b = _cvtsh_ss((unsigned short)h);
        uint32_t ua, ub;
        memcpy(&ua, &a, 4);
        memcpy(&ub, &b, 4);
        if (ua != ub) bad++;
    }
    return bad;
}

/* ------------------------------------------------------------------------ */
/* scalar oracles: src/scalar.rs                                            */
/* ------------------------------------------------------------------------ */

/* src/scalar.rs:3-18 -- naive i-p-j, c += a*b (separate multiply and add). */
void vko_gemm_f32(size_t m, size_t n, size_t k, const float *a, const float *b, float *c) {
    for (size_t i = 0; i < m; i++) {
        for (size_t j = 0; j < n; j++) c[i * n + j] = 0.0f;
        for (size_t p = 0; p < k; p++) {
            float aip = a[i * k + p];
            for (size_t j = 0; j < n; j++) c[i * n + j] += aip * b[p * n + j];
        }
    }
}

/* src/scalar.rs:25-56 -- int32 block sum, then acc += (da*db)*isum in block order. */
void vko_gemm_q8_0(size_t m, size_t n, size_t k, const vko_block_q8_0 *a_q,
                   const vko_block_q8_0 *b_q, float *c) {
    size_t bpr = k / VKO_QK8_0;
    for (size_t i = 0; i < m; i++) {
        const vko_block_q8_0 *ar = a_q + i * bpr;
        for (size_t j = 0; j < n; j++) {
            const vko_block_q8_0 *br = b_q + j * bpr;
            float acc = 0.0f;
            for (size_t bi = 0; bi < bpr; bi++) {
                int32_t isum = 0;
                for (int l = 0; l < VKO_QK8_0; l++)
                    isum += (int32_t)ar[bi].qs[l] * (int32_t)br[bi].qs[l];
                float dd = vko_f16_to_f32(ar[bi].d) * vko_f16_to_f32(br[bi].d);
                acc += dd * (float)isum;
            }
            c[i * n + j] = acc;
        }
    }
}

/* src/scalar.rs:58-63 */
void vko_add(float *dst, const float *src, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] += src[i];
}

/* src/scalar.rs:65-81 */
void vko_add_bias_rows(float *x, size_t rows, size_t cols, const float *bias) {
#pragma omp parallel for OMP_THREADS if (rows >= 32)
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < cols; c++) x[r * cols + c] += bias[c];
}

/* src/scalar.rs:99-114 -- sequential mean, sequential variance, 1/sqrt. */
static void layernorm_row(float *row, size_t cols, const float *gamma, const float *beta,
                          float eps) {
    float sum = RUST_SUM_INIT;
    for (size_t c = 0; c < cols; c++) sum += row[c];
    float mean = sum / (float)cols;
    float sq = RUST_SUM_INIT;
    for (size_t c = 0; c < cols; c++) {
        float d = row[c] - mean;
        sq += d * d;
    }
    float var = sq / (float)cols;
    float inv = 1.0f / sqrtf(var + eps);
    for (size_t c = 0; c < cols; c++) row[c] = (row[c] - mean) * inv * gamma[c] + beta[c];
}

/* src/scalar.rs:83-97 */
void vko_layernorm(float *x, size_t rows, size_t cols, const float *gamma, const float *beta,
                   float eps) {
#pragma omp parallel for OMP_THREADS if (rows >= 32)
    for (size_t r = 0; r < rows; r++) layernorm_row(x + r * cols, cols, gamma, beta, eps);
}

/* The expf that f32::exp calls on Linux (src/scalar.rs:132 uses it): glibc
 * 2.35 on x86-64 with FMA, whose published design is ARM
 * optimized-routines' expf (in glibc since 2.27).  x * 32/ln2 = k + r, k
 * rounded to an integer by adding 1.5 * 2^52; 2^(k/32) from a table of the
 * correctly rounded 2^(i/32) with i << 47 taken off each entry's bits, so
 * that adding k << 47 carries k / 32 into the exponent; 2^(r/32) by a cubic;
 * double precision with every multiply-add fused, one rounding to float.
 * The oracle itself calls the host's expf; this restatement exists to pin
 * the device's transcription (gelu_scalar_form's glibc_expf) against it:
 * vko_expf_form_mismatches counts where the two differ. */
static const uint64_t EXP2F_TAB[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

uint64_t vko_exp2f_table_entry(int i) { return EXP2F_TAB[i & 31]; }

float vko_expf_glibc_form(float x) {
    uint32_t bits;
    memcpy(&bits, &x, 4);
    const uint32_t abstop = (bits >> 20) & 0x7ff;
    if (abstop >= 0x42b) {             /* |x| >= 88, inf or NaN */
        if (bits == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    double kd = fma(inv_ln2_n, xd, shift);
    uint64_t ki, sb;
    memcpy(&ki, &kd, 8);
    kd -= shift;
    const double r = fma(inv_ln2_n, xd, -kd);
    sb = EXP2F_TAB[ki % 32] + (ki << 47);
    double s;
    memcpy(&s, &sb, 8);
    const double z = fma(c0, r, c1), r2 = r * r;
    const double y = fma(z, r2, fma(c2, r, 1.0));
    return (float)(y * s);
}

/* Inputs u = 0, step, 2 step, ... (all 2^32 bit patterns at step 1) where the
 * restatement differs from the host's expf (NaN results compared as NaN). */
uint64_t vko_expf_form_mismatches(uint32_t step) {
    uint64_t bad = 0;
    if (step == 0) step = 1;
#pragma omp parallel for OMP_THREADS reduction(+ : bad) schedule(static)
    for (long long u = 0; u < (1LL << 32); u += step) {
        const uint32_t b = (uint32_t)u;
        float x, e, c;
        memcpy(&x, &b, 4);
        e = expf(x);
        c = vko_expf_glibc_form(x);
        if (isnan(e) && isnan(c)) continue;
        uint32_t be, bc;
        memcpy(&be, &e, 4);
        memcpy(&bc, &c, 4);
        bad += be != bc;
    }
    return bad;
}

/* src/scalar.rs:126-134 -- Abramowitz-Stegun 7.1.26, every op separately rounded. */
float vko_erf(float x) {
    float s = isnan(x) ? x : copysignf(1.0f, x); /* f32::signum */
    x = fabsf(x);
    float t = 1.0f / (1.0f + 0.3275911f * x);
    float poly = (((((1.0614054f * t - 1.453152f) * t) + 1.4214137f) * t - 0.28449674f) * t +
                  0.2548296f);
    float y = 1.0f - poly * t * expf(-x * x);
    return s * y;
}

/* src/scalar.rs:116-121 */
void vko_gelu(float *x, size_t n) {
    const float inv_sqrt2 = 0.70710677f; /* core::f32::consts::FRAC_1_SQRT_2 */
    for (size_t i = 0; i < n; i++) x[i] = 0.5f * x[i] * (1.0f + vko_erf(x[i] * inv_sqrt2));
}

/* src/scalar.rs:139-155 */
void vko_layerscale(float *x, size_t rows, size_t cols, const float *gamma) {
#pragma omp parallel for OMP_THREADS if (rows >= 32)
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < cols; c++) x[r * cols + c] *= gamma[c];
}

/* src/scalar.rs:157-172 */
void vko_softmax_rows(float *x, size_t rows, size_t cols) {
    for (size_t r = 0; r < rows; r++) {
        float *row = x + r * cols;
        float m = -INFINITY;
        for (size_t c = 0; c < cols; c++) m = rmax(m, row[c]);
        float sum = 0.0f;
        for (size_t c = 0; c < cols; c++) {
            row[c] = expf(row[c] - m);
            sum += row[c];
        }
        float inv = 1.0f / sum;
        for (size_t c = 0; c < cols; c++) row[c] *= inv;
    }
}

/* ------------------------------------------------------------------------ */
/* Q8_0                                                                     */
/* ------------------------------------------------------------------------ */

/* src/q8_0_dot.rs:27-46 */
void vko_quantize_row_q8_0(const float *x, size_t nblocks, vko_block_q8_0 *out) {
    for (size_t bi = 0; bi < nblocks; bi++) {
        const float *src = x + bi * VKO_QK8_0;
        float amax = 0.0f;
        for (int j = 0; j < VKO_QK8_0; j++) amax = rmax(amax, fabsf(src[j]));
        float d = amax / 127.0f;
        float inv = d != 0.0f ? 1.0f / d : 0.0f;
        out[bi].d = vko_f32_to_f16(d);
        for (int j = 0; j < VKO_QK8_0; j++) {
            float q = roundf(src[j] * inv); /* f32::round: half away from zero */
            if (isnan(q)) {
                out[bi].qs[j] = 0; /* `NaN as i8` saturates to 0 */
            } else {
                q = q < -127.0f ? -127.0f : (q > 127.0f ? 127.0f : q);
                out[bi].qs[j] = (int8_t)q;
            }
        }
    }
}

/* src/lib.rs:42-50 */
void vko_dequantize_q8_0(const vko_block_q8_0 *blocks, size_t nblocks, float *out) {
    for (size_t b = 0; b < nblocks; b++) {
        float scale = vko_f16_to_f32(blocks[b].d);
        for (int j = 0; j < VKO_QK8_0; j++) out[b * VKO_QK8_0 + j] = scale * (float)blocks[b].qs[j];
    }
}

/* src/simd_avx512.rs:262-280 -- dpbusd on a 64-byte pair, split into two block sums. */
__attribute__((target("avx512f,avx512bw,avx512vnni"))) static inline void
dpbusd_pair_halves(__m512i bx, __m512i by, int32_t *s0, int32_t *s1) {
    const __m512i off = _mm512_set1_epi8((char)-128);
    __m512i ax = _mm512_xor_si512(bx, off);
    const __m512i ones = _mm512_set1_epi8(1);
    const __m512i zero = _mm512_setzero_si512();
    __m512i dot = _mm512_dpbusd_epi32(zero, ax, by);
    __m512i sumb = _mm512_dpbusd_epi32(zero, ones, by);
    int32_t dot_lo = _mm512_reduce_add_epi32(_mm512_maskz_mov_epi32(0x00FF, dot));
    int32_t dot_hi = _mm512_reduce_add_epi32(_mm512_maskz_mov_epi32(0xFF00, dot));
    int32_t sb_lo = _mm512_reduce_add_epi32(_mm512_maskz_mov_epi32(0x00FF, sumb));
    int32_t sb_hi = _mm512_reduce_add_epi32(_mm512_maskz_mov_epi32(0xFF00, sumb));
    *s0 = dot_lo - 128 * sb_lo;
    *s1 = dot_hi - 128 * sb_hi;
}

/* src/simd_avx512.rs:295-351 -- two blocks per VNNI step; scalar tail block. */
__attribute__((target("avx512f,avx512bw,avx512vnni"))) void
vko_gemm_q8_0_avx512(size_t m, size_t n, size_t k, const vko_block_q8_0 *a_q,
                     const vko_block_q8_0 *b_q, float *c) {
    size_t bpr = k / VKO_QK8_0;
    size_t pairs = bpr / 2;
    int has_tail = (int)(bpr % 2);
    /* The reference runs this single-threaded; rows are independent, so
     * splitting them over threads cannot change any output bit. */
#pragma omp parallel for OMP_THREADS schedule(static)
    for (size_t i = 0; i < m; i++) {
        const vko_block_q8_0 *ar = a_q + i * bpr;
        for (size_t j = 0; j < n; j++) {
            const vko_block_q8_0 *br = b_q + j * bpr;
            float acc = 0.0f;
            for (size_t p = 0; p < pairs; p++) {
                size_t idx = p * 2;
                int8_t abuf[64], bbuf[64];
                memcpy(abuf, ar[idx].qs, 32);
                memcpy(abuf + 32, ar[idx + 1].qs, 32);
                memcpy(bbuf, br[idx].qs, 32);
                memcpy(bbuf + 32, br[idx + 1].qs, 32);
                int32_t s0, s1;
                dpbusd_pair_halves(_mm512_loadu_si512(abuf), _mm512_loadu_si512(bbuf), &s0, &s1);
                acc += vko_f16_to_f32(ar[idx].d) * vko_f16_to_f32(br[idx].d) * (float)s0;
                acc += vko_f16_to_f32(ar[idx + 1].d) * vko_f16_to_f32(br[idx + 1].d) * (float)s1;
            }
            if (has_tail) {
                const vko_block_q8_0 *ab = &ar[bpr - 1], *bb = &br[bpr - 1];
                int32_t isum = 0;
                for (int l = 0; l < VKO_QK8_0; l++) isum += (int32_t)ab->qs[l] * (int32_t)bb->qs[l];
                acc += vko_f16_to_f32(ab->d) * vko_f16_to_f32(bb->d) * (float)isum;
            }
            c[i * n + j] = acc;
        }
    }
}

void vko_kernels_gemm_q8_0(size_t m, size_t n, size_t k, const vko_block_q8_0 *a_q,
                           const vko_block_q8_0 *b_q, float *c) {
    if (vko_has_avx512())
        vko_gemm_q8_0_avx512(m, n, k, a_q, b_q, c);
    else
        vko_gemm_q8_0(m, n, k, a_q, b_q, c);
}

/* ------------------------------------------------------------------------ */
/* Cephes exp (src/simd_avx512.rs:22-69 == src/specialized.rs:2700-2744)    */
/* ------------------------------------------------------------------------ */

#define CEPHES_HI 88.37626f
#define CEPHES_LO (-88.37626f)
#define CEPHES_LOG2EF 1.44269504f
#define CEPHES_LN2_HI 0.693359375f
#define CEPHES_LN2_LO (-2.1219444e-4f)
#define CEPHES_P0 1.98756915e-4f
#define CEPHES_P1 1.39819995e-3f
#define CEPHES_P2 8.3334519e-3f
#define CEPHES_P3 4.1665796e-2f
#define CEPHES_P4 1.6666665e-1f
#define CEPHES_P5 5.0000001e-1f

/* Scalar restatement lane by lane: x86 min/max return the second operand
 * when either is NaN; cvttps truncates toward zero. */
static inline float cephes_exp_scalar(float x) {
    x = (x < CEPHES_HI) ? x : CEPHES_HI;
    x = (x > CEPHES_LO) ? x : CEPHES_LO;
    float fx0 = fmaf(x, CEPHES_LOG2EF, 0.5f);
    float tr = (float)(int32_t)fx0;
    float fx = (tr > fx0) ? tr - 1.0f : tr;
    x = fmaf(-fx, CEPHES_LN2_HI, x);
    x = fmaf(-fx, CEPHES_LN2_LO, x);
    float z = x * x;
    float y = CEPHES_P0;
    y = fmaf(y, x, CEPHES_P1);
    y = fmaf(y, x, CEPHES_P2);
    y = fmaf(y, x, CEPHES_P3);
    y = fmaf(y, x, CEPHES_P4);
    y = fmaf(y, x, CEPHES_P5);
    y = fmaf(y, z, x);
    y = y + 1.0f;
    int32_t e = ((int32_t)fx + 0x7f) << 23;
    float p2;
    memcpy(&p2, &e, 4);
    return y * p2;
}

float vko_cephes_exp(float x) { return cephes_exp_scalar(x); }

__attribute__((target("avx512f,fma"))) static inline __m512 exp_avx512(__m512 x) {
    const __m512 one = _mm512_set1_ps(1.0f);
    x = _mm512_min_ps(x, _mm512_set1_ps(CEPHES_HI));
    x = _mm512_max_ps(x, _mm512_set1_ps(CEPHES_LO));
    __m512 fx0 = _mm512_fmadd_ps(x, _mm512_set1_ps(CEPHES_LOG2EF), _mm512_set1_ps(0.5f));
    __m512 tr = _mm512_cvtepi32_ps(_mm512_cvttps_epi32(fx0));
    __mmask16 gt = _mm512_cmp_ps_mask(tr, fx0, _CMP_GT_OQ);
    __m512 fx = _mm512_mask_sub_ps(tr, gt, tr, one);
    x = _mm512_fnmadd_ps(fx, _mm512_set1_ps(CEPHES_LN2_HI), x);
    x = _mm512_fnmadd_ps(fx, _mm512_set1_ps(CEPHES_LN2_LO), x);
    __m512 z = _mm512_mul_ps(x, x);
    __m512 y = _mm512_set1_ps(CEPHES_P0);
    y = _mm512_fmadd_ps(y, x, _mm512_set1_ps(CEPHES_P1));
    y = _mm512_fmadd_ps(y, x, _mm512_set1_ps(CEPHES_P2));
    y = _mm512_fmadd_ps(y, x, _mm512_set1_ps(CEPHES_P3));
    y = _mm512_fmadd_ps(y, x, _mm512_set1_ps(CEPHES_P4));
    y = _mm512_fmadd_ps(y, x, _mm512_set1_ps(CEPHES_P5));
    y = _mm512_fmadd_ps(y, z, x);
    y = _mm512_add_ps(y, one);
    __m512i e = _mm512_slli_epi32(_mm512_add_epi32(_mm512_cvttps_epi32(fx), _mm512_set1_epi32(0x7f)), 23);
    return _mm512_mul_ps(y, _mm512_castsi512_ps(e));
}

/* ------------------------------------------------------------------------ */
/* AVX-512 GELU (src/simd_avx512.rs:141-209) and Kernels dispatch           */
/* ------------------------------------------------------------------------ */

#define ERF_A1 0.25482959f
#define ERF_A2 (-0.28449674f)
#define ERF_A3 1.4214137f
#define ERF_A4 (-1.4531520f)
#define ERF_A5 1.0614054f
#define ERF_C 0.3275911f

__attribute__((target("avx512f,fma"))) static inline __m512 erf_avx512(__m512 x) {
    const __m512 zero = _mm512_setzero_ps(), one = _mm512_set1_ps(1.0f);
    __m512 xa = _mm512_castsi512_ps(
        _mm512_and_epi32(_mm512_castps_si512(x), _mm512_set1_epi32(0x7fffffff)));
    __mmask16 neg = _mm512_cmp_ps_mask(x, zero, _CMP_LT_OQ);
    __m512 sign = _mm512_mask_blend_ps(neg, one, _mm512_set1_ps(-1.0f));
    __m512 t = _mm512_div_ps(one, _mm512_fmadd_ps(_mm512_set1_ps(ERF_C), xa, one));
    __m512 poly = _mm512_set1_ps(ERF_A5);
    poly = _mm512_fmadd_ps(poly, t, _mm512_set1_ps(ERF_A4));
    poly = _mm512_fmadd_ps(poly, t, _mm512_set1_ps(ERF_A3));
    poly = _mm512_fmadd_ps(poly, t, _mm512_set1_ps(ERF_A2));
    poly = _mm512_fmadd_ps(poly, t, _mm512_set1_ps(ERF_A1));
    poly = _mm512_mul_ps(poly, t);
    __m512 e = exp_avx512(_mm512_sub_ps(zero, _mm512_mul_ps(xa, xa)));
    __m512 y = _mm512_fnmadd_ps(poly, e, one);
    return _mm512_mul_ps(sign, y);
}

__attribute__((target("avx512f,fma"))) void vko_gelu_avx512(float *x, size_t n) {
    const __m512 inv_sqrt2 = _mm512_set1_ps(0.70710678f), half = _mm512_set1_ps(0.5f),
                 one = _mm512_set1_ps(1.0f);
    size_t main = n - (n % 16);
    for (size_t i = 0; i < main; i += 16) {
        __m512 v = _mm512_loadu_ps(x + i);
        __m512 e = erf_avx512(_mm512_mul_ps(v, inv_sqrt2));
        _mm512_storeu_ps(x + i, _mm512_mul_ps(_mm512_mul_ps(half, v), _mm512_add_ps(one, e)));
    }
    if (main < n) vko_gelu(x + main, n - main);
}

/* gelu_avx512's arithmetic restated lane by lane in scalar code (FMA where
 * the intrinsics fuse), so hosts without AVX-512 can still check it. */
static inline float gelu_avx512_lane(float v) {
    float a = v * 0.70710678f;
    float xa = fabsf(a);
    float sign = (a < 0.0f) ? -1.0f : 1.0f;
    float t = 1.0f / fmaf(ERF_C, xa, 1.0f);
    float poly = ERF_A5;
    poly = fmaf(poly, t, ERF_A4);
    poly = fmaf(poly, t, ERF_A3);
    poly = fmaf(poly, t, ERF_A2);
    poly = fmaf(poly, t, ERF_A1);
    poly = poly * t;
    float e = cephes_exp_scalar(0.0f - xa * xa);
    float y = fmaf(-poly, e, 1.0f);
    return (0.5f * v) * (1.0f + sign * y);
}

void vko_gelu_avx512_lanes(float *x, size_t n) {
    size_t main = n - (n % 16);
#pragma omp parallel for OMP_THREADS schedule(static) if (n >= 65536)
    for (size_t i = 0; i < main; i++) x[i] = gelu_avx512_lane(x[i]);
    if (main < n) vko_gelu(x + main, n - main);
}

/* src/dispatch.rs:56-73 -- AVX-512 tier: par_chunks_mut(4096) of gelu_avx512. */
void vko_kernels_gelu(float *x, size_t n) {
    if (!vko_has_avx512()) {
        vko_gelu(x, n);
        return;
    }
    size_t chunks = (n + 4095) / 4096;
#pragma omp parallel for OMP_THREADS schedule(static)
    for (size_t c = 0; c < chunks; c++) {
        size_t lo = c * 4096, hi = lo + 4096 < n ? lo + 4096 : n;
        vko_gelu_avx512(x + lo, hi - lo);
    }
}

/* src/dispatch.rs:77-83 -> add_avx512 (src/simd_avx512.rs:215-235): one add
 * per element either way, bit-identical to scalar::add. */
void vko_kernels_add(float *dst, const float *src, size_t n) {
#pragma omp parallel for OMP_THREADS schedule(static) if (n >= 65536)
    for (size_t i = 0; i < n; i++) dst[i] += src[i];
}

/* ------------------------------------------------------------------------ */
/* RoPE                                                                     */
/* ------------------------------------------------------------------------ */

/* src/rope.rs:84-93 */
static inline void rotate_half(float *s, size_t quarter, const float *rot) {
    for (size_t i = 0; i < quarter; i++) {
        float sn = rot[i * 2], cs = rot[i * 2 + 1];
        float a = s[i], b = s[i + quarter];
        s[i] = a * cs - b * sn;
        s[i + quarter] = b * cs + a * sn;
    }
}

/* src/rope.rs:30-80 */
void vko_rope2d(float *x, size_t heads, size_t n, size_t head_dim, const int64_t *pos_yx,
                float freq) {
    size_t half = head_dim / 2, quarter = half / 2;
    float *inv_freq = (float *)malloc(quarter * sizeof(float));
    for (size_t i = 0; i < quarter; i++)
        inv_freq[i] = powf(freq, -2.0f * (float)i / (float)half);
    float *rot = (float *)malloc(n * 2 * quarter * 2 * sizeof(float));
    for (size_t p = 0; p < n; p++) {
        float pos[2] = {(float)pos_yx[2 * p], (float)pos_yx[2 * p + 1]};
        for (int axis = 0; axis < 2; axis++)
            for (size_t i = 0; i < quarter; i++) {
                float arg = pos[axis] * inv_freq[i];
                size_t off = (p * 2 * quarter + axis * quarter + i) * 2;
                rot[off] = sinf(arg);
                rot[off + 1] = cosf(arg);
            }
        for (size_t h = 0; h < heads; h++) {
            float *base = x + (h * n + p) * head_dim;
            rotate_half(base, quarter, rot + (p * 2 * quarter) * 2);
            rotate_half(base + half, quarter, rot + (p * 2 * quarter + quarter) * 2);
        }
    }
    free(rot);
    free(inv_freq);
}

/* src/specialized.rs:389-410 (QUARTER 16, HALF_DIM 32) */
void vko_rope_rotations(const int64_t *pos_yx, size_t tokens, float freq, float *rot) {
    float inv_freq[16];
    for (int i = 0; i < 16; i++) inv_freq[i] = powf(freq, -2.0f * (float)i / 32.0f);
    for (size_t t = 0; t < tokens; t++)
        for (int axis = 0; axis < 2; axis++)
            for (int i = 0; i < 16; i++) {
                float arg = (float)pos_yx[2 * t + axis] * inv_freq[i];
                size_t off = (t * 32 + (size_t)axis * 16 + (size_t)i) * 2;
                rot[off] = sinf(arg);
                rot[off + 1] = cosf(arg);
            }
}

/* src/specialized.rs:412-454 -- per 64-wide row: scalar LN then rotation.
 * The reference indexes the table with row % 865; `tokens` generalises it. */
static void normalize_and_rotate(float *values, size_t rows, size_t tokens, const float *gamma,
                                 const float *beta, float eps, const float *rot) {
#pragma omp parallel for OMP_THREADS schedule(static)
    for (size_t r = 0; r < rows; r++) {
        float *d = values + r * 64;
        float sum = RUST_SUM_INIT;
        for (int i = 0; i < 64; i++) sum += d[i];
        float mean = sum / 64.0f;
        float sq = RUST_SUM_INIT;
        for (int i = 0; i < 64; i++) {
            float t = d[i] - mean;
            sq += t * t;
        }
        float var = sq / 64.0f;
        float inv = 1.0f / sqrtf(var + eps);
        for (int i = 0; i < 64; i++) d[i] = (d[i] - mean) * inv * gamma[i] + beta[i];
        size_t tok = r % tokens;
        for (int axis = 0; axis < 2; axis++)
            rotate_half(d + axis * 32, 16, rot + (tok * 32 + (size_t)axis * 16) * 2);
    }
}

void vko_qk_norm_rope(float *q, float *k, size_t heads, size_t tokens, const float *q_gamma,
                      const float *q_beta, const float *k_gamma, const float *k_beta,
                      const int64_t *pos_yx, float freq, float eps) {
    float *rot = (float *)malloc(tokens * 64 * sizeof(float));
    vko_rope_rotations(pos_yx, tokens, freq, rot);
    normalize_and_rotate(q, heads * tokens, tokens, q_gamma, q_beta, eps, rot);
    normalize_and_rotate(k, heads * tokens, tokens, k_gamma, k_beta, eps, rot);
    free(rot);
}

/* ------------------------------------------------------------------------ */
/* attention                                                                */
/* ------------------------------------------------------------------------ */

/* src/attention.rs:10-59 */
void vko_attention_naive(const float *q, const float *k, const float *v, size_t heads, size_t n,
                         size_t hd, float *out) {
    float scale = 1.0f / sqrtf((float)hd);
    float *scores = (float *)malloc(n * sizeof(float));
    for (size_t h = 0; h < heads; h++) {
        const float *qh = q + h * n * hd, *kh = k + h * n * hd, *vh = v + h * n * hd;
        float *oh = out + h * n * hd;
        for (size_t i = 0; i < n; i++) {
            const float *qi = qh + i * hd;
            float mx = -INFINITY;
            for (size_t j = 0; j < n; j++) {
                const float *kj = kh + j * hd;
                float dot = RUST_SUM_INIT;
                for (size_t d = 0; d < hd; d++) dot += qi[d] * kj[d];
                float s = dot * scale;
                scores[j] = s;
                if (s > mx) mx = s;
            }
            float sum = 0.0f;
            for (size_t j = 0; j < n; j++) {
                scores[j] = expf(scores[j] - mx);
                sum += scores[j];
            }
            float inv = 1.0f / sum;
            float *oi = oh + i * hd;
            for (size_t d = 0; d < hd; d++) oi[d] = 0.0f;
            for (size_t j = 0; j < n; j++) {
                float w = scores[j] * inv;
                const float *vj = vh + j * hd;
                for (size_t d = 0; d < hd; d++) oi[d] += w * vj[d];
            }
        }
    }
    free(scores);
}

/* src/simd_avx512.rs:93-115 -- 16 lanes of mul+add, sequential lane sum, tail. */
__attribute__((target("avx512f"))) static inline float dot_avx512(const float *a, const float *b,
                                                                   size_t len) {
    size_t main = len - (len % 16);
    __m512 lanes = _mm512_setzero_ps();
    for (size_t i = 0; i < main; i += 16)
        lanes = _mm512_add_ps(lanes, _mm512_mul_ps(_mm512_loadu_ps(a + i), _mm512_loadu_ps(b + i)));
    float part[16];
    _mm512_storeu_ps(part, lanes);
    float sum = RUST_SUM_INIT;
    for (int i = 0; i < 16; i++) sum += part[i];
    for (size_t i = main; i < len; i++) sum += a[i] * b[i];
    return sum;
}

/* src/simd_avx512.rs:120-134 */
__attribute__((target("avx512f"))) static inline void scaled_add_avx512(float *dst, float s,
                                                                         const float *src,
                                                                         size_t len) {
    __m512 sv = _mm512_set1_ps(s);
    size_t main = len - (len % 16);
    for (size_t i = 0; i < main; i += 16)
        _mm512_storeu_ps(dst + i, _mm512_add_ps(_mm512_loadu_ps(dst + i),
                                                _mm512_mul_ps(_mm512_loadu_ps(src + i), sv)));
    for (size_t i = main; i < len; i++) dst[i] += s * src[i];
}

/* src/simd_avx512.rs:75-86 */
__attribute__((target("avx512f,fma"))) static inline void exp_in_place_avx512(float *x,
                                                                               size_t len) {
    size_t main = len - (len % 16);
    for (size_t i = 0; i < main; i += 16) _mm512_storeu_ps(x + i, exp_avx512(_mm512_loadu_ps(x + i)));
    for (size_t i = main; i < len; i++) x[i] = expf(x[i]);
}

#define KV_TILE 64 /* src/attention.rs:61 */

/* src/attention.rs:111-201 -- one (head, query) row of the generic online softmax. */
static void attention_row(const float *qh, const float *kh, const float *vh, size_t i, size_t n,
                          size_t hd, float scale, int use_avx512, float *acc, float *oi) {
    const float *qi = qh + i * hd;
    float rmaxv = -INFINITY, rsum = 0.0f;
    for (size_t d = 0; d < hd; d++) acc[d] = 0.0f;
    for (size_t j0 = 0; j0 < n;) {
        size_t j1 = j0 + KV_TILE < n ? j0 + KV_TILE : n;
        float ls[KV_TILE];
        memset(ls, 0, sizeof(ls));
        float tmax = -INFINITY;
        for (size_t j = j0; j < j1; j++) {
            const float *kj = kh + j * hd;
            float dot;
            if (use_avx512) {
                dot = dot_avx512(qi, kj, hd);
            } else {
                dot = RUST_SUM_INIT;
                for (size_t d = 0; d < hd; d++) dot += qi[d] * kj[d];
            }
            float s = dot * scale;
            ls[j - j0] = s;
            if (s > tmax) tmax = s;
        }
        float nmax = rmax(rmaxv, tmax);
        float corr = isfinite(rmaxv) ? expf(rmaxv - nmax) : 0.0f;
        rsum *= corr;
        for (size_t d = 0; d < hd; d++) acc[d] *= corr;
        for (size_t t = 0; t < j1 - j0; t++) ls[t] -= nmax;
        if (use_avx512) {
            exp_in_place_avx512(ls, j1 - j0);
        } else {
            for (size_t t = 0; t < j1 - j0; t++) ls[t] = expf(ls[t]);
        }
        for (size_t j = j0; j < j1; j++) {
            float p = ls[j - j0];
            rsum += p;
            const float *vj = vh + j * hd;
            if (use_avx512) {
                scaled_add_avx512(acc, p, vj, hd);
            } else {
                for (size_t d = 0; d < hd; d++) acc[d] += p * vj[d];
            }
        }
        rmaxv = nmax;
        j0 = j1;
    }
    float inv = 1.0f / rsum;
    for (size_t d = 0; d < hd; d++) oi[d] = acc[d] * inv;
}

static void attention_rows(const float *q, const float *k, const float *v, size_t heads, size_t n,
                           size_t hd, float *out, int use_avx512, int parallel) {
    float scale = 1.0f / sqrtf((float)hd);
    size_t rows = heads * n;
#pragma omp parallel OMP_THREADS if (parallel)
    {
        float *acc = (float *)malloc(hd * sizeof(float));
#pragma omp for schedule(dynamic, 64)
        for (size_t row = 0; row < rows; row++) {
            size_t h = row / n, i = row % n, base = h * n * hd;
            attention_row(q + base, k + base, v + base, i, n, hd, scale, use_avx512, acc,
                          out + row * hd);
        }
        free(acc);
    }
}

/* src/attention.rs:204-233 */
void vko_attention_serial(const float *q, const float *k, const float *v, size_t heads, size_t n,
                          size_t hd, float *out) {
    attention_rows(q, k, v, heads, n, hd, out, 0, 0);
}

/* ---- DA3 flash attention ------------------------------------------------ */

/* One panel's arithmetic for one query row, restating
 * src/specialized.rs:1400-1562 (QT8 tile) with the micro-GEMMs of 2331-2608:
 * s_j = fma chain over d from +0; s *= 1/8 (valid); running max/sum with glibc
 * expf correction; Cephes exp on all 64 lanes (invalid lanes hold +0 -> 1);
 * acc_d = fma chain over the 64 panel keys with zero V rows past the tail. */
static void flash_row_scalar(const float *qi, const float *kh, const float *vh, size_t tokens,
                             float *oi) {
    float acc[64], sc[64];
    for (int d = 0; d < 64; d++) acc[d] = 0.0f;
    float sum = 0.0f, mx = -INFINITY;
    for (size_t k0 = 0; k0 < tokens; k0 += 64) {
        size_t cols = tokens - k0 < 64 ? tokens - k0 : 64;
        for (size_t c = 0; c < 64; c++) {
            float s = 0.0f;
            if (c < cols) {
                const float *kj = kh + (k0 + c) * 64;
                for (int d = 0; d < 64; d++) s = fmaf(qi[d], kj[d], s);
            }
            sc[c] = s;
        }
        float tmax = -INFINITY;
        for (size_t c = 0; c < cols; c++) {
            sc[c] *= 0.125f;
            tmax = rmax(tmax, sc[c]);
        }
        float nmax = rmax(mx, tmax);
        float corr = isfinite(mx) ? expf(mx - nmax) : 0.0f;
        sum *= corr;
        for (int d = 0; d < 64; d++) acc[d] *= corr;
        for (size_t c = 0; c < cols; c++) sc[c] -= nmax;
        for (int c = 0; c < 64; c++) sc[c] = cephes_exp_scalar(sc[c]);
        for (size_t c = 0; c < cols; c++) sum += sc[c];
        mx = nmax;
        for (int d = 0; d < 64; d++) {
            float a = acc[d];
            for (size_t c = 0; c < 64; c++) a = fmaf(sc[c], c < cols ? vh[(k0 + c) * 64 + d] : 0.0f, a);
            acc[d] = a;
        }
    }
    float inv = 1.0f / sum;
    for (int d = 0; d < 64; d++) oi[d] = acc[d] * inv;
}

void vko_flash_attention_scalar(const float *q, const float *k, const float *v, size_t heads,
                                size_t tokens, float *out) {
    size_t rows = heads * tokens;
#pragma omp parallel for OMP_THREADS schedule(dynamic, 16)
    for (size_t row = 0; row < rows; row++) {
        size_t h = row / tokens, base = h * tokens * 64;
        flash_row_scalar(q + row * 64, k + base, v + base, tokens, out + row * 64);
    }
}

/* src/specialized.rs:2331-2362 gemm_8x32_overwrite_stride */
__attribute__((target("avx512f,fma"))) static void
gemm_8x32_overwrite_stride(const float *a, const float *b, size_t stride, size_t column,
                           float *c) {
    for (int col0 = 0; col0 < 64; col0 += 32) {
        __m512 acc[8][2];
        for (int r = 0; r < 8; r++) acc[r][0] = acc[r][1] = _mm512_setzero_ps();
        for (int kk = 0; kk < 64; kk++) {
            const float *bp = b + (size_t)kk * stride + column + col0;
            __m512 b0 = _mm512_loadu_ps(bp), b1 = _mm512_loadu_ps(bp + 16);
            for (int r = 0; r < 8; r++) {
                __m512 av = _mm512_set1_ps(a[r * 64 + kk]);
                acc[r][0] = _mm512_fmadd_ps(av, b0, acc[r][0]);
                acc[r][1] = _mm512_fmadd_ps(av, b1, acc[r][1]);
            }
        }
        for (int r = 0; r < 8; r++) {
            _mm512_storeu_ps(c + r * 64 + col0, acc[r][0]);
            _mm512_storeu_ps(c + r * 64 + col0 + 16, acc[r][1]);
        }
    }
}

/* src/specialized.rs:2403-2463 gemm_4x64_overwrite_stride (masked tail loads) */
__attribute__((target("avx512f,fma"))) static void
gemm_4x64_overwrite_stride(size_t m, const float *a, const float *b, size_t stride, size_t column,
                           size_t columns, float *c) {
    for (size_t row0 = 0; row0 < m; row0 += 4) {
        size_t rows = m - row0 < 4 ? m - row0 : 4;
        __m512 acc[4][4];
        for (int r = 0; r < 4; r++)
            for (int q = 0; q < 4; q++) acc[r][q] = _mm512_setzero_ps();
        for (int kk = 0; kk < 64; kk++) {
            const float *bp = b + (size_t)kk * stride + column;
            __m512 bv[4];
            for (int q = 0; q < 4; q++) {
                size_t rem = columns > (size_t)q * 16 ? columns - (size_t)q * 16 : 0;
                if (rem > 16) rem = 16;
                __mmask16 mk = rem == 16 ? (__mmask16)0xFFFF : (__mmask16)((1u << rem) - 1u);
                bv[q] = columns == 64 ? _mm512_loadu_ps(bp + q * 16) : _mm512_maskz_loadu_ps(mk, bp + q * 16);
            }
            for (size_t r = 0; r < rows; r++) {
                __m512 av = _mm512_set1_ps(a[(row0 + r) * 64 + kk]);
                for (int q = 0; q < 4; q++) acc[r][q] = _mm512_fmadd_ps(av, bv[q], acc[r][q]);
            }
        }
        for (size_t r = 0; r < rows; r++)
            for (int q = 0; q < 4; q++) _mm512_storeu_ps(c + (row0 + r) * 64 + q * 16, acc[r][q]);
    }
}

/* src/specialized.rs:2578-2608 gemm_8x32_accumulate */
__attribute__((target("avx512f,fma"))) static void gemm_8x32_accumulate(const float *a,
                                                                         const float *b, float *c) {
    for (int col0 = 0; col0 < 64; col0 += 32) {
        __m512 acc[8][2];
        for (int r = 0; r < 8; r++) {
            acc[r][0] = _mm512_loadu_ps(c + r * 64 + col0);
            acc[r][1] = _mm512_loadu_ps(c + r * 64 + col0 + 16);
        }
        for (int kk = 0; kk < 64; kk++) {
            const float *bp = b + kk * 64 + col0;
            __m512 b0 = _mm512_loadu_ps(bp), b1 = _mm512_loadu_ps(bp + 16);
            for (int r = 0; r < 8; r++) {
                __m512 av = _mm512_set1_ps(a[r * 64 + kk]);
                acc[r][0] = _mm512_fmadd_ps(av, b0, acc[r][0]);
                acc[r][1] = _mm512_fmadd_ps(av, b1, acc[r][1]);
            }
        }
        for (int r = 0; r < 8; r++) {
            _mm512_storeu_ps(c + r * 64 + col0, acc[r][0]);
            _mm512_storeu_ps(c + r * 64 + col0 + 16, acc[r][1]);
        }
    }
}

/* src/specialized.rs:2533-2574 gemm_4x64_accumulate */
__attribute__((target("avx512f,fma"))) static void gemm_4x64_accumulate(size_t m, const float *a,
                                                                         const float *b, float *c) {
    for (size_t row0 = 0; row0 < m; row0 += 4) {
        size_t rows = m - row0 < 4 ? m - row0 : 4;
        __m512 acc[4][4];
        for (size_t r = 0; r < rows; r++)
            for (int q = 0; q < 4; q++) acc[r][q] = _mm512_loadu_ps(c + (row0 + r) * 64 + q * 16);
        for (int kk = 0; kk < 64; kk++) {
            const float *bp = b + kk * 64;
            __m512 bv[4];
            for (int q = 0; q < 4; q++) bv[q] = _mm512_loadu_ps(bp + q * 16);
            for (size_t r = 0; r < rows; r++) {
                __m512 av = _mm512_set1_ps(a[(row0 + r) * 64 + kk]);
                for (int q = 0; q < 4; q++) acc[r][q] = _mm512_fmadd_ps(av, bv[q], acc[r][q]);
            }
        }
        for (size_t r = 0; r < rows; r++)
            for (int q = 0; q < 4; q++) _mm512_storeu_ps(c + (row0 + r) * 64 + q * 16, acc[r][q]);
    }
}

/* src/specialized.rs:2700-2744 */
__attribute__((target("avx512f,fma"))) static void exp_64_avx512(float *values) {
    for (int b = 0; b < 4; b++) _mm512_storeu_ps(values + b * 16, exp_avx512(_mm512_loadu_ps(values + b * 16)));
}

/* src/specialized.rs:1400-1562 with QT = 8, gemm_8x32 = true, gemm_rows6 = false,
 * persistent dim-major K pack (stride = tokens). */
__attribute__((target("avx512f,fma"))) static void
flash_tile_qt8(const float *q_head, const float *v_head, const float *packed_k, size_t stride,
               size_t tokens, size_t q0, float *out_tile, size_t rows) {
    float accum[8][64];
    float sums[8], maxima[8];
    memset(accum, 0, sizeof(accum));
    for (int r = 0; r < 8; r++) {
        sums[r] = 0.0f;
        maxima[r] = -INFINITY;
    }
    int use_8x32 = rows == 8;
    for (size_t k0 = 0; k0 < tokens; k0 += 64) {
        size_t cols = tokens - k0 < 64 ? tokens - k0 : 64;
        float scores[8][64];
        memset(scores, 0, sizeof(scores));
        const float *qt = q_head + q0 * 64;
        if (use_8x32 && cols == 64)
            gemm_8x32_overwrite_stride(qt, packed_k, stride, k0, &scores[0][0]);
        else
            gemm_4x64_overwrite_stride(rows, qt, packed_k, stride, k0, cols, &scores[0][0]);
        for (size_t r = 0; r < rows; r++) {
            float tmax = -INFINITY;
            for (size_t c = 0; c < cols; c++) {
                scores[r][c] *= 0.125f;
                tmax = rmax(tmax, scores[r][c]);
            }
            float nmax = rmax(maxima[r], tmax);
            float corr = isfinite(maxima[r]) ? expf(maxima[r] - nmax) : 0.0f;
            sums[r] *= corr;
            for (int d = 0; d < 64; d++) accum[r][d] *= corr;
            for (size_t c = 0; c < cols; c++) scores[r][c] -= nmax;
            exp_64_avx512(scores[r]);
            for (size_t c = 0; c < cols; c++) sums[r] += scores[r][c];
            maxima[r] = nmax;
        }
        if (cols == 64) {
            if (use_8x32)
                gemm_8x32_accumulate(&scores[0][0], v_head + k0 * 64, &accum[0][0]);
            else
                gemm_4x64_accumulate(rows, &scores[0][0], v_head + k0 * 64, &accum[0][0]);
        } else {
            float packed_v[64 * 64];
            memset(packed_v, 0, sizeof(packed_v));
            memcpy(packed_v, v_head + k0 * 64, cols * 64 * sizeof(float));
            gemm_4x64_accumulate(rows, &scores[0][0], packed_v, &accum[0][0]);
        }
    }
    for (size_t r = 0; r < rows; r++) {
        float inv = 1.0f / sums[r];
        for (int d = 0; d < 64; d++) out_tile[r * 64 + d] = accum[r][d] * inv;
    }
}

/* src/specialized.rs:1307-1318 pack_key_head_dim_major */
static void pack_key_head_dim_major(const float *k_head, size_t tokens, size_t stride,
                                    float *packed) {
    /* The dense layout has stride == tokens; the final masked panel never
     * reads past `tokens`, but the 64-wide unmasked 8x32 loads of interior
     * panels stay within each dim row as well. */
    for (size_t key = 0; key < tokens; key++)
        for (int d = 0; d < 64; d++) packed[(size_t)d * stride + key] = k_head[key * 64 + d];
}

/* src/specialized.rs:730-765 gate + 1906-2258 default scheduling. */
int vko_flash_attention_avx512(const float *q, const float *k, const float *v, size_t heads,
                               size_t tokens, float *out) {
    if (tokens == 0 || tokens % DA3_TOKENS != 0 || !has_avx512f_fma()) return 0;
    size_t stride = tokens;
    float *packed = (float *)malloc(heads * 64 * stride * sizeof(float));
#pragma omp parallel for OMP_THREADS schedule(static)
    for (size_t h = 0; h < heads; h++)
        pack_key_head_dim_major(k + h * tokens * 64, tokens, stride, packed + h * 64 * stride);
    size_t tiles = (tokens + 7) / 8;
#pragma omp parallel for OMP_THREADS schedule(dynamic, 4)
    for (size_t job = 0; job < heads * tiles; job++) {
        size_t h = job / tiles, t = job % tiles, q0 = t * 8;
        size_t rows = tokens - q0 < 8 ? tokens - q0 : 8;
        size_t base = h * tokens * 64;
        flash_tile_qt8(q + base, v + base, packed + h * 64 * stride, stride, tokens, q0,
                       out + base + q0 * 64, rows);
    }
    free(packed);
    return 1;
}

/* src/attention.rs:66-108 */
void vko_attention(const float *q, const float *k, const float *v, size_t heads, size_t n,
                   size_t hd, float *out) {
    if (hd == 64 && vko_flash_attention_avx512(q, k, v, heads, n, out)) return;
    attention_rows(q, k, v, heads, n, hd, out, has_avx512f_fma(), 1);
}

/* ------------------------------------------------------------------------ */
/* DA3 projections                                                          */
/* ------------------------------------------------------------------------ */

/* Per output: acc = 0; for k ascending acc = fma(a[i,k], b[k,j], acc).
 * This is the arithmetic of every variant in src/specialized.rs:880-1300. */
void vko_linear_fma_scalar(size_t m, size_t n, size_t k, const float *a, const float *b,
                           float *c) {
#pragma omp parallel for OMP_THREADS schedule(static)
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++) {
            float acc = 0.0f;
            for (size_t p = 0; p < k; p++) acc = fmaf(a[i * k + p], b[p * n + j], acc);
            c[i * n + j] = acc;
        }
}

/* One 6-row x 64-column tile: src/specialized.rs:1272-1296 (the inner loop
 * of linear_avx512_column_split_rows<6>).  mode 0: store acc; 1: acc+bias;
 * 2: (acc+bias)*scale.  dst rows are `ldc` apart. */
__attribute__((target("avx512f,fma"))) static inline void
tile_6x64(size_t rows, size_t k, size_t n, const float *a, const float *b, size_t col0, int mode,
          const float *bias, const float *scale, float *dst, size_t ldc) {
    __m512 acc[6][4];
    for (int r = 0; r < 6; r++)
        for (int q = 0; q < 4; q++) acc[r][q] = _mm512_setzero_ps();
    for (size_t kk = 0; kk < k; kk++) {
        const float *bp = b + kk * n + col0;
        __m512 bv0 = _mm512_loadu_ps(bp), bv1 = _mm512_loadu_ps(bp + 16),
               bv2 = _mm512_loadu_ps(bp + 32), bv3 = _mm512_loadu_ps(bp + 48);
        for (size_t r = 0; r < rows; r++) {
            __m512 av = _mm512_set1_ps(a[r * k + kk]);
            acc[r][0] = _mm512_fmadd_ps(av, bv0, acc[r][0]);
            acc[r][1] = _mm512_fmadd_ps(av, bv1, acc[r][1]);
            acc[r][2] = _mm512_fmadd_ps(av, bv2, acc[r][2]);
            acc[r][3] = _mm512_fmadd_ps(av, bv3, acc[r][3]);
        }
    }
    for (size_t r = 0; r < rows; r++)
        for (int q = 0; q < 4; q++) {
            __m512 o = acc[r][q];
            if (mode >= 1) o = _mm512_add_ps(o, _mm512_loadu_ps(bias + col0 + q * 16));
            if (mode == 2) o = _mm512_mul_ps(o, _mm512_loadu_ps(scale + col0 + q * 16));
            _mm512_storeu_ps(dst + r * ldc + q * 16, o);
        }
}

/* linear_avx512_column_split_rows<6> (src/specialized.rs:1252-1300): one
 * 64-column panel per task; any m (rows tail), n % 64 == 0. */
static void linear_avx512(size_t m, size_t n, size_t k, const float *a, const float *b, int mode,
                          const float *bias, const float *scale, float *c) {
    size_t panels = n / 64;
#pragma omp parallel for OMP_THREADS schedule(dynamic, 1)
    for (size_t p = 0; p < panels; p++) {
        size_t col0 = p * 64;
        for (size_t row0 = 0; row0 < m; row0 += 6) {
            size_t rows = m - row0 < 6 ? m - row0 : 6;
            tile_6x64(rows, k, n, a + row0 * k, b, col0, mode, bias, scale, c + row0 * n + col0, n);
        }
    }
}

/* linear_bias_scale_avx512_rows<6> (src/specialized.rs:880-929), the default
 * out-proj / fc2 schedule: one task per 6-row tile, each walking every
 * 64-column panel.  Per output the arithmetic is the column split's. */
static void linear_avx512_rows(size_t m, size_t n, size_t k, const float *a, const float *b,
                               int mode, const float *bias, const float *scale, float *c) {
    size_t tiles = (m + 5) / 6;
#pragma omp parallel for OMP_THREADS schedule(dynamic, 1)
    for (size_t t = 0; t < tiles; t++) {
        size_t row0 = t * 6, rows = m - row0 < 6 ? m - row0 : 6;
        for (size_t col0 = 0; col0 < n; col0 += 64)
            tile_6x64(rows, k, n, a + row0 * k, b, col0, mode, bias, scale, c + row0 * n + col0, n);
    }
}

static void linear_scalar_epilogue(size_t m, size_t n, size_t k, const float *a, const float *b,
                                   int mode, const float *bias, const float *scale, float *c) {
    vko_linear_fma_scalar(m, n, k, a, b, c);
    if (mode == 0) return;
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++) {
            float o = c[i * n + j] + bias[j];
            if (mode == 2) o = o * scale[j];
            c[i * n + j] = o;
        }
}

/* linear_f32_da3_base (src/specialized.rs:770-806) for any m; falls back to
 * the identical-arithmetic scalar form when AVX-512 or n % 64 is missing. */
void vko_linear(size_t m, size_t n, size_t k, const float *a, const float *b, float *c) {
    if (has_avx512f_fma() && n % 64 == 0)
        linear_avx512(m, n, k, a, b, 0, NULL, NULL, c);
    else
        linear_scalar_epilogue(m, n, k, a, b, 0, NULL, NULL, c);
}

/* linear_bias_scale_f32_da3_base (src/specialized.rs:811-929): (acc+bias)*scale. */
void vko_linear_bias_scale(size_t m, size_t n, size_t k, const float *a, const float *b,
                           const float *bias, const float *scale, float *c) {
    if (has_avx512f_fma() && n % 64 == 0)
        linear_avx512_rows(m, n, k, a, b, 2, bias, scale, c);
    else
        linear_scalar_epilogue(m, n, k, a, b, 2, bias, scale, c);
}

/* qkv_avx512_column_split (src/specialized.rs:1101-1167): panel col0 is head
 * (col0%768)/64 of group col0/768; rows written head-major [12][m][64]. */
void vko_qkv(size_t m, const float *a, const float *w, const float *bias, float *q, float *k,
             float *v) {
    const size_t N = 2304, K = 768;
    if (!has_avx512f_fma()) {
        float *tmp = (float *)malloc(m * N * sizeof(float));
        linear_scalar_epilogue(m, N, K, a, w, 1, bias, NULL, tmp);
        vko_split_qkv_hnd(tmp, m, 12, 64, q, k, v);
        free(tmp);
        return;
    }
#pragma omp parallel for OMP_THREADS schedule(dynamic, 1)
    for (size_t p = 0; p < N / 64; p++) {
        size_t col0 = p * 64, group = col0 / 768, head = (col0 % 768) / 64;
        float *dst = group == 0 ? q : (group == 1 ? k : v);
        for (size_t row0 = 0; row0 < m; row0 += 6) {
            size_t rows = m - row0 < 6 ? m - row0 : 6;
            tile_6x64(rows, K, N, a + row0 * K, w, col0, 1, bias, NULL, dst + (head * m + row0) * 64,
                      64);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* layout helpers (semantics of src/cuda.rs:243-276)                        */
/* ------------------------------------------------------------------------ */

void vko_split_qkv_hnd(const float *qkv, size_t tokens, size_t heads, size_t hd, float *q,
                       float *k, float *v) {
    size_t per = heads * hd;
    for (size_t t = 0; t < tokens; t++)
        for (size_t w = 0; w < per; w++) {
            size_t src = t * 3 * per + w;
            size_t hm = (w / hd) * tokens * hd + t * hd + (w % hd);
            q[hm] = qkv[src];
            k[hm] = qkv[src + per];
            v[hm] = qkv[src + 2 * per];
        }
}

void vko_hnd_to_token(const float *hnd, size_t tokens, size_t heads, size_t hd, float *tm) {
    size_t per = heads * hd;
    for (size_t t = 0; t < tokens; t++)
        for (size_t w = 0; w < per; w++) tm[t * per + w] = hnd[(w / hd) * tokens * hd + t * hd + (w % hd)];
}

/* ------------------------------------------------------------------------ */
/* DA3-BASE ViT block (the engine composition of the crate kernels)         */
/* ------------------------------------------------------------------------ */

/* Q8_0 blocks of W^T for W [k][n] row-major: quantize_row_q8_0 of each of
 * the n columns, the pre-transposed row-block operand of Kernels::gemm_q8_0
 * (src/scalar.rs:25-56). */
static vko_block_q8_0 *q8_weight(const float *w, size_t k, size_t n) {
    float *wt = (float *)malloc(k * n * sizeof(float));
    vko_block_q8_0 *q = (vko_block_q8_0 *)malloc(n * (k / 32) * sizeof(vko_block_q8_0));
    for (size_t i = 0; i < k; i++)
        for (size_t j = 0; j < n; j++) wt[j * k + i] = w[i * n + j];
    vko_quantize_row_q8_0(wt, n * (k / 32), q);
    free(wt);
    return q;
}

/* c [m][n] = Kernels::gemm_q8_0(quantize_row_q8_0(a rows), wq) */
static void q8_project(size_t m, size_t n, size_t k, const float *a, const vko_block_q8_0 *wq,
                       float *c) {
    vko_block_q8_0 *aq = (vko_block_q8_0 *)malloc(m * (k / 32) * sizeof(vko_block_q8_0));
    vko_quantize_row_q8_0(a, m * (k / 32), aq);
    vko_kernels_gemm_q8_0(m, n, k, aq, wq, c);
    free(aq);
}

static void vit_block_impl(float *x_all, size_t images, size_t tokens,
                           const vko_block_weights *w, const int64_t *pos_yx, float rope_freq,
                           float eps, float *tap_ln1, float *tap_attn, float *tap_gelu, int q8) {
    const size_t D = 768, H = 12, F = 3072;
    size_t T = tokens;
    vko_block_q8_0 *wq_qkv = NULL, *wq_proj = NULL, *wq_fc1 = NULL, *wq_fc2 = NULL;
    float *qkv = NULL;
    if (q8) {
        wq_qkv = q8_weight(w->w_qkv, D, 3 * D);
        wq_proj = q8_weight(w->w_proj, D, D);
        wq_fc1 = q8_weight(w->w_fc1, D, F);
        wq_fc2 = q8_weight(w->w_fc2, F, D);
        qkv = (float *)malloc(T * 3 * D * sizeof(float));
    }
    float *h = (float *)malloc(T * D * sizeof(float));
    float *qb = (float *)malloc(T * D * sizeof(float));
    float *kb = (float *)malloc(T * D * sizeof(float));
    float *vb = (float *)malloc(T * D * sizeof(float));
    float *ob = (float *)malloc(T * D * sizeof(float));
    float *att = (float *)malloc(T * D * sizeof(float));
    float *y = (float *)malloc(T * D * sizeof(float));
    float *f = (float *)malloc(T * F * sizeof(float));
    for (size_t img = 0; img < images; img++) {
        float *x = x_all + img * T * D;
        /* pre-LN (scalar::layernorm, src/scalar.rs:83) */
        memcpy(h, x, T * D * sizeof(float));
        vko_layernorm(h, T, D, w->ln1_gamma, w->ln1_beta, eps);
        if (tap_ln1) memcpy(tap_ln1 + img * T * D, h, T * D * sizeof(float));
        if (q8) {
            /* Q8_0 QKV, then add_bias_rows, then the head-major split */
            q8_project(T, 3 * D, D, h, wq_qkv, qkv);
            vko_add_bias_rows(qkv, T, 3 * D, w->b_qkv);
            vko_split_qkv_hnd(qkv, T, H, 64, qb, kb, vb);
        } else {
            /* QKV with bias, head-major (src/specialized.rs:996) */
            vko_qkv(T, h, w->w_qkv, w->b_qkv, qb, kb, vb);
        }
        if (w->q_norm_gamma) {
            /* late block: Q/K LayerNorm fused with the RoPE
             * (src/specialized.rs:278-316); without positions every token
             * sits at (0, 0), whose rotation (sin 0, cos 1) is exact identity */
            int64_t *zero = NULL;
            if (!pos_yx) zero = (int64_t *)calloc(T * 2, sizeof(int64_t));
            vko_qk_norm_rope(qb, kb, H, T, w->q_norm_gamma, w->q_norm_beta, w->k_norm_gamma,
                             w->k_norm_beta, pos_yx ? pos_yx : zero, rope_freq, eps);
            free(zero);
        } else if (pos_yx) {
            /* 2-D RoPE on Q and K (src/rope.rs:30) */
            vko_rope2d(qb, H, T, 64, pos_yx, rope_freq);
            vko_rope2d(kb, H, T, 64, pos_yx, rope_freq);
        }
        /* attention (src/attention.rs:66 -> DA3 flash when T % 865 == 0) */
        vko_attention(qb, kb, vb, H, T, 64, ob);
        vko_hnd_to_token(ob, T, H, 64, att);
        if (tap_attn) memcpy(tap_attn + img * T * D, att, T * D * sizeof(float));
        /* out-projection + LayerScale, residual (src/specialized.rs:811, dispatch.rs:77) */
        if (q8) {
            /* (acc + bias) * ls: add_bias_rows then layerscale */
            q8_project(T, D, D, att, wq_proj, y);
            vko_add_bias_rows(y, T, D, w->b_proj);
            vko_layerscale(y, T, D, w->ls1);
        } else {
            vko_linear_bias_scale(T, D, D, att, w->w_proj, w->b_proj, w->ls1, y);
        }
        vko_kernels_add(x, y, T * D);
        /* MLP */
        memcpy(h, x, T * D * sizeof(float));
        vko_layernorm(h, T, D, w->ln2_gamma, w->ln2_beta, eps);
        if (q8)
            q8_project(T, F, D, h, wq_fc1, f);
        else
            vko_linear(T, F, D, h, w->w_fc1, f);
        vko_add_bias_rows(f, T, F, w->b_fc1);
        vko_kernels_gelu(f, T * F);
        if (tap_gelu) memcpy(tap_gelu + img * T * F, f, T * F * sizeof(float));
        if (q8) {
            q8_project(T, D, F, f, wq_fc2, y);
            vko_add_bias_rows(y, T, D, w->b_fc2);
            vko_layerscale(y, T, D, w->ls2);
        } else {
            vko_linear_bias_scale(T, D, F, f, w->w_fc2, w->b_fc2, w->ls2, y);
        }
        vko_kernels_add(x, y, T * D);
    }
    free(wq_qkv);
    free(wq_proj);
    free(wq_fc1);
    free(wq_fc2);
    free(qkv);
    free(h);
    free(qb);
    free(kb);
    free(vb);
    free(ob);
    free(att);
    free(y);
    free(f);
}

void vko_vit_block(float *x_all, size_t images, size_t tokens, const vko_block_weights *w,
                   const int64_t *pos_yx, float rope_freq, float eps, float *tap_ln1,
                   float *tap_attn, float *tap_gelu) {
    vit_block_impl(x_all, images, tokens, w, pos_yx, rope_freq, eps, tap_ln1, tap_attn, tap_gelu,
                   0);
}

void vko_vit_block_q8_0(float *x_all, size_t images, size_t tokens, const vko_block_weights *w,
                        const int64_t *pos_yx, float rope_freq, float eps, float *tap_ln1,
                        float *tap_attn, float *tap_gelu) {
    vit_block_impl(x_all, images, tokens, w, pos_yx, rope_freq, eps, tap_ln1, tap_attn, tap_gelu,
                   1);
}

/* ------------------------------------------------------------------------ */
/* DPT head: convolution, transposed convolution, bilinear resize           */
/* ------------------------------------------------------------------------ */

/* conv::conv2d_naive (src/conv.rs:950-998): direct definition, taps outside
 * the padded input skipped, acc += iv*wv unfused in (ic, ky, kx) order, then
 * the bias.  Output channels run in parallel (each output keeps its order). */
void vko_conv2d_naive(const float *input, size_t in_c, size_t ih, size_t iw, const float *weight,
                      size_t out_c, size_t kh, size_t kw, size_t stride, size_t pad,
                      const float *bias, float *out) {
    const size_t oh = (ih + 2 * pad - kh) / stride + 1, ow = (iw + 2 * pad - kw) / stride + 1;
#pragma omp parallel for OMP_THREADS schedule(static)
    for (size_t oc = 0; oc < out_c; oc++)
        for (size_t oy = 0; oy < oh; oy++)
            for (size_t ox = 0; ox < ow; ox++) {
                float acc = 0.0f;
                for (size_t ic = 0; ic < in_c; ic++)
                    for (size_t ky = 0; ky < kh; ky++) {
                        const long iy = (long)(oy * stride + ky) - (long)pad;
                        if (iy < 0 || iy >= (long)ih) continue;
                        for (size_t kx = 0; kx < kw; kx++) {
                            const long ix = (long)(ox * stride + kx) - (long)pad;
                            if (ix < 0 || ix >= (long)iw) continue;
                            const float iv = input[(ic * ih + (size_t)iy) * iw + (size_t)ix];
                            const float wv = weight[((oc * in_c + ic) * kh + ky) * kw + kx];
                            acc = acc + iv * wv;
                        }
                    }
                if (bias) acc = acc + bias[oc];
                out[(oc * oh + oy) * ow + ox] = acc;
            }
}

/* conv::transformed_winograd_filter (src/conv.rs:121-173): the F(2x2, 3x3)
 * filter transform U = G g G^T of every (oc, ic) 3x3 kernel with
 * G = [[1, 0, 0], [1/2, 1/2, 1/2], [1/2, -1/2, 1/2], [0, 0, 1]], rows first
 * then columns, each sum left to right and then halved, stored
 * U[position][ic][oc] (output channels innermost). */
void vko_winograd_f2_filter(const float *weight, size_t in_c, size_t out_c, float *u) {
    for (size_t oc = 0; oc < out_c; oc++)
        for (size_t ic = 0; ic < in_c; ic++) {
            const float *g = weight + (oc * in_c + ic) * 9;
            float t[4][3], uu[16];
            for (int j = 0; j < 3; j++) {
                const float a = g[j], b = g[3 + j], c = g[6 + j];
                t[0][j] = a;
                t[1][j] = 0.5f * ((a + b) + c);
                t[2][j] = 0.5f * ((a - b) + c);
                t[3][j] = c;
            }
            for (int i = 0; i < 4; i++) {
                const float a = t[i][0], b = t[i][1], c = t[i][2];
                uu[i * 4] = a;
                uu[i * 4 + 1] = 0.5f * ((a + b) + c);
                uu[i * 4 + 2] = 0.5f * ((a - b) + c);
                uu[i * 4 + 3] = c;
            }
            for (int pos = 0; pos < 16; pos++) u[((size_t)pos * in_c + ic) * out_c + oc] = uu[pos];
        }
}

/* specialized::winograd_f2_blocked_f32's AVX-512 product
 * (src/specialized.rs:597-633): per transform position and 16-wide group of
 * output channels, one accumulator per tile, FMA over the input channels in
 * order: m[pos][tile][oc] = fma(u[pos][ic][oc], v[pos][ic][tile], .). */
__attribute__((target("avx512f,fma"))) static void wino_products_avx512(
    const float *u, const float *v, float *m, size_t in_c, size_t out_c, size_t tiles) {
    for (size_t pos = 0; pos < 16; pos++) {
        const float *up = u + pos * in_c * out_c, *vp = v + pos * in_c * tiles;
        float *mp = m + pos * tiles * out_c;
        for (size_t o0 = 0; o0 < out_c; o0 += 16) {
            __m512 acc[8];
            for (size_t t = 0; t < 8; t++) acc[t] = _mm512_setzero_ps();
            for (size_t ic = 0; ic < in_c; ic++) {
                const __m512 f = _mm512_loadu_ps(up + ic * out_c + o0);
                for (size_t t = 0; t < tiles; t++)
                    acc[t] = _mm512_fmadd_ps(f, _mm512_set1_ps(vp[ic * tiles + t]), acc[t]);
            }
            for (size_t t = 0; t < tiles; t++) _mm512_storeu_ps(mp + t * out_c + o0, acc[t]);
        }
    }
}

/* The same product lane by lane (fmaf in the same order), for the bitwise
 * check of the AVX-512 form. */
static void wino_products_lanes(const float *u, const float *v, float *m, size_t in_c,
                                size_t out_c, size_t tiles) {
    for (size_t pos = 0; pos < 16; pos++)
        for (size_t t = 0; t < tiles; t++)
            for (size_t oc = 0; oc < out_c; oc++) {
                float acc = 0.0f;
                for (size_t ic = 0; ic < in_c; ic++)
                    acc = fmaf(u[(pos * in_c + ic) * out_c + oc], v[(pos * in_c + ic) * tiles + t], acc);
                m[(pos * tiles + t) * out_c + oc] = acc;
            }
}

/* The crate's scalar fallback product (src/conv.rs:775-788): unfused
 * sum += u * v from 0 over the input channels. */
static void wino_products_scalar(const float *u, const float *v, float *m, size_t in_c,
                                 size_t out_c, size_t tiles) {
    for (size_t pos = 0; pos < 16; pos++)
        for (size_t t = 0; t < tiles; t++)
            for (size_t oc = 0; oc < out_c; oc++) {
                float sum = 0.0f;
                for (size_t ic = 0; ic < in_c; ic++)
                    sum = sum + u[(pos * in_c + ic) * out_c + oc] * v[(pos * in_c + ic) * tiles + t];
                m[(pos * tiles + t) * out_c + oc] = sum;
            }
}

/* 0: the crate's dispatch (AVX-512 product when avx512f+fma and out_c % 16
 * == 0, else its scalar product); 1: the AVX-512 product restated with fmaf. */
static int g_wino_lanes = 0;
void vko_winograd_use_lanes(int on) { g_wino_lanes = on ? 1 : 0; }

/* conv::conv3x3_winograd_f2_impl (src/conv.rs:681-829): 3x3, stride 1,
 * pad 1, CHW.  Output tiles of 2x2 in row-major order, in blocks of four
 * (winograd_tile_block, src/conv.rs:30-39) run in parallel (at least four
 * blocks per task, src/conv.rs:41-51, here OpenMP chunks of four blocks).
 * Per block:
 *  - input transform B^T d B of each tile's 4x4 patch (zero outside the
 *    image; max(x, 0) first when relu_input), columns then rows, stored
 *    v[position][ic][tile];
 *  - the per-position product over the input channels (above);
 *  - output transform A^T m A, left to right, plus the bias, written to the
 *    tile's 2x2 outputs inside the image. */
void vko_conv3x3_winograd_f2(const float *input, size_t in_c, size_t ih, size_t iw,
                             const float *u, size_t out_c, const float *bias, int relu_input,
                             float *out) {
    const size_t oh = ih, ow = iw, tiles_x = (ow + 1) / 2, tiles_y = (oh + 1) / 2;
    const size_t tiles = tiles_x * tiles_y, tb = 4, blocks = (tiles + tb - 1) / tb;
    const int avx = !g_wino_lanes && has_avx512f_fma() && out_c % 16 == 0;
#pragma omp parallel OMP_THREADS
    {
        float *v = malloc(16 * in_c * tb * sizeof(float));
        float *prod = malloc(16 * tb * out_c * sizeof(float));
#pragma omp for schedule(dynamic, 4)
        for (size_t blk = 0; blk < blocks; blk++) {
            const size_t tile0 = blk * tb, active = tiles - tile0 < tb ? tiles - tile0 : tb;
            for (size_t lt = 0; lt < active; lt++) {
                const size_t tile = tile0 + lt, y = tile / tiles_x * 2, x = tile % tiles_x * 2;
                for (size_t ic = 0; ic < in_c; ic++) {
                    float d[16], col[16];
                    for (int dy = 0; dy < 4; dy++)
                        for (int dx = 0; dx < 4; dx++) {
                            const long sy = (long)y + dy - 1, sx = (long)x + dx - 1;
                            float smp = 0.0f;
                            if (sy >= 0 && sy < (long)ih && sx >= 0 && sx < (long)iw)
                                smp = input[(ic * ih + (size_t)sy) * iw + (size_t)sx];
                            d[dy * 4 + dx] = relu_input ? rmax(smp, 0.0f) : smp;
                        }
                    for (int j = 0; j < 4; j++) {
                        const float a = d[j], b = d[4 + j], c = d[8 + j], e = d[12 + j];
                        col[j] = a - c;
                        col[4 + j] = b + c;
                        col[8 + j] = c - b;
                        col[12 + j] = b - e;
                    }
                    for (int i = 0; i < 4; i++) {
                        const float a = col[i * 4], b = col[i * 4 + 1], c = col[i * 4 + 2],
                                    e = col[i * 4 + 3];
                        v[((size_t)(i * 4) * in_c + ic) * active + lt] = a - c;
                        v[((size_t)(i * 4 + 1) * in_c + ic) * active + lt] = b + c;
                        v[((size_t)(i * 4 + 2) * in_c + ic) * active + lt] = c - b;
                        v[((size_t)(i * 4 + 3) * in_c + ic) * active + lt] = b - e;
                    }
                }
            }
            if (avx) wino_products_avx512(u, v, prod, in_c, out_c, active);
            else if (g_wino_lanes) wino_products_lanes(u, v, prod, in_c, out_c, active);
            else wino_products_scalar(u, v, prod, in_c, out_c, active);
            for (size_t lt = 0; lt < active; lt++) {
                const size_t tile = tile0 + lt, ty = tile / tiles_x, tx = tile % tiles_x;
                for (size_t oc = 0; oc < out_c; oc++) {
                    float p[8];
#define WM(pos) prod[((size_t)(pos) * active + lt) * out_c + oc]
                    for (int j = 0; j < 4; j++) {
                        p[j] = (WM(j) + WM(4 + j)) + WM(8 + j);
                        p[4 + j] = (WM(4 + j) - WM(8 + j)) - WM(12 + j);
                    }
#undef WM
                    const float b = bias ? bias[oc] : 0.0f;
                    const float vals[4] = {((p[0] + p[1]) + p[2]) + b, ((p[1] - p[2]) - p[3]) + b,
                                           ((p[4] + p[5]) + p[6]) + b, ((p[5] - p[6]) - p[7]) + b};
                    for (int dy = 0; dy < 2; dy++)
                        for (int dx = 0; dx < 2; dx++) {
                            const size_t oy = ty * 2 + dy, ox = tx * 2 + dx;
                            if (oy < oh && ox < ow) out[(oc * oh + oy) * ow + ox] = vals[dy * 2 + dx];
                        }
                }
            }
        }
        free(v);
        free(prod);
    }
}

/* conv::conv_transpose2d (src/conv.rs:1009-1098), its three routes:
 *  - kernel == stride and in_c % 16 == 0 on an AVX-512 host: the prepacked
 *    non-overlap kernel (src/specialized.rs:206-271): sixteen FMA lanes over
 *    the input channels, lanes summed in order from -0.0, then + bias;
 *  - kernel == stride otherwise: per output element the unfused sum over the
 *    input channels, then + bias (src/conv.rs:1040-1070);
 *  - otherwise the serial scatter from zero, skipping zero inputs, then
 *    + bias (src/conv.rs:1072-1097). */
void vko_conv_transpose2d(const float *input, size_t in_c, size_t ih, size_t iw,
                          const float *weight, size_t out_c, size_t kh, size_t kw, size_t stride,
                          const float *bias, float *out) {
    const size_t oh = (ih - 1) * stride + kh, ow = (iw - 1) * stride + kw;
    if (kh == stride && kw == stride && in_c % 16 == 0 && vko_has_avx512()) {
#pragma omp parallel for OMP_THREADS schedule(static)
        for (size_t oc = 0; oc < out_c; oc++) {
            const float b = bias ? bias[oc] : 0.0f;
            for (size_t iy = 0; iy < ih; iy++)
                for (size_t ix = 0; ix < iw; ix++)
                    for (size_t ky = 0; ky < kh; ky++)
                        for (size_t kx = 0; kx < kw; kx++) {
                            float lanes[16] = {0};
                            for (size_t c0 = 0; c0 < in_c; c0 += 16)
                                for (int l = 0; l < 16; l++) {
                                    const size_t ic = c0 + (size_t)l;
                                    lanes[l] = fmaf(input[(ic * ih + iy) * iw + ix],
                                                    weight[((ic * out_c + oc) * kh + ky) * kw + kx],
                                                    lanes[l]);
                                }
                            float sum = RUST_SUM_INIT;
                            for (int l = 0; l < 16; l++) sum = sum + lanes[l];
                            out[(oc * oh + iy * kh + ky) * ow + ix * kw + kx] = sum + b;
                        }
        }
        return;
    }
    if (kh == stride && kw == stride) {
#pragma omp parallel for OMP_THREADS schedule(static)
        for (size_t oc = 0; oc < out_c; oc++) {
            float *plane = out + oc * oh * ow;
            for (size_t iy = 0; iy < ih; iy++)
                for (size_t ix = 0; ix < iw; ix++)
                    for (size_t ky = 0; ky < kh; ky++)
                        for (size_t kx = 0; kx < kw; kx++) {
                            float sum = 0.0f;
                            for (size_t ic = 0; ic < in_c; ic++)
                                sum = sum + input[(ic * ih + iy) * iw + ix] *
                                                weight[((ic * out_c + oc) * kh + ky) * kw + kx];
                            plane[(iy * stride + ky) * ow + ix * stride + kx] = sum;
                        }
            if (bias)
                for (size_t i = 0; i < oh * ow; i++) plane[i] = plane[i] + bias[oc];
        }
        return;
    }
    memset(out, 0, out_c * oh * ow * sizeof(float));
    for (size_t ic = 0; ic < in_c; ic++)
        for (size_t iy = 0; iy < ih; iy++)
            for (size_t ix = 0; ix < iw; ix++) {
                const float iv = input[(ic * ih + iy) * iw + ix];
                if (iv == 0.0f) continue;
                for (size_t oc = 0; oc < out_c; oc++)
                    for (size_t ky = 0; ky < kh; ky++)
                        for (size_t kx = 0; kx < kw; kx++) {
                            float *o = &out[(oc * oh + iy * stride + ky) * ow + ix * stride + kx];
                            *o = *o + iv * weight[((ic * out_c + oc) * kh + ky) * kw + kx];
                        }
            }
    if (bias)
        for (size_t oc = 0; oc < out_c; oc++)
            for (size_t i = 0; i < oh * ow; i++) out[oc * oh * ow + i] = out[oc * oh * ow + i] + bias[oc];
}

/* The crate's gather-form test oracle conv_transpose2d_naive
 * (src/conv.rs:1646-1704): per output, (ic, ky, kx) ascending over the taps
 * that land on it, unfused, then the bias. */
void vko_conv_transpose2d_naive(const float *input, size_t in_c, size_t ih, size_t iw,
                                const float *weight, size_t out_c, size_t kh, size_t kw,
                                size_t stride, const float *bias, float *out) {
    const size_t oh = (ih - 1) * stride + kh, ow = (iw - 1) * stride + kw;
#pragma omp parallel for OMP_THREADS schedule(static)
    for (size_t oc = 0; oc < out_c; oc++)
        for (size_t oy = 0; oy < oh; oy++)
            for (size_t ox = 0; ox < ow; ox++) {
                float acc = 0.0f;
                for (size_t ic = 0; ic < in_c; ic++)
                    for (size_t ky = 0; ky < kh; ky++) {
                        if (oy < ky || (oy - ky) % stride) continue;
                        const size_t iy = (oy - ky) / stride;
                        if (iy >= ih) continue;
                        for (size_t kx = 0; kx < kw; kx++) {
                            if (ox < kx || (ox - kx) % stride) continue;
                            const size_t ix = (ox - kx) / stride;
                            if (ix >= iw) continue;
                            acc = acc + input[(ic * ih + iy) * iw + ix] *
                                            weight[((ic * out_c + oc) * kh + ky) * kw + kx];
                        }
                    }
                if (bias) acc = acc + bias[oc];
                out[(oc * oh + oy) * ow + ox] = acc;
            }
}

typedef struct {
    size_t i0, i1;
    float frac;
} vko_tap;

/* Rust `f as usize` saturates: negative and NaN go to 0. */
static inline size_t sat_usize(float f) { return f > 0.0f ? (size_t)f : 0; }

/* resample::src_coord (src/resample.rs:82-95): half-pixel centres. */
static vko_tap src_coord(size_t dst, float scale, size_t len_in) {
    const float src = ((float)dst + 0.5f) * scale - 0.5f;
    const float sc = rmax(src, 0.0f);
    size_t i0 = sat_usize(floorf(sc));
    const size_t last = len_in ? len_in - 1 : 0;
    if (i0 > last) i0 = last;
    const size_t i1 = i0 + 1 < last ? i0 + 1 : last;
    float frac = i1 == i0 ? 0.0f : sc - (float)i0;
    frac = fminf(fmaxf(frac, 0.0f), 1.0f);
    vko_tap t = {i0, i1, frac};
    return t;
}

/* resample::src_coord_align_corners (src/resample.rs:151-166). */
static vko_tap src_coord_align_corners(size_t dst, size_t len_in, size_t len_out) {
    vko_tap t = {0, 0, 0.0f};
    if (len_in <= 1) return t;
    float src = len_out <= 1 ? 0.0f : (float)dst * (float)(len_in - 1) / (float)(len_out - 1);
    src = fminf(fmaxf(src, 0.0f), (float)(len_in - 1));
    size_t i0 = sat_usize(floorf(src));
    if (i0 > len_in - 1) i0 = len_in - 1;
    const size_t i1 = i0 + 1 < len_in - 1 ? i0 + 1 : len_in - 1;
    float frac = i1 == i0 ? 0.0f : src - (float)i0;
    t.i0 = i0;
    t.i1 = i1;
    t.frac = fminf(fmaxf(frac, 0.0f), 1.0f);
    return t;
}

static void bilinear_tables(const float *input, size_t c, size_t ih, size_t iw, size_t oh,
                            size_t ow, const vko_tap *ty, const vko_tap *tx, float *out) {
#pragma omp parallel for OMP_THREADS schedule(static)
    for (size_t ch = 0; ch < c; ch++) {
        const float *plane = input + ch * ih * iw;
        for (size_t oy = 0; oy < oh; oy++) {
            const float *row0 = plane + ty[oy].i0 * iw, *row1 = plane + ty[oy].i1 * iw;
            const float fy = ty[oy].frac;
            for (size_t ox = 0; ox < ow; ox++) {
                const size_t x0 = tx[ox].i0, x1 = tx[ox].i1;
                const float fx = tx[ox].frac;
                const float top = row0[x0] * (1.0f - fx) + row0[x1] * fx;
                const float bot = row1[x0] * (1.0f - fx) + row1[x1] * fx;
                out[(ch * oh + oy) * ow + ox] = top * (1.0f - fy) + bot * fy;
            }
        }
    }
}

/* resample::bilinear_resize (src/resample.rs:10-77): per-axis tables, then
 * the two-row blend.  Empty input or output: out is left untouched. */
void vko_bilinear_resize(const float *input, size_t c, size_t ih, size_t iw, size_t oh, size_t ow,
                         float *out) {
    if (!ih || !iw || !oh || !ow) return;
    const float sy = (float)ih / (float)oh, sx = (float)iw / (float)ow;
    vko_tap *ty = (vko_tap *)malloc(oh * sizeof(vko_tap)), *tx = (vko_tap *)malloc(ow * sizeof(vko_tap));
    for (size_t y = 0; y < oh; y++) ty[y] = src_coord(y, sy, ih);
    for (size_t x = 0; x < ow; x++) tx[x] = src_coord(x, sx, iw);
    bilinear_tables(input, c, ih, iw, oh, ow, ty, tx, out);
    free(ty);
    free(tx);
}

/* resample::bilinear_resize_naive (src/resample.rs:101-149): coordinates
 * recomputed for every output element. */
void vko_bilinear_resize_naive(const float *input, size_t c, size_t ih, size_t iw, size_t oh,
                               size_t ow, float *out) {
    if (!ih || !iw || !oh || !ow) return;
    const float scale_y = (float)ih / (float)oh, scale_x = (float)iw / (float)ow;
    for (size_t ch = 0; ch < c; ch++)
        for (size_t oy = 0; oy < oh; oy++) {
            const float sy = rmax(((float)oy + 0.5f) * scale_y - 0.5f, 0.0f);
            size_t y0 = sat_usize(floorf(sy));
            if (y0 > ih - 1) y0 = ih - 1;
            const size_t y1 = y0 + 1 < ih - 1 ? y0 + 1 : ih - 1;
            const float fy = y1 == y0 ? 0.0f : fminf(fmaxf(sy - (float)y0, 0.0f), 1.0f);
            for (size_t ox = 0; ox < ow; ox++) {
                const float sx = rmax(((float)ox + 0.5f) * scale_x - 0.5f, 0.0f);
                size_t x0 = sat_usize(floorf(sx));
                if (x0 > iw - 1) x0 = iw - 1;
                const size_t x1 = x0 + 1 < iw - 1 ? x0 + 1 : iw - 1;
                const float fx = x1 == x0 ? 0.0f : fminf(fmaxf(sx - (float)x0, 0.0f), 1.0f);
                const float *p = input + ch * ih * iw;
                const float top = p[y0 * iw + x0] * (1.0f - fx) + p[y0 * iw + x1] * fx;
                const float bot = p[y1 * iw + x0] * (1.0f - fx) + p[y1 * iw + x1] * fx;
                out[(ch * oh + oy) * ow + ox] = top * (1.0f - fy) + bot * fy;
            }
        }
}

/* resample::bilinear_resize_align_corners (src/resample.rs:184-245). */
void vko_bilinear_resize_align_corners(const float *input, size_t c, size_t ih, size_t iw,
                                       size_t oh, size_t ow, float *out) {
    if (!ih || !iw || !oh || !ow) return;
    vko_tap *ty = (vko_tap *)malloc(oh * sizeof(vko_tap)), *tx = (vko_tap *)malloc(ow * sizeof(vko_tap));
    for (size_t y = 0; y < oh; y++) ty[y] = src_coord_align_corners(y, ih, oh);
    for (size_t x = 0; x < ow; x++) tx[x] = src_coord_align_corners(x, iw, ow);
    bilinear_tables(input, c, ih, iw, oh, ow, ty, tx, out);
    free(ty);
    free(tx);
}
