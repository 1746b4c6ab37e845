// Q8_0 quantisation and block-dot GEMM for gfx950, bit-exact with the
// reference's scalar oracle.
//
// Storage: a [rows, k] Q8_0 matrix is held as qs [rows][k] int8 and
// d [rows][k/32] binary16 bits (the 34-byte BlockQ8_0 AoS of src/lib.rs:33-38
// split into two dense arrays so MFMA operands load as aligned 8-byte words).
//
// GEMM: per 32-wide block b, one v_mfma_i32_16x16x32_i8 produces the exact
// int32 sums isum_b of a 16x16 tile (|isum| <= 32*127*127 < 2^24, so the
// float conversion is exact).  Each lane then folds its four outputs in block
// order exactly as src/scalar.rs:51 does: acc = acc + (d_a * d_b) * isum,
// three separately rounded ops.
#include "common.h"
#include "kernels.h"

namespace vh {
namespace {

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// quantize_row_q8_0 (src/q8_0_dot.rs:27-46): one thread per 32-value block.
__global__ void quantize_q8_0_kernel(const float *__restrict__ x, int8_t *__restrict__ qs,
                                     uint16_t *__restrict__ dbits, size_t nblocks) {
    size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const f32x4 *src = reinterpret_cast<const f32x4 *>(x + b * 32);
    f32x4 v[8];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        v[i] = src[i];
#pragma unroll
        for (int e = 0; e < 4; e++) amax = fmaxf(amax, fabsf(v[i][e]));
    }
    const float d = div_rn(amax, 127.0f);
    const float inv = d != 0.0f ? div_rn(1.0f, d) : 0.0f;
    dbits[b] = __builtin_bit_cast(uint16_t, (_Float16)d);
    uint32_t packed[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float q = roundf(mul_rn(v[i][e], inv));  // f32::round: half away from zero
            int qi;
            if (isnan(q)) {
                qi = 0;  // `NaN as i8` saturates to 0
            } else {
                q = fminf(fmaxf(q, -127.0f), 127.0f);
                qi = (int)q;
            }
            w |= ((uint32_t)(qi & 0xff)) << (8 * e);
        }
        packed[i] = w;
    }
    uint4 *dst = reinterpret_cast<uint4 *>(qs + b * 32);
    dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
}

// 256 threads = 4 waves in a 2x2 arrangement over a 64x64 output tile; each
// wave owns 32x32 = 2x2 MFMA fragments.
__global__ __launch_bounds__(256) void gemm_q8_0_kernel(const int8_t *__restrict__ a_qs,
                                                        const uint16_t *__restrict__ a_d,
                                                        const int8_t *__restrict__ b_qs,
                                                        const uint16_t *__restrict__ b_d,
                                                        float *__restrict__ c, int M, int N,
                                                        int K) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lh = lane >> 4;
    const int wm = wave >> 1, wn = wave & 1;
    const int mw = blockIdx.y * 64 + wm * 32;
    const int nw = blockIdx.x * 64 + wn * 32;
    const int nb = K / 32;

    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    for (int b = 0; b < nb; b++) {
        long av[2], bv[2];
        float da[2][4], db[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int row = mw + i * 16 + li;
            av[i] = row < M ? *reinterpret_cast<const long *>(a_qs + (size_t)row * K + b * 32 + 8 * lh) : 0;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int orow = mw + i * 16 + 4 * lh + r;
                da[i][r] = orow < M ? half_bits_to_float(a_d[(size_t)orow * nb + b]) : 0.0f;
            }
        }
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = nw + j * 16 + li;
            bv[j] = col < N ? *reinterpret_cast<const long *>(b_qs + (size_t)col * K + b * 32 + 8 * lh) : 0;
            db[j] = col < N ? half_bits_to_float(b_d[(size_t)col * nb + b]) : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                i32x4 is = mfma16x16x32_i8(av[i], bv[j], i32x4{0, 0, 0, 0});
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc[i][j][r] = add_rn(acc[i][j][r], mul_rn(mul_rn(da[i][r], db[j]), (float)is[r]));
            }
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = nw + j * 16 + li;
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = mw + i * 16 + 4 * lh + r;
                if (row < M) c[(size_t)row * N + col] = acc[i][j][r];
            }
        }
}

}  // namespace

hipError_t launch_quantize_q8_0(hipStream_t s, const float *x, int8_t *qs, uint16_t *d,
                                size_t rows, size_t k) {
    size_t nblocks = rows * (k / 32);
    if (nblocks == 0) return hipSuccess;
    quantize_q8_0_kernel<<<(unsigned)((nblocks + 255) / 256), 256, 0, s>>>(x, qs, d, nblocks);
    return hipGetLastError();
}

hipError_t launch_gemm_q8_0(hipStream_t s, const int8_t *a_qs, const uint16_t *a_d,
                            const int8_t *b_qs, const uint16_t *b_d, float *c, size_t m,
                            size_t n, size_t k) {
    if (m == 0 || n == 0) return hipSuccess;
    dim3 grid((unsigned)((n + 63) / 64), (unsigned)((m + 63) / 64));
    gemm_q8_0_kernel<<<grid, 256, 0, s>>>(a_qs, a_d, b_qs, b_d, c, (int)m, (int)n, (int)k);
    return hipGetLastError();
}

}  // namespace vh
