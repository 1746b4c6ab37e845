// Q8_0 quantisation and block-dot GEMM for gfx950, bit-exact with the
// reference's scalar oracle.
//
// Storage: a [rows, k] Q8_0 matrix is held block-major, qs [k/32][rows][32]
// int8 and d [k/32][rows] binary16 bits: the 34-byte BlockQ8_0 AoS of
// src/lib.rs:33-38 split into two dense arrays, with the blocks of one
// 32-wide k-slice of all rows adjacent, so that a 16-row MFMA fragment of one
// block is 512 contiguous bytes and a k-slice of scales is contiguous.
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

// quantize_row_q8_0 (src/q8_0_dot.rs:27-46): eight lanes per 32-value block,
// four values each; amax is a max (order-free) over the eight lanes.  Block b
// of the row-major input (row b / nbr, k-slice b % nbr) is stored block-major.
__global__ __launch_bounds__(256) void quantize_q8_0_kernel(const float *__restrict__ x,
                                                            int8_t *__restrict__ qs,
                                                            uint16_t *__restrict__ dbits,
                                                            size_t nblocks, size_t rows,
                                                            size_t nbr) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t b = t >> 3;
    const int part = (int)(t & 7);
    const bool live = b < nblocks;
    const size_t bb = live ? b : nblocks - 1;  // idle lanes shadow the last block
    const size_t dst = (bb % nbr) * rows + bb / nbr;  // block-major index
    const f32x4 v = reinterpret_cast<const f32x4 *>(x + bb * 32)[part];
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
    const float d = div_rn(amax, 127.0f);
    const float inv = d != 0.0f ? div_rn(1.0f, d) : 0.0f;
    if (!live) return;
    if (part == 0) dbits[dst] = __builtin_bit_cast(uint16_t, (_Float16)d);
    uint32_t w = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        float q = roundf(mul_rn(v[e], inv));  // f32::round: half away from zero
        int qi;
        if (isnan(q)) {
            qi = 0;  // `NaN as i8` saturates to 0
        } else {
            q = fminf(fmaxf(q, -127.0f), 127.0f);
            qi = (int)q;
        }
        w |= ((uint32_t)(qi & 0xff)) << (8 * e);
    }
    reinterpret_cast<uint32_t *>(qs + dst * 32)[part] = w;
}

// 256 threads = 4 waves in a 2x2 arrangement over a 64x64 output tile; each
// wave owns 32x32 = 2x2 MFMA fragments.  The scales of a chunk of up to
// QCH blocks are staged in LDS as floats, [block][row] and [block][col], so
// a lane's four output rows (4*lh..4*lh+3 of a fragment) are one 16-byte
// read.  The int8 operands stream from global memory (clamped rows, no
// select) with a register prefetch PF blocks ahead.
constexpr int QCH = 32;  // blocks per scale chunk (a multiple of QPF)
constexpr int QPF = 4;   // prefetch distance in blocks

// Epilogue of a Q8_0 projection, applied to the exact block-order sum with
// separately rounded ops (the f32 ops the engine applies after
// Kernels::gemm_q8_0): Store c = (acc + bias) * gamma; Gelu c = gelu(acc +
// bias) (AVX-512 form below tail_start, scalar form after); Residual
// c = c + (acc + bias) * gamma.  bias / gamma may be null.
struct Q8Epi {
    const float *bias, *gamma;
    size_t tail_start;
};

template <Epi EPI>
__global__ __launch_bounds__(256) void gemm_q8_0_kernel(const int8_t *__restrict__ a_qs,
                                                        const uint16_t *__restrict__ a_d,
                                                        const int8_t *__restrict__ b_qs,
                                                        const uint16_t *__restrict__ b_d,
                                                        float *__restrict__ c, int M, int N,
                                                        int K, Q8Epi ep) {
    __shared__ __attribute__((aligned(16))) float sa[QCH][64];
    __shared__ __attribute__((aligned(16))) float sb[QCH][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lh = lane >> 4;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    const int mw = m0 + wm * 32;
    const int nw = n0 + wn * 32;
    const int nb = K / 32;

    // Operand rows of this lane (clamped: rows past M / N compute values
    // that are never stored); block b of row r sits at (b * rows + r) * 32.
    const int8_t *arow[2], *brow[2];
#pragma unroll
    for (int i = 0; i < 2; i++) arow[i] = a_qs + (size_t)min(mw + i * 16 + li, M - 1) * 32 + 8 * lh;
#pragma unroll
    for (int j = 0; j < 2; j++) brow[j] = b_qs + (size_t)min(nw + j * 16 + li, N - 1) * 32 + 8 * lh;

    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    long pa[QPF][2], pb[QPF][2];
    auto fetch = [&](int b, int slot) {
        const int bc = min(b, nb - 1);
#pragma unroll
        for (int i = 0; i < 2; i++)
            pa[slot][i] = *reinterpret_cast<const long *>(arow[i] + (size_t)bc * M * 32);
#pragma unroll
        for (int j = 0; j < 2; j++)
            pb[slot][j] = *reinterpret_cast<const long *>(brow[j] + (size_t)bc * N * 32);
    };
    if (nb > 0) {  // K == 0 stores zeros
#pragma unroll
        for (int p = 0; p < QPF; p++) fetch(p, p);
    }

    for (int c0 = 0; c0 < nb; c0 += QCH) {
        const int cn = min(QCH, nb - c0);
        __syncthreads();  // previous chunk's scales are no longer read
        for (int e = tid; e < 64 * cn; e += 256) {
            const int blk = e / 64, rr = e % 64;
            sa[blk][rr] = half_bits_to_float(a_d[(size_t)(c0 + blk) * M + min(m0 + rr, M - 1)]);
            sb[blk][rr] = half_bits_to_float(b_d[(size_t)(c0 + blk) * N + min(n0 + rr, N - 1)]);
        }
        __syncthreads();
        // Groups of QPF blocks with the prefetch slot fixed at compile time
        // (QCH is a multiple of QPF, so block c0 + bl + u sits in slot u).
        for (int bl = 0; bl < cn; bl += QPF) {
#pragma unroll
            for (int u = 0; u < QPF; u++) {
                if (bl + u >= cn) break;
                const int b = c0 + bl + u;
                const long av[2] = {pa[u][0], pa[u][1]}, bv[2] = {pb[u][0], pb[u][1]};
                fetch(b + QPF, u);
                f32x4 da[2];
#pragma unroll
                for (int i = 0; i < 2; i++)
                    da[i] = *reinterpret_cast<const f32x4 *>(&sa[bl + u][wm * 32 + i * 16 + 4 * lh]);
                float db[2];
#pragma unroll
                for (int j = 0; j < 2; j++) db[j] = sb[bl + u][wn * 32 + j * 16 + li];
                i32x4 is[2][2];
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++) is[i][j] = mfma16x16x32_i8(av[i], bv[j], i32x4{0, 0, 0, 0});
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
#pragma unroll
                        for (int r = 0; r < 4; r++)
                            acc[i][j][r] = add_rn(acc[i][j][r],
                                                  mul_rn(mul_rn(da[i][r], db[j]), (float)is[i][j][r]));
            }
        }
    }
    // Epilogue reads (bias, gamma, residual) from clamped indices before any
    // store, so that they overlap.
    float bias[2], gamma[2], resid[2][2][4];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int col = min(nw + j * 16 + li, N - 1);
        bias[j] = ep.bias ? ep.bias[col] : 0.0f;
        gamma[j] = ep.gamma ? ep.gamma[col] : 1.0f;
    }
    if constexpr (EPI == Epi::Residual) {
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    resid[i][j][r] = c[(size_t)min(mw + i * 16 + 4 * lh + r, M - 1) * N +
                                       min(nw + j * 16 + li, N - 1)];
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
                if (row >= M) continue;
                const size_t idx = (size_t)row * N + col;
                float v = acc[i][j][r];
                if (ep.bias) v = add_rn(v, bias[j]);
                if constexpr (EPI == Epi::Gelu) {
                    c[idx] = idx < ep.tail_start ? gelu_avx512_form(v) : gelu_scalar_form(v);
                } else {
                    if (ep.gamma) v = mul_rn(v, gamma[j]);
                    c[idx] = EPI == Epi::Residual ? add_rn(resid[i][j][r], v) : v;
                }
            }
        }
}

}  // namespace

hipError_t launch_quantize_q8_0(hipStream_t s, const float *x, int8_t *qs, uint16_t *d,
                                size_t rows, size_t k) {
    size_t nblocks = rows * (k / 32);
    if (nblocks == 0) return hipSuccess;
    quantize_q8_0_kernel<<<(unsigned)((nblocks * 8 + 255) / 256), 256, 0, s>>>(x, qs, d, nblocks, rows,
                                                                             k / 32);
    return hipGetLastError();
}

hipError_t launch_gemm_q8_0(hipStream_t s, const int8_t *a_qs, const uint16_t *a_d,
                            const int8_t *b_qs, const uint16_t *b_d, float *c, size_t m,
                            size_t n, size_t k, Epi epi, const float *bias, const float *gamma) {
    if (m == 0 || n == 0) return hipSuccess;
    dim3 grid((unsigned)((n + 63) / 64), (unsigned)((m + 63) / 64));
    const Q8Epi ep{bias, gamma, m * n - (m * n) % 16};
    const int M = (int)m, N = (int)n, K = (int)k;
    switch (epi) {
        case Epi::Store: gemm_q8_0_kernel<Epi::Store><<<grid, 256, 0, s>>>(a_qs, a_d, b_qs, b_d, c, M, N, K, ep); break;
        case Epi::Gelu: gemm_q8_0_kernel<Epi::Gelu><<<grid, 256, 0, s>>>(a_qs, a_d, b_qs, b_d, c, M, N, K, ep); break;
        case Epi::Residual: gemm_q8_0_kernel<Epi::Residual><<<grid, 256, 0, s>>>(a_qs, a_d, b_qs, b_d, c, M, N, K, ep); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace vh
