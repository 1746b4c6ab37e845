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
// int32 sums isum_b of a 16x16 tile (|isum| <= 32*128*128 < 2^24, so the
// float conversion is exact).  Each lane then folds its four outputs in block
// order exactly as src/scalar.rs:51 does: acc = acc + (d_a * d_b) * isum,
// three separately rounded ops.  (Holding the int8 values as halves for the
// f16 MFMA would drop the conversion, but doubles the operand bytes and
// measured slower: the operands no longer stay in L2.)
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "common.h"
#include "kernels.h"

namespace vh {
namespace {

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// quantize_row_q8_0 (src/q8_0_dot.rs:27-46) of a tile of R consecutive rows
// per workgroup (8, or 4 when there are few rows), up to 768 columns (24
// blocks) at a time:
//  - loads: float4 u of the tile is row u / (cw/4), column 4 (u % (cw/4)),
//    so each load instruction of the workgroup reads 4 KB of consecutive row
//    memory (the rows are adjacent in memory when cw == k) and a block's
//    eight float4 sit in eight adjacent lanes;
//  - arithmetic: amax over the block's lanes (three DPP steps: lane ^ 1,
//    lane ^ 2, then the mirror pairing the two quads), d = amax / 127 and
//    1 / d correctly rounded, d stored as binary16 (RNE), each value
//    roundf(x * (1/d)) clamped to +-127 (NaN -> 0);
//  - stores: through LDS, so that block j of the R rows, block-major slots
//    j * rows + r0 .. r0 + R - 1, is written as one run of 32 R bytes.
// NT: non-temporal loads.  k % 32 == 0; x 16-byte aligned (device tensors
// and workspaces always are).
template <bool NT, int R>
__global__ __launch_bounds__(256) void quantize_tile_q8_0_kernel(const float *__restrict__ x,
                                                                 int8_t *__restrict__ qs,
                                                                 uint16_t *__restrict__ dbits,
                                                                 int rows, int nbr) {
    constexpr int CB = 24;  // blocks per column chunk
    static_assert(R * CB * 8 % 256 == 0, "whole float4 per thread");
    __shared__ __attribute__((aligned(16))) uint32_t sq[CB][R][8];
    __shared__ __attribute__((aligned(16))) uint16_t sd[CB][R];
    const int tid = threadIdx.x, lane = tid & 63;
    const int r0 = blockIdx.x * R;
    const int nr = min(R, rows - r0);
    for (int j0 = 0; j0 < nbr; j0 += CB) {
        const int cb = min(CB, nbr - j0);  // blocks in this chunk
        const int c4 = cb * 8;             // float4 per row in this chunk
        constexpr int U = R * CB * 8 / 256;  // float4 per thread
        f32x4 v[U];
#pragma unroll
        for (int i = 0; i < U; i++) {
            const int u = i * 256 + tid;
            const int r = min(u / c4, nr - 1), c = u % c4;  // past the tile: a clamped row
            const f32x4 *src = reinterpret_cast<const f32x4 *>(x + (size_t)(r0 + r) * nbr * 32 +
                                                               (size_t)j0 * 32) + c;
            if constexpr (NT) v[i] = __builtin_nontemporal_load(src);
            else v[i] = *src;
        }
#pragma unroll
        for (int i = 0; i < U; i++) {
            const int u = i * 256 + tid;
            float amax = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; e++) amax = q8_absmax(amax, v[i][e]);
            amax = q8_absmax(amax, dpp_f32<0xb1>(amax));
            amax = q8_absmax(amax, dpp_f32<0x4e>(amax));
            amax = q8_absmax(amax, dpp_f32<0x141>(amax));
            float d, inv;
            q8_scale(amax, d, inv);
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
            const int r = u / c4, c = u % c4, jb = c >> 3;
            if (r < nr) {
                sq[jb][r][c & 7] = w;
                if ((lane & 7) == 0) sd[jb][r] = __builtin_bit_cast(uint16_t, (_Float16)d);
            }
        }
        __syncthreads();
        // Block column jb: R slots x 32 bytes = 2R chunks of 16 bytes.
        for (int u = tid; u < cb * 2 * R; u += 256) {
            const int jb = u / (2 * R), r = (u % (2 * R)) >> 1, half = u & 1;
            if (r < nr) {
                const size_t slot = (size_t)(j0 + jb) * rows + r0 + r;
                reinterpret_cast<uint4 *>(qs + slot * 32)[half] =
                    reinterpret_cast<const uint4 *>(&sq[jb][r][0])[half];
            }
        }
        if (R == 8 && nr == R && (rows & 7) == 0 && (reinterpret_cast<uintptr_t>(dbits) & 15) == 0) {
            // The 8 scales of a block column are 16 contiguous, aligned
            // bytes: one store each instead of eight 2-byte stores (measured
            // at 131072 x 768: 95 -> 84 us, the 2-byte stores alone had cost
            // 11 us).
            for (int jb = tid; jb < cb; jb += 256)
                *reinterpret_cast<uint4 *>(dbits + (size_t)(j0 + jb) * rows + r0) =
                    *reinterpret_cast<const uint4 *>(&sd[jb][0]);
        } else {
            for (int u = tid; u < cb * R; u += 256) {
                const int jb = u / R, r = u % R;
                if (r < nr) dbits[(size_t)(j0 + jb) * rows + r0 + r] = sd[jb][r];
            }
        }
        __syncthreads();
    }
}

// LayerNorm of a row (the arithmetic of layernorm_kernel: ln_row_stats and
// ln_apply) straight into Q8_0 blocks, bit-identical to LayerNorm followed by
// quantize_q8_0_kernel.  One wave per row, float4 slot j of lane l holding
// columns 4(l + 64j) .. +3, so a 32-column block is eight adjacent lanes and
// its max takes three DPP steps (lane ^ 1, lane ^ 2, then the mirror that
// pairs the two quads of eight lanes).  cols % 32 == 0, cols <= 1024.
__global__ __launch_bounds__(256) void layernorm_q8_0_kernel(const float *__restrict__ in,
                                                             const float *__restrict__ gamma,
                                                             const float *__restrict__ beta,
                                                             int8_t *__restrict__ qs,
                                                             uint16_t *__restrict__ dbits,
                                                             int rows, int cols, float eps) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const f32x4 *x = reinterpret_cast<const f32x4 *>(in + (size_t)row * cols);
    const int n4 = cols >> 2;
    // The row, gamma and beta (clamped indices) are all read before the
    // statistics, so the loads are in flight together.
    f32x4 r[4], g[4], b[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int idx = lane + j * 64, gi = min(idx, n4 - 1);
        r[j] = idx < n4 ? x[idx] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        g[j] = reinterpret_cast<const f32x4 *>(gamma)[gi];
        b[j] = reinterpret_cast<const f32x4 *>(beta)[gi];
    }
    float mean, inv;
    ln_row_stats(r, lane, n4, cols, eps, mean, inv);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int idx = lane + j * 64;
        const bool live = idx < n4;  // whole 8-lane groups, as n4 % 8 == 0
        const f32x4 y = ln_apply(r[j], mean, inv, g[j], b[j]);
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) amax = q8_absmax(amax, y[e]);
        amax = q8_absmax(amax, dpp_f32<0xb1>(amax));
        amax = q8_absmax(amax, dpp_f32<0x4e>(amax));
        amax = q8_absmax(amax, dpp_f32<0x141>(amax));
        float d, qinv;
        q8_scale(amax, d, qinv);
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float q = roundf(mul_rn(y[e], qinv));  // f32::round: half away from zero
            int qi;
            if (isnan(q)) {
                qi = 0;  // `NaN as i8` saturates to 0
            } else {
                q = fminf(fmaxf(q, -127.0f), 127.0f);
                qi = (int)q;
            }
            w |= ((uint32_t)(qi & 0xff)) << (8 * e);
        }
        if (live) {
            const size_t slot = (size_t)(idx >> 3) * rows + row;
            reinterpret_cast<uint32_t *>(qs + slot * 32)[idx & 7] = w;
            if ((idx & 7) == 0) dbits[slot] = __builtin_bit_cast(uint16_t, (_Float16)d);
        }
    }
}

// 256 threads = 4 waves in a 2x2 arrangement; each wave owns FM x FN MFMA
// fragments of 16x16, so a workgroup covers (32*FM) x (32*FN) outputs (FM,
// FN in {1, 2}: the small tiles give the narrow projections enough
// workgroups, since the block-order fold cannot be split along K).  The
// scales of a chunk of up to QCH blocks are staged in LDS as floats,
// [block][row] and [block][col], so a lane's four output rows (4*lh..4*lh+3
// of a fragment) are one 16-byte read.  The operands stream from global
// memory (clamped rows, no select) with a register prefetch QPF blocks
// ahead, and the MFMAs of block b+1 are issued before the fold of block b,
// so the matrix core works while the VALU folds.


// Epilogue of a Q8_0 projection, applied to the exact block-order sum with
// separately rounded ops (the f32 ops the engine applies after
// Kernels::gemm_q8_0): Store c = (acc + bias) * gamma; Gelu c = gelu(acc +
// bias) (AVX-512 form below tail_start, scalar form after); Residual
// c = c + (acc + bias) * gamma.  bias / gamma may be null.
struct Q8Epi {
    const float *bias, *gamma;
    size_t tail_start;
    // Qkv: c is unused; columns [0, 3*heads*64) go to q / k / v head-major
    // [img][head][token][64] with the bias added, and when rot is non-null the
    // 2-D RoPE (rot [tokens][2][16][sin, cos]) rotates the q and k columns.
    float *q, *k, *v;
    const float *rot;
    int tokens, heads;
    // Gelu with FN == 2 and N % 32 == 0: when q8_qs is set, the GELU output
    // is written as block-major Q8_0 rows (quantize_row_q8_0 of the f32
    // values) instead of f32; c is unused.
    int8_t *q8_qs;
    uint16_t *q8_d;
};

template <Epi EPI, int FM, int FN, int QPF>
__global__ __launch_bounds__(256) void gemm_q8_0_kernel(const int8_t *__restrict__ a_qs,
                                                        const uint16_t *__restrict__ a_d,
                                                        const int8_t *__restrict__ b_qs,
                                                        const uint16_t *__restrict__ b_d,
                                                        float *__restrict__ c, int M, int N,
                                                        int K, Q8Epi ep) {
    static_assert(EPI != Epi::Qkv || FN == 2, "the QKV epilogue pairs fragments j = 0, 1");
    constexpr int TR = 32 * FM, TC = 32 * FN;  // workgroup tile
    // QCH: blocks per scale chunk.  The 32x32 tile (the narrow projections,
    // K up to 3072) stages 96 blocks, so those are one chunk; the larger
    // tiles stage 32 (K = 768 is one chunk), which keeps the staging
    // registers at 16 per thread.  Later chunks wait for their scales with
    // the operand prefetch drained, once per chunk.
    // QPF: prefetch distance in blocks (q8_qpf), a divisor of the block
    // count and of QCH.
    constexpr int QCH = FM * FN == 1 ? 96 : 32;
    static_assert(QCH % QPF == 0, "scale chunks hold whole prefetch groups");
    __shared__ __attribute__((aligned(16))) float sa[QCH][TR];
    __shared__ __attribute__((aligned(16))) float sb[QCH][TC];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lh = lane >> 4;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * TR, n0 = blockIdx.x * TC;
    const int mw = m0 + wm * 16 * FM;
    const int nw = n0 + wn * 16 * FN;
    const int nb = K / 32;

    // Operand rows of this lane (clamped: rows past M / N compute values
    // that are never stored); block b of row r sits at byte (b * rows + r) *
    // 32.  Buffer loads take the per-lane row offset in a VGPR and the
    // block's offset b * rows * 32 in an SGPR, so a block costs no vector
    // address arithmetic.  The host keeps rows * K below 2^31.
    const __amdgpu_buffer_rsrc_t rsa =
        __builtin_amdgcn_make_buffer_rsrc((void *)a_qs, (short)0, M * K, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsb =
        __builtin_amdgcn_make_buffer_rsrc((void *)b_qs, (short)0, N * K, 0x00020000);
    int aoff[FM], boff[FN];
#pragma unroll
    for (int i = 0; i < FM; i++) aoff[i] = min(mw + i * 16 + li, M - 1) * 32 + 8 * lh;
#pragma unroll
    for (int j = 0; j < FN; j++) boff[j] = min(nw + j * 16 + li, N - 1) * 32 + 8 * lh;

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    long pa[QPF][FM], pb[QPF][FN];
    auto fetch = [&](int b, int slot) {
        const int bc = min(b, nb - 1);
#pragma unroll
        for (int i = 0; i < FM; i++)
            pa[slot][i] = __builtin_bit_cast(
                long, __builtin_amdgcn_raw_buffer_load_b64(rsa, aoff[i], bc * M * 32, 0));
#pragma unroll
        for (int j = 0; j < FN; j++)
            pb[slot][j] = __builtin_bit_cast(
                long, __builtin_amdgcn_raw_buffer_load_b64(rsb, boff[j], bc * N * 32, 0));
    };
    // Exact int32 block sums of the block held in prefetch slot `slot`.
    auto block_sums = [&](int slot, i32x4 (&is)[FM][FN]) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++)
                is[i][j] = mfma16x16x32_i8(pa[slot][i], pb[slot][j], i32x4{0, 0, 0, 0});
    };
    // Scales of one chunk (up to QCH blocks), NA + NB per thread from
    // clamped indices, all loads issued before any is waited on; stored to
    // LDS as floats at the chunk's start.  Chunk 0's loads go out before
    // the operand prefetch, so that the first wait for them leaves the
    // prefetch in flight.
    // Thread tid stages element e = tid + 256 t of the chunk: block e / TR
    // (clamped to the last block), row m0 + e % TR (clamped).  As TR divides
    // 64, e % TR is lane % TR, a loop-invariant lane offset.  With 64-row
    // (64-column) tiles the block e / TR = wave + 4 t is uniform per wave: a
    // buffer load then takes it as an SGPR offset, with no vector address
    // arithmetic; 32-row tiles form the offset in 32-bit lane arithmetic.
    // Blocks past the chunk fill LDS rows that are never read.
    constexpr int NA = TR * QCH / 256, NB = TC * QCH / 256;
    static_assert(64 % TR == 0 && 64 % TC == 0, "staging layout");
    const __amdgpu_buffer_rsrc_t rsda =
        __builtin_amdgcn_make_buffer_rsrc((void *)a_d, (short)0, nb * M * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsdb =
        __builtin_amdgcn_make_buffer_rsrc((void *)b_d, (short)0, nb * N * 2, 0x00020000);
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int rowa = min(m0 + lane % TR, M - 1), colb = min(n0 + lane % TC, N - 1);
    uint16_t ra[NA], rb[NB];
    auto load_scales = [&](int c) {
#pragma unroll
        for (int t = 0; t < NA; t++) {
            if constexpr (TR == 64) {
                const int blk = min(c + wv + 4 * t, nb - 1);
                ra[t] = __builtin_amdgcn_raw_buffer_load_b16(rsda, rowa * 2, blk * M * 2, 0);
            } else {
                const int blk = min(c + (tid + 256 * t) / TR, nb - 1);
                ra[t] = __builtin_amdgcn_raw_buffer_load_b16(rsda, (blk * M + rowa) * 2, 0, 0);
            }
        }
#pragma unroll
        for (int t = 0; t < NB; t++) {
            if constexpr (TC == 64) {
                const int blk = min(c + wv + 4 * t, nb - 1);
                rb[t] = __builtin_amdgcn_raw_buffer_load_b16(rsdb, colb * 2, blk * N * 2, 0);
            } else {
                const int blk = min(c + (tid + 256 * t) / TC, nb - 1);
                rb[t] = __builtin_amdgcn_raw_buffer_load_b16(rsdb, (blk * N + colb) * 2, 0, 0);
            }
        }
    };
    auto store_scales = [&]() {
#pragma unroll
        for (int t = 0; t < NA; t++) (&sa[0][0])[tid + 256 * t] = half_bits_to_float(ra[t]);
#pragma unroll
        for (int t = 0; t < NB; t++) (&sb[0][0])[tid + 256 * t] = half_bits_to_float(rb[t]);
    };
    i32x4 cur[FM][FN];
    if (nb > 0) {  // K == 0 stores zeros
        load_scales(0);
        // Slot by slot, in the loop's order, so that the loop's first waits
        // need only their own slot's loads.
#pragma unroll
        for (int p = 0; p < QPF; p++) {
            fetch(p, p);
            __builtin_amdgcn_sched_barrier(0x0006);
        }
        block_sums(0, cur);
        fetch(QPF, 0);
        __builtin_amdgcn_sched_barrier(0x0006);
        // Chunk 0's scales, outside the chunk loop so that their wait
        // leaves the operand prefetch in flight.
        store_scales();
    }

    for (int c0 = 0; c0 < nb; c0 += QCH) {
        const int cn = min(QCH, nb - c0);  // a multiple of QPF (host check)
        if (c0 > 0) {
            __syncthreads();  // the previous chunk's scales are no longer read
            load_scales(c0);
            store_scales();
        }
        __syncthreads();
        // Groups of QPF blocks with the prefetch slots fixed at compile time
        // (QPF divides the chunk, so block c0 + bl + u sits in slot u).  A
        // group has no early exit and issues its loads in the same order
        // as the prologue, so the wait before each block's MFMAs covers only
        // that block's operands, QPF blocks after their loads went out.
        // The scales of block bl + u are read from LDS one block ahead of
        // its fold (past the chunk's last block, a clamped re-read).
        auto read_scales = [&](int blk, f32x4 (&da)[FM], float (&db)[FN]) {
#pragma unroll
            for (int i = 0; i < FM; i++)
                da[i] = *reinterpret_cast<const f32x4 *>(&sa[blk][wm * 16 * FM + i * 16 + 4 * lh]);
#pragma unroll
            for (int j = 0; j < FN; j++) db[j] = sb[blk][wn * 16 * FN + j * 16 + li];
        };
        f32x4 da[FM];
        float db[FN];
        read_scales(0, da, db);
        for (int bl = 0; bl < cn; bl += QPF) {
#pragma unroll
            for (int u = 0; u < QPF; u++) {
                const int b = c0 + bl + u;
                // Block b+1 (slot (u+1) % QPF) goes to the matrix core first;
                // past the last block it recomputes a clamped block, unused.
                i32x4 nxt[FM][FN];
                block_sums((u + 1) % QPF, nxt);
                fetch(b + 1 + QPF, (u + 1) % QPF);
                // Keep each block's MFMAs and the loads that refill its slot
                // in this order (only VALU and SALU work may move across):
                // hoisting the next block's MFMAs above these loads makes
                // the loop wait for every load in flight.
                __builtin_amdgcn_sched_barrier(0x0006);
                f32x4 da_n[FM];
                float db_n[FN];
                read_scales(min(bl + u + 1, cn - 1), da_n, db_n);
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++)
#pragma unroll
                        for (int r = 0; r < 4; r++)
                            acc[i][j][r] = add_rn(acc[i][j][r],
                                                  mul_rn(mul_rn(da[i][r], db[j]), (float)cur[i][j][r]));
#pragma unroll
                for (int i = 0; i < FM; i++) {
                    da[i] = da_n[i];
#pragma unroll
                    for (int j = 0; j < FN; j++) cur[i][j] = nxt[i][j];
                }
#pragma unroll
                for (int j = 0; j < FN; j++) db[j] = db_n[j];
            }
        }
    }
    // Epilogue reads (bias, gamma, residual) from clamped indices before any
    // store, so that they overlap.
    float bias[FN], gamma[FN], resid[FM][FN][4];
#pragma unroll
    for (int j = 0; j < FN; j++) {
        const int col = min(nw + j * 16 + li, N - 1);
        bias[j] = ep.bias ? ep.bias[col] : 0.0f;
        gamma[j] = ep.gamma ? ep.gamma[col] : 1.0f;
    }
    // A whole tile (and, for GELU, wholly below tail_start) addresses its
    // elements as a wave-uniform row pointer plus one 32-bit lane offset,
    // with no bounds checks: no vector address arithmetic per element.
    const int mwu = m0 + (wv >> 1) * 16 * FM, nwu = n0 + (wv & 1) * 16 * FN;  // mw, nw
    const bool whole = m0 + TR <= M && n0 + TC <= N &&
                       (EPI != Epi::Gelu || (size_t)(m0 + TR - 1) * N + n0 + TC <= ep.tail_start);
    const unsigned loff = (unsigned)(4 * lh * N + li);
    auto row_ptr = [&](int i, int j, int r) { return c + (size_t)(mwu + i * 16 + r) * N + nwu + j * 16; };
    if constexpr (EPI == Epi::Residual) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    resid[i][j][r] = whole ? row_ptr(i, j, r)[loff]
                                           : c[(size_t)min(mw + i * 16 + 4 * lh + r, M - 1) * N +
                                               min(nw + j * 16 + li, N - 1)];
    }
    // One wait for every load in flight (these reads and the loop's last,
    // unused prefetch) before the stores.  Without it the optional bias and
    // gamma loads leave a possibly pending load at every join of the guarded
    // stores below, and as vmcnt counts stores too, each store then waited
    // for the one before it (about 2.4 us for a tile's 16 stores).
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    if constexpr (EPI == Epi::Gelu && FN == 2) {
        if (ep.q8_qs) {
            // A row's 32-column block nw .. nw + 31 is fragments j = 0, 1 of
            // the 16 lanes sharing lh: its max takes four DPP steps within
            // the 16-lane row.  Rows past M compute and are not stored.
            const size_t kslice = (size_t)(nw >> 5);
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = mw + i * 16 + 4 * lh + r;
                    float g[2];
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        const size_t idx = (size_t)row * N + nw + j * 16 + li;
                        float v = acc[i][j][r];
                        if (ep.bias) v = add_rn(v, bias[j]);
                        g[j] = idx < ep.tail_start ? gelu_avx512_form(v) : gelu_scalar_form(v);
                    }
                    float amax = q8_absmax(q8_absmax(0.0f, g[0]), g[1]);
                    amax = q8_absmax(amax, dpp_f32<0xb1>(amax));
                    amax = q8_absmax(amax, dpp_f32<0x4e>(amax));
                    amax = q8_absmax(amax, dpp_f32<0x141>(amax));
                    amax = q8_absmax(amax, dpp_f32<0x140>(amax));
                    float d, qinv;
                    q8_scale(amax, d, qinv);
                    if (row >= M) continue;
                    const size_t slot = kslice * M + row;
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        float q = roundf(mul_rn(g[j], qinv));  // f32::round: half away from zero
                        int qi;
                        if (isnan(q)) {
                            qi = 0;  // `NaN as i8` saturates to 0
                        } else {
                            q = fminf(fmaxf(q, -127.0f), 127.0f);
                            qi = (int)q;
                        }
                        ep.q8_qs[slot * 32 + j * 16 + li] = (int8_t)qi;
                    }
                    if (li == 0) ep.q8_d[slot] = __builtin_bit_cast(uint16_t, (_Float16)d);
                }
            return;
        }
    }
    if constexpr (EPI == Epi::Qkv) {
        // The wave's 32 columns are one axis half of one head (N is a
        // multiple of 64): fragment j = 0 holds dims d0 + li, j = 1 holds
        // d0 + 16 + li, the (i, i + 16) pairs of rope::rotate_half
        // (src/rope.rs:84-93).
        if (nw >= N) return;
        const int per = ep.heads * 64;
        const int group = nw / per, head = (nw % per) / 64, d0 = nw % 64;
        float *dst = group == 0 ? ep.q : (group == 1 ? ep.k : ep.v);
        const bool rope = ep.rot != nullptr && group < 2;
        float2 rot[FM][4];
        if (rope) {
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int t = min(mw + i * 16 + 4 * lh + r, M - 1) % ep.tokens;
                    rot[i][r] = *reinterpret_cast<const float2 *>(
                        ep.rot + (((size_t)t * 2 + d0 / 32) * 16 + li) * 2);
                }
        }
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = mw + i * 16 + 4 * lh + r;
                if (row >= M) continue;
                const int img = row / ep.tokens, t = row % ep.tokens;
                float a = acc[i][0][r], b = acc[i][1][r];
                if (ep.bias) {
                    a = add_rn(a, bias[0]);
                    b = add_rn(b, bias[1]);
                }
                if (rope) {
                    const float sn = rot[i][r].x, cs = rot[i][r].y;
                    const float ra = sub_rn(mul_rn(a, cs), mul_rn(b, sn));
                    b = add_rn(mul_rn(b, cs), mul_rn(a, sn));
                    a = ra;
                }
                float *orow = dst + (((size_t)img * ep.heads + head) * ep.tokens + t) * 64 + d0;
                orow[li] = a;
                orow[16 + li] = b;
            }
        return;
    }
    if (whole) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float v = acc[i][j][r];
                    if (ep.bias) v = add_rn(v, bias[j]);
                    if constexpr (EPI == Epi::Gelu) {
                        v = gelu_avx512_form(v);
                    } else {
                        if (ep.gamma) v = mul_rn(v, gamma[j]);
                        if constexpr (EPI == Epi::Residual) v = add_rn(resid[i][j][r], v);
                    }
                    stream_store(row_ptr(i, j, r) + loff, v);
                }
        return;
    }
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) {
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
    if (rows > (size_t)INT32_MAX / 4 || k / 32 > (size_t)INT32_MAX / rows) return hipErrorInvalidValue;
    // Eight rows per workgroup (measured faster than sixteen past the
    // Infinity Cache), four below 2048 rows so that small inputs still spread
    // over every CU.  Past 128 MiB of input the loads are non-temporal:
    // nothing of it stays cached for a consumer at that size.
    const int nbr = (int)(k / 32);
    const bool nt = rows * k * 4 >= (size_t(128) << 20);
    if (rows >= 2048) {
        const unsigned blocks = (unsigned)((rows + 7) / 8);
        if (nt) quantize_tile_q8_0_kernel<true, 8><<<blocks, 256, 0, s>>>(x, qs, d, (int)rows, nbr);
        else quantize_tile_q8_0_kernel<false, 8><<<blocks, 256, 0, s>>>(x, qs, d, (int)rows, nbr);
    } else {
        const unsigned blocks = (unsigned)((rows + 3) / 4);
        quantize_tile_q8_0_kernel<false, 4><<<blocks, 256, 0, s>>>(x, qs, d, (int)rows, nbr);
    }
    return hipGetLastError();
}

// Workgroup tile (FM, FN) of a Q8_0 GEMM: 64x64 when the grid has enough
// workgroups for the 256 CUs, else 32x32 (VESTRA_HIP_Q8_TILE=2x2|2x1|1x2|1x1
// overrides).
static void q8_tile(size_t m, size_t n, int *fm, int *fn) {
    static const char *env = std::getenv("VESTRA_HIP_Q8_TILE");
    if (env && std::strlen(env) == 3 && (env[0] == '1' || env[0] == '2') && env[1] == 'x' &&
        (env[2] == '1' || env[2] == '2')) {
        *fm = env[0] - '0';
        *fn = env[2] - '0';
        return;
    }
    const size_t tiles64 = ((m + 63) / 64) * ((n + 63) / 64);
    *fm = *fn = tiles64 >= 480 ? 2 : 1;
}

// Prefetch distance in blocks: 2, lowered to 1 when the block count is odd
// so that every prefetch group is whole (VESTRA_HIP_Q8_QPF=1|2|4 overrides
// for A/B studies, again lowered to a divisor).  Measured on MI355X with
// the loop's waits exact: 2 and 4 blocks ahead run within 2% of each other
// (config-4 GEMM 19.1 vs 19.3 us, Q8_0 block 102.6 vs 103.6 us), and 2 keeps
// the 64x64 tile at 118 VGPRs (4 waves per SIMD against 3); 8 ahead (176
// VGPRs, 2 waves) took 23.1 us.
static int q8_qpf(size_t nb) {
    static const char *env = std::getenv("VESTRA_HIP_Q8_QPF");
    int want = 2;
    if (env && (env[0] == '1' || env[0] == '2' || env[0] == '4') && env[1] == 0) want = env[0] - '0';
    for (int q = want; q > 1; q /= 2)
        if (nb % q == 0) return q;
    return 1;
}

template <Epi EPI, int FM, int FN>
static void q8_launch(hipStream_t s, const int8_t *a_qs, const uint16_t *a_d, const int8_t *b_qs,
                      const uint16_t *b_d, float *c, size_t m, size_t n, size_t k,
                      const Q8Epi &ep) {
    dim3 grid((unsigned)((n + 32 * FN - 1) / (32 * FN)), (unsigned)((m + 32 * FM - 1) / (32 * FM)));
    switch (q8_qpf(k / 32)) {
        case 4: gemm_q8_0_kernel<EPI, FM, FN, 4><<<grid, 256, 0, s>>>(a_qs, a_d, b_qs, b_d, c, (int)m, (int)n, (int)k, ep); break;
        case 2: gemm_q8_0_kernel<EPI, FM, FN, 2><<<grid, 256, 0, s>>>(a_qs, a_d, b_qs, b_d, c, (int)m, (int)n, (int)k, ep); break;
        default: gemm_q8_0_kernel<EPI, FM, FN, 1><<<grid, 256, 0, s>>>(a_qs, a_d, b_qs, b_d, c, (int)m, (int)n, (int)k, ep); break;
    }
}

template <Epi EPI>
static void q8_dispatch(hipStream_t s, const int8_t *a_qs, const uint16_t *a_d,
                        const int8_t *b_qs, const uint16_t *b_d, float *c, size_t m, size_t n,
                        size_t k, const Q8Epi &ep) {
    int fm, fn;
    q8_tile(m, n, &fm, &fn);
    if (fm == 2 && fn == 2) q8_launch<EPI, 2, 2>(s, a_qs, a_d, b_qs, b_d, c, m, n, k, ep);
    else if (fm == 2) q8_launch<EPI, 2, 1>(s, a_qs, a_d, b_qs, b_d, c, m, n, k, ep);
    else if (fn == 2) q8_launch<EPI, 1, 2>(s, a_qs, a_d, b_qs, b_d, c, m, n, k, ep);
    else q8_launch<EPI, 1, 1>(s, a_qs, a_d, b_qs, b_d, c, m, n, k, ep);
}

// The kernel addresses each operand with 32-bit buffer offsets.
static bool q8_operands_fit(size_t m, size_t n, size_t k) {
    return m * k <= (size_t)INT32_MAX && n * k <= (size_t)INT32_MAX;
}

hipError_t launch_layernorm_q8_0(hipStream_t s, const float *x, const float *gamma,
                                 const float *beta, int8_t *qs, uint16_t *d, size_t rows,
                                 size_t cols, float eps) {
    if (rows == 0) return hipSuccess;
    if (cols % 32 != 0 || cols > 1024 || cols == 0 || rows > (size_t)INT32_MAX / 4 ||
        ((((uintptr_t)x) | ((uintptr_t)gamma) | ((uintptr_t)beta)) & 15) != 0)
        return hipErrorInvalidValue;
    // Four rows (waves) per workgroup: at 865 rows, one row per workgroup
    // measured no faster here.
    layernorm_q8_0_kernel<<<(unsigned)((rows + 3) / 4), 256, 0, s>>>(x, gamma, beta, qs, d,
                                                                     (int)rows, (int)cols, eps);
    return hipGetLastError();
}

hipError_t launch_gemm_q8_0(hipStream_t s, const int8_t *a_qs, const uint16_t *a_d,
                            const int8_t *b_qs, const uint16_t *b_d, float *c, size_t m,
                            size_t n, size_t k, Epi epi, const float *bias, const float *gamma,
                            int8_t *q8_qs, uint16_t *q8_d, bool *quantized) {
    if (quantized) *quantized = false;
    if (m == 0 || n == 0) return hipSuccess;
    if (!q8_operands_fit(m, n, k)) return hipErrorInvalidValue;
    Q8Epi ep{};
    ep.bias = bias;
    ep.gamma = gamma;
    ep.tail_start = m * n - (m * n) % 16;
    if (epi == Epi::Gelu && q8_qs && q8_d && n % 32 == 0) {
        int fm, fn;
        q8_tile(m, n, &fm, &fn);
        if (fn == 2) {
            // The quantised GELU output needs whole 32-column blocks per wave.
            ep.q8_qs = q8_qs;
            ep.q8_d = q8_d;
            if (quantized) *quantized = true;
        }
    }
    switch (epi) {
        case Epi::Store: q8_dispatch<Epi::Store>(s, a_qs, a_d, b_qs, b_d, c, m, n, k, ep); break;
        case Epi::Gelu: q8_dispatch<Epi::Gelu>(s, a_qs, a_d, b_qs, b_d, c, m, n, k, ep); break;
        case Epi::Residual: q8_dispatch<Epi::Residual>(s, a_qs, a_d, b_qs, b_d, c, m, n, k, ep); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemm_q8_0_qkv(hipStream_t s, const int8_t *a_qs, const uint16_t *a_d,
                                const int8_t *b_qs, const uint16_t *b_d, size_t m, size_t k,
                                const float *bias, float *q, float *kk, float *v, size_t tokens,
                                size_t heads, const float *rot) {
    const size_t n = 3 * heads * 64;
    if (m == 0 || heads == 0) return hipSuccess;
    if (tokens == 0 || m % tokens != 0 || !q8_operands_fit(m, n, k)) return hipErrorInvalidValue;
    Q8Epi ep{};
    ep.bias = bias;
    ep.q = q;
    ep.k = kk;
    ep.v = v;
    ep.rot = rot;
    ep.tokens = (int)tokens;
    ep.heads = (int)heads;
    int fm, fn;
    q8_tile(m, n, &fm, &fn);
    if (fm == 2) q8_launch<Epi::Qkv, 2, 2>(s, a_qs, a_d, b_qs, b_d, nullptr, m, n, k, ep);
    else q8_launch<Epi::Qkv, 1, 2>(s, a_qs, a_d, b_qs, b_d, nullptr, m, n, k, ep);
    return hipGetLastError();
}

}  // namespace vh
