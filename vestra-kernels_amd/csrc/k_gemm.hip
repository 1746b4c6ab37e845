// fp32-MFMA projection GEMM for gfx950 with fused epilogues.
//
// C[m,n] = sum_k A[m,k] * Bt[n,k]; A is the activation (row-major), Bt the
// weight prepared once in [out, in] order so both operands stream k-contiguous
// rows.  A workgroup of WM x WN wave64s owns a BM x BN tile and stages BK-wide
// slices of A and Bt in LDS (double-buffered, staged through registers).  A
// slice row is BK floats with no padding; its 16-byte granule g is stored at
// granule g ^ (row % (BK / 4)).  A fragment read (lane l: row l % 16 plus a
// multiple of 16, granule kk/4 + l / 16) then spreads the rows a 16-byte LDS
// access serves together over distinct granules, and so do the slice stores
// (lane l: row l / (BK/4), granule l % (BK/4)).  Measured with
// SQ_LDS_BANK_CONFLICT on MI355X: 0 for this layout at BK = 32 and 64; the
// rows-padded-by-4 layout it replaces conflicted as often as it issued
// MFMAs, and swizzling by row % 8 alone still conflicted at BK = 64.  Each
// wave computes a (BM/WM) x
// (BN/WN) sub-tile with v_mfma_f32_16x16x4_f32: one ds_read_b128 per 16-row
// fragment feeds four MFMA k-steps (lane group h supplies k = kk+4h+s at
// step s).
//
// Split-K (grid.z > 1) is deterministic: each split writes its partial tile
// to a workspace and a reduction kernel sums the partials in split order
// before applying the epilogue.
//
// Epilogues (all separately rounded, as the reference's):
//   Store    : c = (acc + bias) * gamma          (CudaLinearF32::run)
//   Gelu     : c = gelu(acc + bias)              (fc1; the A&S 7.1.26 erf of
//              Kernels::gelu on the hardware reciprocal and exp2, gelu_fast_form)
//   Residual : c = c + (acc + bias) * gamma      (out-proj / fc2 + residual)
//   Qkv      : head-major Q/K/V with bias and the 2-D RoPE rotation of Q, K
//
// LayerNorm fold (LNF, Gelu and Qkv): the GEMM of a pre-norm sub-layer,
// LayerNorm(x) . W^T + b with LayerNorm gamma g and beta be, is computed as
//     rstd * (x . W'^T - mean * c) + b',   W' = W diag(g),
//     c[n] = sum_k W'[n][k],               b' = b + W . be,
// on the raw rows x (W', c and b' prepared once).  Every workgroup sees
// whole rows of A (K is not split), so the row statistics come either from
// the producer of x (LNF == 2: per-chunk mean and M2, merged with Chan's
// formula) or from the A slices as they pass through registers on their way
// to LDS (LNF == 1): each thread sums (x - s) and (x - s)^2 over its chunks,
// with s the mean of the row's first slice, and the threads of a row reduce
// once after the slice loop.  Balanced-tail pieces publish their sums beside
// their partial tiles; the last piece adds them in piece order.  The GEMM
// term x . W'^T - mean * c cancels in proportion to |mean| / std, as the
// crate's own float32 LayerNorm sums do (scalar::layernorm sums the raw row
// in float32 too); staging x - s instead costs fc1 about 1 us per block on
// gfx950, because the subtraction pulls the wait for the next slice's loads
// ahead of the slice's last MFMAs.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace vh {
namespace {

struct EpiArgs {
    float *c;
    const float *bias;
    const float *gamma;
    float *q, *k, *v;
    int tokens, heads;
    const float *rot;
    float *partial;  // split-K: raw partial tiles [split][M][N]
    // Implicit convolution (CONV kernels): Bt is a zero-padded channel-last
    // image [rows][conv_in_c] and row n of the GEMM's Bt for k-slice k0 is
    // image row n + (ky * conv_wp + kx), tap = k0 / conv_in_c = ky * conv_kw + kx.
    // C[m][n] (out channel m, padded-grid position n = y * conv_wp + x) goes
    // to c[m * conv_plane + y * conv_ow + x] for x < conv_ow.
    int conv_in_c, conv_kw, conv_wp, conv_ow;
    size_t conv_plane;
    // Patch scatter (CONV == 2, a kernel == stride transposed convolution):
    // C[m = (oc * kh + ky) * kw + kx][n = iy * iw + ix] goes to
    // c[oc][iy * kh + ky][ix * kw + kx]; bias is per row m.
    int scat_kh, scat_kw, scat_iw;
    // Direct convolution (CONV == 3): Bt is the CHW image [conv_in_c][cd_ih]
    // [cd_iw] read in place; column n is output pixel (n / conv_ow, n %
    // conv_ow) and the output is c[m * N + n]; ReLU on the image when cd_relu.
    int cd_ih, cd_iw, cd_stride, cd_pad, cd_relu;
    // Balanced tail (TAIL kernels): tiles [0, tail_full) run whole; each of
    // the tail_count tiles after them runs as tail_splits K pieces of
    // tail_kps, whose partials (in `partial`, one [FM][FN][4][threads] block
    // per piece) the last piece to finish sums in piece order before the
    // epilogue.  tail_cnt holds one arrival counter per tail tile: zero
    // between launches (the last piece resets it).
    int tail_full, tail_splits, tail_count, tail_kps;
    unsigned *tail_cnt;
    // LayerNorm fold (LNF kernels): per-row sums of the tail pieces
    // ([tail tile][piece][2 * ACH][threads]), c[n] = sum_k Bt[n][k] and eps.
    float *tail_stats;
    const float *ln_c;
    float ln_eps;
    // Row statistics per 32-column chunk, (mean, M2) pairs [M][stats_chunks]:
    // written by a Residual epilogue (stats_out, wave tiles 32 columns wide)
    // for the next pre-norm GEMM, read by LNF == 2 kernels (stats_in).
    float2 *stats_out;
    const float2 *stats_in;
    int stats_chunks;
};

// Applies a Store / Gelu / Residual epilogue to one output element.
template <Epi EPI>
__device__ __forceinline__ void epilogue_store(const EpiArgs &ep, size_t idx, int col, float v) {
    if (ep.bias) v = add_rn(v, ep.bias[col]);
    if constexpr (EPI == Epi::Store) {
        if (ep.gamma) v = mul_rn(v, ep.gamma[col]);
        ep.c[idx] = v;
    } else if constexpr (EPI == Epi::Gelu) {
        ep.c[idx] = gelu_fast_form(v);
    } else {
        if (ep.gamma) v = mul_rn(v, ep.gamma[col]);
        ep.c[idx] = add_rn(ep.c[idx], v);
    }
}

// Workgroup -> (row tile, column tile, split).  The hardware deals
// workgroups round-robin over the 8 XCDs, each with its own L2; the linear
// id is renumbered so that each XCD receives a contiguous run of tile ids
// (a bijection: the first total % 8 XCDs take one more), and tile ids walk
// groups of 8 row tiles column by column, so the run of one XCD covers a
// compact block of C and fetches fewer A row panels and B column panels.
// Measured on MI355X this pays for the batched shapes (M = 4 x 865) and costs
// a little at M = 865, where the GEMMs are not fetch-bound; without
// xcd_order the tiles follow the launch grid.
__device__ __forceinline__ void tile_walk(int t, int nx, int ny, int &tm, int &tn) {
    const int gm = min(8, ny);
    const int group = t / (gm * nx);
    const int first = group * gm;
    const int rows = min(ny - first, gm);
    const int local = t - group * gm * nx;
    tm = first + local % rows;
    tn = local / rows;
}

__device__ __forceinline__ void tile_of_block(bool xcd_order, int &tm, int &tn, int &z) {
    if (!xcd_order) {
        tm = blockIdx.y;
        tn = blockIdx.x;
        z = blockIdx.z;
        return;
    }
    const int nx = gridDim.x, ny = gridDim.y;
    const int total = nx * ny * gridDim.z;
    const int bid = blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z);
    const int q = total / 8, r = total % 8, x = bid % 8;
    const int pid = x * q + min(x, r) + bid / 8;
    const int per = nx * ny;
    z = pid / per;
    tile_walk(pid - z * per, nx, ny, tm, tn);
}

// TAIL grids are one-dimensional: workgroups [0, tail_full) take the whole
// tiles (tail_full % 8 == 0; with xcd_order renumbered as above), and the
// rest the K pieces of the tail tiles, numbered so that the tail_splits
// pieces of one tile share bid % 8, i.e. one XCD and its L2 (with xcd_order
// each XCD's tail tiles are also consecutive in tile_walk order).  Tail
// indices past tail_count (padding to a multiple of 8) return -1.
__device__ __forceinline__ int tail_tile_of_block(const EpiArgs &ep, bool xcd_order, int nx, int ny,
                                                  int &tm, int &tn, int &piece, int &u) {
    const int bid = blockIdx.x;
    int t;
    if (bid < ep.tail_full) {
        piece = -1;
        u = 0;
        t = xcd_order ? (bid % 8) * (ep.tail_full / 8) + bid / 8 : bid;
    } else {
        const int q = bid - ep.tail_full, r = q / 8;
        piece = r % ep.tail_splits;
        // xcd_order: XCD q % 8 takes a contiguous run of tail tiles (a
        // compact patch of C) instead of every 8th.
        u = xcd_order ? (q % 8) * ((ep.tail_count + 7) / 8) + r / ep.tail_splits
                      : (r / ep.tail_splits) * 8 + q % 8;
        if (u >= ep.tail_count) return -1;
        t = ep.tail_full + u;
    }
    if (xcd_order) {
        tile_walk(t, nx, ny, tm, tn);
    } else {
        tm = t / nx;
        tn = t - tm * nx;
    }
    return 0;
}

// Float offset of granule g (4 floats) of slice row r: rows of BK floats,
// granules XOR-swizzled by the row (BK / 4 granules per row, BK >= 32).
template <int BK>
__device__ __forceinline__ int swz(int r, int g) {
    static_assert(BK % 32 == 0, "a slice row holds at least 8 granules");
    return r * BK + 4 * (g ^ (r & (BK / 4 - 1)));
}

template <int BM, int BN, int BK>
constexpr size_t gemm_lds_bytes() {
    return 2 * (size_t)(BM + BN) * BK * sizeof(float);
}

// EXACT: K and the split length are multiples of BK and K % 4 == 0, so every
// k-slice is whole.  Rows past M (columns past N) load a clamped in-range row
// and are NOT zeroed: C[m][n] depends only on A row m and Bt row n, and rows
// or columns past the edge are never stored.  Selecting on the loaded value
// would make the compiler wait for the prefetch before the MFMAs of the
// current slice, so the load path stays select-free.
// CONV (EXACT only): the Bt rows of a k-slice are the padded image rows of
// one convolution tap, shifted by that tap's offset (see EpiArgs); conv_in_c
// is a multiple of BK, so a slice never straddles two taps.  A is the weight
// [out_c][K], so the output tile is channel-major and is written straight to
// the CHW output.  CONV == 2 (EXACT only) is a plain GEMM whose tile rows
// are (out channel, tap) and columns input pixels, stored by the patch
// scatter of EpiArgs; CONV == 4 is the same GEMM with Bt read as CONV == 3
// reads it (a 1 x 1 tap over the CHW input, no transposed copy).  CONV == 3
// (EXACT only) reads the Bt tile straight
// from a CHW image: a thread owns one output pixel of the tile and 8
// channels of the k-slice, so 64 lanes load 64 consecutive pixels of one
// channel; taps outside the image load a clamped in-range pixel and are
// zeroed when the slice is stored to LDS (after the MFMAs), and the output
// is the channel-major tile itself, i.e. CHW.
template <int BM, int BN, int BK, int WM, int WN, Epi EPI, bool SPLIT, bool EXACT, int CONV = 0,
          bool TAIL = false, int LNF = 0>
__global__ __launch_bounds__(WM *WN * 64) void gemm_nt_kernel(const float *__restrict__ A,
                                                              const float *__restrict__ Bt,
                                                              int M, int N, int K,
                                                              int k_per_split, int xcd_order,
                                                              EpiArgs ep) {
    constexpr int NT = WM * WN * 64;
    constexpr int CPR = BK / 4;  // float4 chunks per row slice
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 16, FN = TN / 16;
    constexpr int ACH = BM * CPR / NT;
    constexpr int BCH = BN * CPR / NT;
    static_assert((BM * CPR) % NT == 0 && (BN * CPR) % NT == 0, "tile / thread mismatch");
    static_assert(ACH >= 1 && BCH >= 1, "tile too small for the thread count");
    static_assert(TM % 16 == 0 && TN % 16 == 0 && BK % 16 == 0, "fragment shape");
    static_assert(EPI != Epi::Qkv || TN == 32 || TN == 64,
                  "QKV epilogue needs whole 32-wide RoPE halves of one head per wave tile");

    // LDS buffer b: A slice [BM][BK], then Bt slice [BN][BK].
    constexpr int STAGE = (BM + BN) * BK;
    extern __shared__ __attribute__((aligned(16))) float smem[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lh = lane >> 4;
    const int wm = wave / WN, wn = wave % WN;
    int tile_m, tile_n, split, kbeg, kend;
    int piece = -1, tail_u = 0;
    if constexpr (TAIL) {
        static_assert(!SPLIT && EXACT && (CONV == 0 || CONV == 3),
                      "balanced tail: whole-slice GEMMs and the direct convolution");
        if (tail_tile_of_block(ep, xcd_order != 0, (N + BN - 1) / BN, (M + BM - 1) / BM, tile_m, tile_n,
                               piece, tail_u) < 0)
            return;
        split = 0;
        kbeg = piece < 0 ? 0 : piece * ep.tail_kps;
        kend = piece < 0 ? K : kbeg + ep.tail_kps;
    } else {
        tile_of_block(xcd_order != 0, tile_m, tile_n, split);
        kbeg = split * k_per_split;
        kend = min(K, kbeg + k_per_split);
    }
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const bool vec = (K & 3) == 0;

    // CONV == 3: this thread's pixel (tile column cd_p), channel group and
    // the image position of its (0, 0) tap; cd_ok marks whether the tap of
    // the prefetched slice lies inside the image.
    int cd_p = 0, cd_cg = 0, cd_y = 0, cd_x = 0;
    bool cd_live = false, cd_ok = false;
    if constexpr (CONV == 3 || CONV == 4) {
        static_assert(BN * BK == 8 * NT && NT % BN == 0 && BCH == 2,
                      "direct convolution: one pixel x 8 channels per thread");
        cd_p = tid % BN;
        cd_cg = tid / BN;
        const int n = n0 + cd_p;
        cd_live = n < N;
        const int nc = min(n, N - 1);
        const int y = nc / ep.conv_ow, x = nc - y * ep.conv_ow;
        cd_y = y * ep.cd_stride - ep.cd_pad;
        cd_x = x * ep.cd_stride - ep.cd_pad;
    }

    // A registers of the slice in flight.  LNF keeps two sets, by slice
    // parity, so that the LayerNorm sums of a slice read registers that no
    // load is writing (and need no wait of their own); otherwise one set.
    constexpr bool LN_LOOP = LNF == 1;  // row sums taken from the A slices
    constexpr bool LN_ANY = LNF != 0;
    // LayerNorm fold, statistics from the A slices (LNF == 1): this thread's
    // A chunks c = tid + i * NT all lie in row c / CPR of the tile (NT is a
    // multiple of CPR); ln_s1 / ln_s2 sum x - s and (x - s)^2 over the chunks
    // it sees, with s = ln_sh[i] the mean of the row's first BK elements.
    // Then (s - mean)^2 <= M2 / BK, so S2 = M2 + K (s - mean)^2 stays within
    // (1 + K / BK) M2 whatever the row holds, and S2 / K - (S1 / K)^2 does not
    // cancel (a shift by one element does: x[row][0] far from the mean).
    // The CPR threads of a row hold those BK elements between them (chunk
    // tid % CPR of slice 0), loaded here and summed after the first slice is
    // stored.  Every piece of a balanced-tail tile derives the same shift
    // from the same loads, so their partial sums add.
    constexpr int LA = LN_LOOP ? ACH : 1;
    float ln_sh[LA], ln_s1[LA], ln_s2[LA];
    f32x4 ln_first[LA];
    if constexpr (LN_ANY) {
        static_assert(EXACT && !SPLIT && CONV == 0 && (EPI == Epi::Gelu || EPI == Epi::Qkv),
                      "LayerNorm fold: whole-slice Gelu / Qkv GEMMs");
        static_assert(NT % CPR == 0, "a thread's chunks share one row");
    }
    if constexpr (LN_LOOP) {
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            ln_first[i] = *reinterpret_cast<const f32x4 *>(A + (size_t)min(m0 + (tid + i * NT) / CPR, M - 1) * K +
                                                            (tid % CPR) * 4);
            ln_s1[i] = 0.0f;
            ln_s2[i] = 0.0f;
        }
    }
    f32x4 ra_sets[LN_LOOP ? 2 : 1][ACH], rb[BCH];
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    auto gload = [&](int k0, auto par) {
        f32x4 *ra = ra_sets[LN_LOOP ? decltype(par)::value : 0];
        if constexpr (EXACT) {
#pragma unroll
            for (int i = 0; i < ACH; i++) {
                int c = tid + i * NT, row = c / CPR, kq = (c % CPR) * 4;
                ra[i] = *reinterpret_cast<const f32x4 *>(A + (size_t)min(m0 + row, M - 1) * K + k0 + kq);
            }
        }
        if constexpr (EXACT && CONV == 1) {
            const int tap = k0 / ep.conv_in_c;
            const int shift = (tap / ep.conv_kw) * ep.conv_wp + tap % ep.conv_kw;
            const int kin = k0 - tap * ep.conv_in_c;
#pragma unroll
            for (int i = 0; i < BCH; i++) {
                int c = tid + i * NT, row = c / CPR, kq = (c % CPR) * 4;
                rb[i] = *reinterpret_cast<const f32x4 *>(
                    Bt + ((size_t)min(n0 + row, N - 1) + shift) * ep.conv_in_c + kin + kq);
            }
            return;
        } else if constexpr (EXACT && (CONV == 3 || CONV == 4)) {
            const int tap = k0 / ep.conv_in_c, kin = k0 - tap * ep.conv_in_c;
            const int ky = tap / ep.conv_kw, kx = tap - ky * ep.conv_kw;
            const int yi = cd_y + ky, xi = cd_x + kx;
            cd_ok = cd_live && yi >= 0 && yi < ep.cd_ih && xi >= 0 && xi < ep.cd_iw;
            const size_t hw = (size_t)ep.cd_ih * ep.cd_iw;
            const float *src = Bt + (size_t)(kin + 8 * cd_cg) * hw +
                               (size_t)min(max(yi, 0), ep.cd_ih - 1) * ep.cd_iw + min(max(xi, 0), ep.cd_iw - 1);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                rb[0][e] = src[e * hw];
                rb[1][e] = src[(e + 4) * hw];
            }
            return;
        } else if constexpr (EXACT) {
#pragma unroll
            for (int i = 0; i < BCH; i++) {
                int c = tid + i * NT, row = c / CPR, kq = (c % CPR) * 4;
                rb[i] = *reinterpret_cast<const f32x4 *>(Bt + (size_t)min(n0 + row, N - 1) * K + k0 + kq);
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            int c = tid + i * NT, row = c / CPR, kq = (c % CPR) * 4;
            int gm = m0 + row, gk = k0 + kq;
            const float *p = A + (size_t)gm * K + gk;
            if (vec && gm < M && gk < kend) {
                ra[i] = *reinterpret_cast<const f32x4 *>(p);
            } else {
                f32x4 t;
#pragma unroll
                for (int e = 0; e < 4; e++) t[e] = (gm < M && gk + e < kend) ? p[e] : 0.0f;
                ra[i] = t;
            }
        }
#pragma unroll
        for (int i = 0; i < BCH; i++) {
            int c = tid + i * NT, row = c / CPR, kq = (c % CPR) * 4;
            int gn = n0 + row, gk = k0 + kq;
            const float *p = Bt + (size_t)gn * K + gk;
            if (vec && gn < N && gk < kend) {
                rb[i] = *reinterpret_cast<const f32x4 *>(p);
            } else {
                f32x4 t;
#pragma unroll
                for (int e = 0; e < 4; e++) t[e] = (gn < N && gk + e < kend) ? p[e] : 0.0f;
                rb[i] = t;
            }
        }
    };
    auto lstore = [&](int buf, auto par) {
        const f32x4 *ra = ra_sets[LN_LOOP ? decltype(par)::value : 0];
        float *as = smem + buf * STAGE;
        float *bs = as + BM * BK;
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            int c = tid + i * NT;
            *reinterpret_cast<f32x4 *>(&as[swz<BK>(c / CPR, c % CPR)]) = ra[i];
        }
        if constexpr (CONV == 3 || CONV == 4) {
            // Pixel cd_p, channels 8 cd_cg .. +7 of the slice: ReLU on the
            // image values when asked, zeros for taps outside the image.
#pragma unroll
            for (int i = 0; i < 2; i++) {
                f32x4 v = rb[i];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    if (ep.cd_relu) v[e] = fmaxf(v[e], 0.0f);
                    v[e] = cd_ok ? v[e] : 0.0f;
                }
                *reinterpret_cast<f32x4 *>(&bs[swz<BK>(cd_p, 2 * cd_cg + i)]) = v;
            }
        } else {
#pragma unroll
            for (int i = 0; i < BCH; i++) {
                int c = tid + i * NT;
                *reinterpret_cast<f32x4 *>(&bs[swz<BK>(c / CPR, c % CPR)]) = rb[i];
            }
        }
    };

    // LNF == 2: the producer's statistics of this tile's rows, one (mean,
    // M2) per 32-column chunk of the row (stats_chunks per row), prefetched
    // before the slice loop: TPR threads per row, ln_cpt chunks each (host:
    // stats_chunks == ln_cpt * TPR, ln_cpt <= LCP).  The loads are clamped,
    // not selected, so that nothing waits for them before the loop.
    constexpr int TPR = NT / BM, LCP = 8;
    float2 ln_ch[LNF == 2 ? LCP : 1];
    int ln_cpt = 0;
    if constexpr (LNF == 2) {
        static_assert(NT % BM == 0 && TPR >= 2 && TPR <= 16, "row statistics: 2-16 threads per row");
        ln_cpt = ep.stats_chunks / TPR;
        const float2 *src = ep.stats_in + (size_t)min(m0 + tid / TPR, M - 1) * ep.stats_chunks +
                            (tid % TPR) * ln_cpt;
#pragma unroll
        for (int c = 0; c < LCP; c++) ln_ch[c] = src[min(c, ln_cpt - 1)];
    }
    auto ln_acc = [&](auto par) {
        if constexpr (LN_LOOP) {
            const f32x4 *ra = ra_sets[decltype(par)::value];
#pragma unroll
            for (int i = 0; i < ACH; i++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float d = ra[i][e] - ln_sh[i];
                    ln_s1[i] += d;
                    ln_s2[i] = fmaf(d, d, ln_s2[i]);
                }
        }
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Fragment i (A) / j (Bt) of k-step kk from buffer buf: rows wm*TM + 16i + li
    // (wn*TN + 16j + li), granule kk/4 + lh, i.e. swz(row, kk/4 + lh).  The
    // rows of a lane are li plus multiples of 16, so the swizzle depends on
    // li alone: one per-lane offset per k-step, and everything else is an
    // immediate.
    int goff[BK / 16];
#pragma unroll
    for (int q = 0; q < BK / 16; q++) goff[q] = 4 * ((4 * q + lh) ^ (li & (CPR - 1)));
    f32x4 a[2][FM], b[2][FN];
    auto fetch = [&](int slot, int buf, int kk) {
        const float *as = smem + buf * STAGE + (wm * TM + li) * BK + goff[kk / 16];
        const float *bs = smem + buf * STAGE + BM * BK + (wn * TN + li) * BK + goff[kk / 16];
#pragma unroll
        for (int i = 0; i < FM; i++) a[slot][i] = *reinterpret_cast<const f32x4 *>(as + i * 16 * BK);
#pragma unroll
        for (int j = 0; j < FN; j++) b[slot][j] = *reinterpret_cast<const f32x4 *>(bs + j * 16 * BK);
    };
    auto mstep = [&](int cur, int s) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) acc[i][j] = mfma16x16x4(a[cur][i][s], b[cur][j][s], acc[i][j]);
    };
    // Fragments of k-step kk+16 are read from LDS while the MFMAs of k-step
    // kk run (register double buffering).
    auto compute = [&](int buf) {
        fetch(0, buf, 0);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            const int cur = (kk / 16) & 1;
            if (kk + 16 < BK) fetch(cur ^ 1, buf, kk + 16);
#pragma unroll
            for (int s = 0; s < 4; s++) mstep(cur, s);
        }
    };

    const int ktiles = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    gload(kbeg, P0{});
    lstore(0, P0{});
    __syncthreads();
    if constexpr (LN_LOOP) {
        // After the first slice's stores, so that they do not wait for it.
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            const float part = (ln_first[i][0] + ln_first[i][1]) + (ln_first[i][2] + ln_first[i][3]);
            ln_sh[i] = group_sum<CPR>(part) * (1.0f / BK);
        }
    }
    if constexpr (EXACT) {
        // Branch-free slice loop: the last iteration reloads its own slice
        // into the idle buffer (never read again), so each iteration is one
        // basic block and its instruction order can be pinned: the fragment
        // reads of k-step s+1 and the LDS stores of the next slice issue in
        // the shadow of the MFMAs of k-step s, and the global loads of the
        // next slice go out first.  Unrolled by two, so that the buffer of
        // each slice is a constant and every LDS address is a loop-invariant
        // register plus an immediate.
        // LNF: slice t's own elements (register set t % 2, loaded during
        // slice t - 1 and already waited for by its LDS stores) go into the
        // LayerNorm sums while this slice's loads fill the other set; the
        // sums are free to sit anywhere in the slice.
        auto slice = [&](int t, auto curc) {
            constexpr int cur = decltype(curc)::value;
            using Next = std::integral_constant<int, cur ^ 1>;
            gload(kbeg + min(t + 1, ktiles - 1) * BK, Next{});
            ln_acc(curc);
            compute(cur);
            lstore(cur ^ 1, Next{});
            constexpr int NR = FM + FN, NM = 4 * FM * FN, NL = ACH + BCH;
            __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);  // k-step 0 fragments
            __builtin_amdgcn_sched_group_barrier(0x020, NL, 0);  // next slice, global
#pragma unroll
            for (int s = 0; s + 1 < BK / 16; s++) {
#pragma unroll
                for (int r = 0; r < NR; r++) {
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, NM - NR, 0);
            }
            constexpr int NW = NL < NM ? NL : NM;
#pragma unroll
            for (int r = 0; r < NW; r++) {
                __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, NM - NW, 0);
            __builtin_amdgcn_sched_group_barrier(0x200, NL - NW, 0);
            __syncthreads();
        };
        int t = 0;
        for (; t + 1 < ktiles; t += 2) {
            slice(t, P0{});
            slice(t + 1, P1{});
        }
        if (t < ktiles) slice(t, P0{});
    } else {
        for (int t = 0; t < ktiles; t++) {
            const int cur = t & 1;
            const bool next = t + 1 < ktiles;
            if (next) gload(kbeg + (t + 1) * BK, P0{});
            compute(cur);
            if (next) lstore(cur ^ 1, P0{});
            __syncthreads();
        }
    }

    if constexpr (TAIL) {
        if (piece >= 0) {
            // Publish this piece's partial (coalesced: consecutive threads,
            // consecutive floats), then count it in.  Ordering, step by step:
            //  1. Partials are agent-scope atomic stores, which write through
            //     the XCD's L2 (not coherent across XCDs) to the point where
            //     every XCD reads; none stays dirty in L2.
            //  2. Each thread then waits for its stores to be acknowledged
            //     (vmcnt(0) counts stores on gfx9).  The wait is inline asm
            //     with a memory clobber, so the compiler cannot move a store
            //     past it.
            //  3. The barrier orders every thread's wait before thread 0's
            //     agent-scope counter increment.
            //  4. The piece that sees the last count reads the partials with
            //     agent-scope atomic loads, after the barrier that follows
            //     the increment's return.  Those loads bypass the L2, so they
            //     cannot hit stale lines.
            // This is what an agent-scope release / acquire pair would
            // provide, minus its L2-wide writeback and invalidate, which
            // only non-atomic data needs.  An agent-scope fence here doubled
            // the kernel's time.  No piece waits for another, so the grid
            // drains whatever the residency.
            __shared__ int tail_last;
            constexpr int PER = FM * FN * 4;
            const size_t tile_base = (size_t)tail_u * ep.tail_splits * PER * NT;
            float *mine = ep.partial + tile_base + (size_t)piece * PER * NT;
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        __hip_atomic_store(mine + ((i * FN + j) * 4 + r) * NT + tid, acc[i][j][r],
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            constexpr int LS = 2 * LA;  // LayerNorm sums per thread and piece
            const size_t stats_base = (size_t)tail_u * ep.tail_splits * LS * NT;
            if constexpr (LN_LOOP) {
                float *st = ep.tail_stats + stats_base + (size_t)piece * LS * NT;
#pragma unroll
                for (int i = 0; i < LA; i++) {
                    __hip_atomic_store(st + (2 * i) * NT + tid, ln_s1[i], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(st + (2 * i + 1) * NT + tid, ln_s2[i], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (tid == 0)
                tail_last = __hip_atomic_fetch_add(ep.tail_cnt + tail_u, 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(ep.tail_splits - 1);
            __syncthreads();
            if (!tail_last) return;
            // The sum in piece order, whichever piece finished last.  Every
            // piece's values are loaded before the first add (a uniform
            // branch per piece, no loop-carried wait), so the loads are in
            // flight together rather than one round trip per piece and value.
            constexpr int MAXS = 4;  // tail_splits <= 4 (tail_plan)
            const float *parts = ep.partial + tile_base;
            float pv[MAXS][PER];
            float ps[MAXS][LN_LOOP ? LS : 1];
#pragma unroll
            for (int p = 0; p < MAXS; p++) {
                if (p < ep.tail_splits) {
#pragma unroll
                    for (int e = 0; e < PER; e++)
                        pv[p][e] = __hip_atomic_load(parts + (size_t)(p * PER + e) * NT + tid, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
                    if constexpr (LN_LOOP) {
#pragma unroll
                        for (int e = 0; e < LS; e++)
                            ps[p][e] = __hip_atomic_load(ep.tail_stats + stats_base + (size_t)(p * LS + e) * NT + tid,
                                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < PER; e++) pv[p][e] = 0.0f;
                    if constexpr (LN_LOOP) {
#pragma unroll
                        for (int e = 0; e < LS; e++) ps[p][e] = 0.0f;
                    }
                }
            }
            if constexpr (LN_LOOP) {
#pragma unroll
                for (int i = 0; i < LA; i++) {
                    float s1 = ps[0][2 * i], s2 = ps[0][2 * i + 1];
#pragma unroll
                    for (int p = 1; p < MAXS; p++)
                        if (p < ep.tail_splits) {
                            s1 += ps[p][2 * i];
                            s2 += ps[p][2 * i + 1];
                        }
                    ln_s1[i] = s1;
                    ln_s2[i] = s2;
                }
            }
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int e = (i * FN + j) * 4 + r;
                        float v = pv[0][e];
#pragma unroll
                        for (int p = 1; p < MAXS; p++)
                            if (p < ep.tail_splits) v = v + pv[p][e];
                        acc[i][j][r] = v;
                    }
            if (tid == 0) __hip_atomic_store(ep.tail_cnt + tail_u, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }

    // LayerNorm fold: each row's sums are spread over CPR consecutive lanes;
    // after the reduction one lane per row writes (mean, rstd) to LDS for the
    // epilogue.  LDS is free: every slice ends with a barrier, after the
    // last fragment reads.  mean = s + S1/K, var = S2/K - (S1/K)^2 about the
    // shift s.
    if constexpr (LN_LOOP) {
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            ln_s1[i] = group_sum<CPR>(ln_s1[i]);
            ln_s2[i] = group_sum<CPR>(ln_s2[i]);
        }
        float2 *lns = reinterpret_cast<float2 *>(smem);
        if (tid % CPR == 0) {
            const float kf = (float)K;
#pragma unroll
            for (int i = 0; i < ACH; i++) {
                const float m1 = ln_s1[i] / kf;
                const float var = fmaxf(ln_s2[i] / kf - m1 * m1, 0.0f);
                lns[(tid + i * NT) / CPR] = float2{ln_sh[i] + m1, 1.0f / sqrtf(var + ep.ln_eps)};
            }
        }
        __syncthreads();
    } else if constexpr (LNF == 2) {
        // Chan's merge of equal-width chunks: mean = mean of the chunk
        // means, M2 = sum of (M2_c + w * (mean_c - mean)^2).
        const float w = (float)(K / ep.stats_chunks);
        float msum = 0.0f;
#pragma unroll
        for (int c = 0; c < LCP; c++)
            if (c < ln_cpt) msum += ln_ch[c].x;
        const float mean = group_sum<TPR>(msum) / (float)ep.stats_chunks;
        float q = 0.0f;
#pragma unroll
        for (int c = 0; c < LCP; c++)
            if (c < ln_cpt) {
                const float d = ln_ch[c].x - mean;
                q += fmaf(w * d, d, ln_ch[c].y);
            }
        q = group_sum<TPR>(q);
        if (tid % TPR == 0)
            reinterpret_cast<float2 *>(smem)[tid / TPR] = float2{mean, 1.0f / sqrtf(q / (float)K + ep.ln_eps)};
        __syncthreads();
    }
    // (mean, rstd) of tile row r (LNF only).
    auto ln_row = [&](int r) { return reinterpret_cast<const float2 *>(smem)[r]; };

    // C fragment layout: register r of lane l holds row 4*(l/16)+r, column l%16.
    const int rbase = m0 + wm * TM + 4 * lh;
    if constexpr (SPLIT) {
        float *part = ep.partial + (size_t)split * M * N;
        const int cbase = n0 + wn * TN + li;
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int col = cbase + j * 16;
            if (col >= N) continue;
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = rbase + i * 16 + r;
                    if (row < M) part[(size_t)row * N + col] = acc[i][j][r];
                }
        }
    } else if constexpr (CONV == 2 || CONV == 4) {
        // Row m = (oc, ky, kx), column n = input pixel (iy, ix): the output
        // element (oc, iy * kh + ky, ix * kw + kx).  A lane's four rows 4lh..
        // 4lh+3 are kx = 0..3 of one (oc, ky) when kw == 4 (rows are aligned to
        // 4), i.e. one 16-byte store, and the 16 lanes of a group store 16
        // consecutive pixels of one output row.
        const int kh = ep.scat_kh, kw = ep.scat_kw, iw = ep.scat_iw;
        const int ow = iw * kw;
        const size_t plane = (size_t)(N / iw) * kh * ow;
        const int cbase = n0 + wn * TN + li;
        float bias[FM][4];
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) bias[i][r] = ep.bias ? ep.bias[min(rbase + i * 16 + r, M - 1)] : 0.0f;
        wait_vmem_all();  // then the guarded stores need no waits between them
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int n = cbase + j * 16;
            if (n >= N) continue;
            const int iy = n / iw, ix = n - iy * iw;
#pragma unroll
            for (int i = 0; i < FM; i++) {
                const int m4 = rbase + i * 16;  // multiple of 4
                f32x4 v;
#pragma unroll
                for (int r = 0; r < 4; r++) v[r] = ep.bias ? add_rn(acc[i][j][r], bias[i][r]) : acc[i][j][r];
                if (kw == 4 && m4 + 3 < M) {
                    const int oc = m4 / (4 * kh), ky = (m4 / 4) % kh;
                    *reinterpret_cast<f32x4 *>(ep.c + oc * plane + (size_t)(iy * kh + ky) * ow + ix * 4) = v;
                } else {
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int m = m4 + r;
                        if (m >= M) continue;
                        const int kx = m % kw, ky = (m / kw) % kh, oc = m / (kw * kh);
                        ep.c[oc * plane + (size_t)(iy * kh + ky) * ow + ix * kw + kx] = v[r];
                    }
                }
            }
        }
    } else if constexpr (CONV == 1 || CONV == 3) {
        // Output channel m = row, padded-grid position n = column: conv + bias
        // to CHW, dropping the wp - ow junk columns.  The 16 lanes of a lane
        // group store 16 consecutive positions of one channel.
        float bias[FM][4];
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) bias[i][r] = ep.bias ? ep.bias[min(rbase + i * 16 + r, M - 1)] : 0.0f;
        wait_vmem_all();  // then the guarded stores need no waits between them
        const int cbase = n0 + wn * TN + li;
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int n = cbase + j * 16;
            if (n >= N) continue;
            size_t pix = n;  // CONV == 3: columns are the output pixels
            if constexpr (CONV == 1) {
                const int y = n / ep.conv_wp, x = n - y * ep.conv_wp;
                if (x >= ep.conv_ow) continue;
                pix = (size_t)y * ep.conv_ow + x;
            }
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = rbase + i * 16 + r;
                    if (row >= M) continue;
                    float v = acc[i][j][r];
                    if (ep.bias) v = add_rn(v, bias[i][r]);
                    ep.c[(size_t)row * ep.conv_plane + pix] = v;
                }
        }
    } else if constexpr (EPI == Epi::Qkv) {
        const int colw = n0 + wn * TN;  // first column of this wave's sub-tile
        if (colw >= N) return;
        const int per = ep.heads * 64;
        const int group = colw / per, head = (colw % per) / 64;
        const int d0 = colw % 64;       // 0 or 32 (32-wide tile) / 0 (64-wide)
        float *dst = group == 0 ? ep.q : (group == 1 ? ep.k : ep.v);
        const bool rope = ep.rot != nullptr && group < 2;
        float bias[FN], lc[FN];
#pragma unroll
        for (int j = 0; j < FN; j++) {
            bias[j] = ep.bias[colw + j * 16 + li];
            if constexpr (LN_ANY) lc[j] = ep.ln_c[colw + j * 16 + li];
        }
        // Rotation (sin, cos) of every row this lane stores, read before any
        // store from clamped rows so that the reads overlap.
        float2 rot[FM][4][FN / 2];
        if (rope) {
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int t = min(rbase + i * 16 + r, M - 1) % ep.tokens;
#pragma unroll
                    for (int h = 0; h < FN / 2; h++) {
                        const int axis = d0 / 32 + h;
                        rot[i][r][h] = *reinterpret_cast<const float2 *>(
                            ep.rot + (((size_t)t * 2 + axis) * 16 + li) * 2);
                    }
                }
        }
        wait_vmem_all();  // then the guarded stores need no waits between them
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = rbase + i * 16 + r;
                if (row >= M) continue;
                const int img = row / ep.tokens, t = row % ep.tokens;
                float vals[FN];
                if constexpr (LN_ANY) {
                    const float2 st = ln_row(row - m0);
#pragma unroll
                    for (int j = 0; j < FN; j++) vals[j] = fmaf(st.y, fmaf(-st.x, lc[j], acc[i][j][r]), bias[j]);
                } else {
#pragma unroll
                    for (int j = 0; j < FN; j++) vals[j] = add_rn(acc[i][j][r], bias[j]);
                }
                if (rope) {
                    // rope::rotate_half (src/rope.rs:84-93): dims (i, i+16) of
                    // each 32-wide axis half sit in fragments (2h, 2h+1).
#pragma unroll
                    for (int h = 0; h < FN / 2; h++) {
                        const float sn = rot[i][r][h].x, cs = rot[i][r][h].y;
                        const float a = vals[2 * h], b = vals[2 * h + 1];
                        vals[2 * h] = sub_rn(mul_rn(a, cs), mul_rn(b, sn));
                        vals[2 * h + 1] = add_rn(mul_rn(b, cs), mul_rn(a, sn));
                    }
                }
                float *orow = dst + (((size_t)img * ep.heads + head) * ep.tokens + t) * 64 + d0;
#pragma unroll
                for (int j = 0; j < FN; j++) orow[j * 16 + li] = vals[j];
            }
    } else {
        // Every global read of the epilogue (bias, gamma, and the residual
        // for Residual) is issued from a clamped in-range index before any
        // store, so the reads overlap instead of each waiting behind the
        // bounds branch of its element.
        const int cbase = n0 + wn * TN + li;
        float bias[FN], gamma[FN], lc[FN];
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int col = min(cbase + j * 16, N - 1);
            bias[j] = load_or(ep.bias, (const float *)ep.c, col, 0.0f);
            gamma[j] = load_or(ep.gamma, (const float *)ep.c, col, 1.0f);
            if constexpr (LN_ANY) lc[j] = ep.ln_c[col];
        }
        float2 lnst[LN_ANY ? FM : 1][4];
        if constexpr (LN_ANY) {
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) lnst[i][r] = ln_row(wm * TM + 4 * lh + i * 16 + r);
        }
        float resid[EPI == Epi::Residual ? FM : 1][FN][4];
        float outv[EPI == Epi::Residual ? FM : 1][FN][4];
        if constexpr (EPI == Epi::Residual) {
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const size_t row = min(rbase + i * 16 + r, M - 1);
                        resid[i][j][r] = ep.c[row * N + min(cbase + j * 16, N - 1)];
                    }
        }
        wait_vmem_all();  // then the guarded stores need no waits between them
        // A tile wholly inside C stores without per-element checks; the
        // decision is per tile, so the branch is uniform and the arithmetic
        // is the same either way.
        auto store_all = [&](auto whole_tile) {
            constexpr bool WHOLE = decltype(whole_tile)::value;
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int col = cbase + j * 16;
                if (!WHOLE && col >= N) continue;
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int row = rbase + i * 16 + r;
                        if (!WHOLE && row >= M) continue;
                        const size_t idx = (size_t)row * N + col;
                        float v = acc[i][j][r];
                        if constexpr (LN_ANY)
                            v = fmaf(lnst[i][r].y, fmaf(-lnst[i][r].x, lc[j], v), bias[j]);
                        else if (ep.bias)
                            v = add_rn(v, bias[j]);
                        if constexpr (EPI == Epi::Store) {
                            if (ep.gamma) v = mul_rn(v, gamma[j]);
                            stream_store(ep.c + idx, v);
                        } else if constexpr (EPI == Epi::Gelu) {
                            stream_store(ep.c + idx, gelu_fast_form(v));
                        } else {
                            if (ep.gamma) v = mul_rn(v, gamma[j]);
                            const float o = add_rn(resid[i][j][r], v);
                            stream_store(ep.c + idx, o);
                            if constexpr (EPI == Epi::Residual) outv[i][j][r] = o;
                        }
                    }
            }
        };
        const bool whole = m0 + BM <= M && n0 + BN <= N;
        if (whole)
            store_all(std::true_type{});
        else
            store_all(std::false_type{});
        // Row statistics of the updated rows for the next sub-layer's
        // LayerNorm fold: a wave's 32 columns are one chunk; the 16 lanes of
        // a lane group hold a row's 32 values (two per lane), so the chunk's
        // mean and M2 take two 16-lane sums (two passes, no cancellation).
        if constexpr (EPI == Epi::Residual && TN == 32) {
            if (ep.stats_out && n0 + wn * TN < N) {
                const int chunk = (n0 + wn * TN) / 32;
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float mean = group_sum<16>(outv[i][0][r] + outv[i][1][r]) * (1.0f / 32.0f);
                        const float d0 = outv[i][0][r] - mean, d1 = outv[i][1][r] - mean;
                        const float m2 = group_sum<16>(fmaf(d0, d0, d1 * d1));
                        const int row = rbase + i * 16 + r;
                        if (li == 0 && row < M)
                            ep.stats_out[(size_t)row * ep.stats_chunks + chunk] = float2{mean, m2};
                    }
            }
        }
    }
}

// Residual (or Store) GEMM with the K split inside the workgroup, for the
// narrow short-K projection (the out-projection: 865 x 768 x 768, whose 64 x 64 tiles are
// fewer than the CUs).  KG groups of WM x WN waves share a BM x BN tile;
// group g runs K range [g K / KG, (g + 1) K / KG) through its own double-
// buffered LDS stages (the slice layout and fragment schedule of
// gemm_nt_kernel), all groups in step at one barrier per slice.  The groups'
// partial tiles are then summed through LDS in group order (a fixed order,
// so the result does not depend on timing) and group 0 applies the Residual
// epilogue: c = c + (acc + bias) * gamma.  With 32 x 96 tiles, 2 x 2 waves
// and two K groups the 865-row projection is 224 workgroups of 8 waves, one
// per CU, two waves per SIMD, with no partial tiles leaving the CU and no
// second launch.  With ep.stats_out, group 0 also writes each row's (mean,
// M2) over each wave's TN columns: one chunk per wave column.
template <int BM, int BN, int BK, int WM, int WN, int KG, Epi EPI = Epi::Residual>
__global__ __launch_bounds__(WM *WN *KG * 64) void gemm_kgroup_kernel(const float *__restrict__ A,
                                                                      const float *__restrict__ Bt,
                                                                      int M, int N, int K, EpiArgs ep) {
    constexpr int GT = WM * WN * 64;  // threads per K group
    constexpr int CPR = BK / 4;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 16, FN = TN / 16;
    constexpr int ACH = BM * CPR / GT, BCH = BN * CPR / GT;
    static_assert((BM * CPR) % GT == 0 && (BN * CPR) % GT == 0 && ACH >= 1 && BCH >= 1, "tile / thread mismatch");
    static_assert(TM % 16 == 0 && TN % 16 == 0 && BK % 16 == 0, "fragment shape");
    constexpr int STAGE = (BM + BN) * BK;
    static_assert((KG - 1) * FM * FN * 4 * GT <= KG * 2 * STAGE, "partials fit the staging LDS");
    extern __shared__ __attribute__((aligned(16))) float smem[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kg = wave / (WM * WN), gw = wave % (WM * WN), gt = tid % GT;
    const int li = lane & 15, lh = lane >> 4;
    const int wm = gw / WN, wn = gw % WN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int kper = K / KG, kbeg = kg * kper, ktiles = kper / BK;
    float *gsm = smem + kg * 2 * STAGE;  // this group's two stages

    f32x4 ra[1][ACH], rb[1][BCH];
    auto gload = [&](int k0, int set) {
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            const int c = gt + i * GT, row = c / CPR, kq = (c % CPR) * 4;
            ra[set][i] = *reinterpret_cast<const f32x4 *>(A + (size_t)min(m0 + row, M - 1) * K + k0 + kq);
        }
#pragma unroll
        for (int i = 0; i < BCH; i++) {
            const int c = gt + i * GT, row = c / CPR, kq = (c % CPR) * 4;
            rb[set][i] = *reinterpret_cast<const f32x4 *>(Bt + (size_t)min(n0 + row, N - 1) * K + k0 + kq);
        }
    };
    auto lstore = [&](int buf, int set) {
        float *as = gsm + buf * STAGE;
        float *bs = as + BM * BK;
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            const int c = gt + i * GT;
            *reinterpret_cast<f32x4 *>(&as[swz<BK>(c / CPR, c % CPR)]) = ra[set][i];
        }
#pragma unroll
        for (int i = 0; i < BCH; i++) {
            const int c = gt + i * GT;
            *reinterpret_cast<f32x4 *>(&bs[swz<BK>(c / CPR, c % CPR)]) = rb[set][i];
        }
    };
    const int rbase = m0 + wm * TM + 4 * lh;
    const int cbase = n0 + wn * TN + li;
    float bias[FN], gamma[FN], resid[FM][FN][4];
    static_assert(EPI == Epi::Residual || EPI == Epi::Store, "K-group epilogues: Residual and Store");
    // The epilogue's reads (group 0): bias, LayerScale and the residual tile.
    auto epi_loads = [&]() {
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int col = min(cbase + j * 16, N - 1);
            bias[j] = load_or(ep.bias, (const float *)ep.c, col, 0.0f);
            gamma[j] = load_or(ep.gamma, (const float *)ep.c, col, 1.0f);
        }
        if constexpr (EPI == Epi::Residual) {
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        resid[i][j][r] =
                            ep.c[(size_t)min(rbase + i * 16 + r, M - 1) * N + min(cbase + j * 16, N - 1)];
        }
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    int goff[BK / 16];
#pragma unroll
    for (int q = 0; q < BK / 16; q++) goff[q] = 4 * ((4 * q + lh) ^ (li & (CPR - 1)));
    f32x4 a[2][FM], b[2][FN];
    auto fetch = [&](int slot, int buf, int kk) {
        const float *as = gsm + buf * STAGE + (wm * TM + li) * BK + goff[kk / 16];
        const float *bs = gsm + buf * STAGE + BM * BK + (wn * TN + li) * BK + goff[kk / 16];
#pragma unroll
        for (int i = 0; i < FM; i++) a[slot][i] = *reinterpret_cast<const f32x4 *>(as + i * 16 * BK);
#pragma unroll
        for (int j = 0; j < FN; j++) b[slot][j] = *reinterpret_cast<const f32x4 *>(bs + j * 16 * BK);
    };
    auto compute = [&](int buf) {
        fetch(0, buf, 0);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            const int cur = (kk / 16) & 1;
            if (kk + 16 < BK) fetch(cur ^ 1, buf, kk + 16);
#pragma unroll
            for (int st = 0; st < 4; st++)
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++) acc[i][j] = mfma16x16x4(a[cur][i][st], b[cur][j][st], acc[i][j]);
        }
    };

    gload(kbeg, 0);
    lstore(0, 0);
    __syncthreads();
    // The slice loop of gemm_nt_kernel's whole-slice path: the last slice
    // reloads its own slice into the idle buffer, so every iteration is one
    // basic block whose order is pinned (next slice's global loads first,
    // fragment reads and LDS stores in the shadow of the MFMAs).
    auto slice = [&](int t, int cur) {
        gload(kbeg + min(t + 1, ktiles - 1) * BK, 0);
        compute(cur);
        lstore(cur ^ 1, 0);
        constexpr int NR = FM + FN, NM = 4 * FM * FN, NL = ACH + BCH;
        __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, NL, 0);
#pragma unroll
        for (int st = 0; st + 1 < BK / 16; st++) {
#pragma unroll
            for (int r = 0; r < NR; r++) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, NM - NR, 0);
        }
        constexpr int NW = NL < NM ? NL : NM;
#pragma unroll
        for (int r = 0; r < NW; r++) {
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, NM - NW, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, NL - NW, 0);
        __syncthreads();
    };
    int t = 0;
    for (; t + 1 < ktiles; t += 2) {
        slice(t, 0);
        slice(t + 1, 1);
    }
    if (t < ktiles) slice(t, 0);

    // Group g > 0 leaves its partial tile in LDS (thread-major: conflict-
    // free), and group 0 adds them in group order.  The staging LDS is free:
    // every slice ends with a barrier after its last fragment reads.
    constexpr int PER = FM * FN * 4;
    if (kg > 0) {
        float *mine = smem + (size_t)(kg - 1) * PER * GT;
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) mine[((i * FN + j) * 4 + r) * GT + gt] = acc[i][j][r];
    }
    __syncthreads();
    if (kg > 0) return;
#pragma unroll
    for (int g = 1; g < KG; g++) {
        const float *part = smem + (size_t)(g - 1) * PER * GT;
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) acc[i][j][r] = acc[i][j][r] + part[((i * FN + j) * 4 + r) * GT + gt];
    }

    // Residual epilogue (gemm_nt_kernel's), reads issued before any store.
    epi_loads();
    float outv[FM][FN][4];
    wait_vmem_all();
#pragma unroll
    for (int j = 0; j < FN; j++)
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float v = acc[i][j][r];
                if (ep.bias) v = add_rn(v, bias[j]);
                if (ep.gamma) v = mul_rn(v, gamma[j]);
                const float o = EPI == Epi::Residual ? add_rn(resid[i][j][r], v) : v;
                outv[i][j][r] = o;
                const int row = rbase + i * 16 + r, col = cbase + j * 16;
                if (row < M && col < N) stream_store(ep.c + (size_t)row * N + col, o);
            }
    {
        // The 16 lanes of a lane group hold a row's TN values of this wave
        // (FN per lane): mean and M2 over them by two 16-lane sums.
        if (EPI == Epi::Residual && ep.stats_out) {
            const int chunk = (n0 + wn * TN) / TN;
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float sum = 0.0f;
#pragma unroll
                    for (int j = 0; j < FN; j++) sum += outv[i][j][r];
                    const float mean = group_sum<16>(sum) / (float)TN;
                    float m2 = 0.0f;
#pragma unroll
                    for (int j = 0; j < FN; j++) {
                        const float d = outv[i][j][r] - mean;
                        m2 = fmaf(d, d, m2);
                    }
                    m2 = group_sum<16>(m2);
                    const int row = rbase + i * 16 + r;
                    if (li == 0 && row < M) ep.stats_out[(size_t)row * ep.stats_chunks + chunk] = float2{mean, m2};
                }
        }
    }
}

// Sums the split-K partials in split order, then applies the epilogue; four
// consecutive outputs per thread (N % 4 == 0) so every access is a 16-byte
// vector.
template <Epi EPI>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(int splits, int M, int N, EpiArgs ep) {
    const size_t mn = (size_t)M * N;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    if ((N & 3) == 0) {
        const f32x4 *part = reinterpret_cast<const f32x4 *>(ep.partial);
        for (size_t i4 = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i4 < mn / 4; i4 += stride) {
            // Eight partials in flight at a time (clamped split index: every
            // load in range, none behind a select), added in split order.
            f32x4 v = part[i4];
            for (int base = 1; base < splits; base += 8) {
                f32x4 w[8];
#pragma unroll
                for (int u = 0; u < 8; u++) w[u] = part[(size_t)min(base + u, splits - 1) * (mn / 4) + i4];
#pragma unroll
                for (int u = 0; u < 8; u++)
                    if (base + u < splits)
#pragma unroll
                        for (int e = 0; e < 4; e++) v[e] = add_rn(v[e], w[u][e]);
            }
            const size_t idx = i4 * 4;
            const int col = (int)(idx % N);
#pragma unroll
            for (int e = 0; e < 4; e++) epilogue_store<EPI>(ep, idx + e, col + e, v[e]);
        }
        return;
    }
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < mn; idx += stride) {
        float v = ep.partial[idx];
        for (int base = 1; base < splits; base += 8) {
            float w[8];
#pragma unroll
            for (int u = 0; u < 8; u++) w[u] = ep.partial[(size_t)min(base + u, splits - 1) * mn + idx];
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (base + u < splits) v = add_rn(v, w[u]);
        }
        epilogue_store<EPI>(ep, idx, (int)(idx % N), v);
    }
}

// Split-K of the direct convolution: C = the split-order sum of the
// partials [splits][M][N] plus the bias of row m (the output channel),
// stored to c[m * N + n] (the CHW output).
__global__ __launch_bounds__(256) void conv_splitk_reduce_kernel(int splits, int M, int N,
                                                                 const float *__restrict__ part,
                                                                 const float *__restrict__ bias,
                                                                 float *__restrict__ c) {
    const size_t mn = (size_t)M * N;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= mn) return;
    // Sixteen partials in flight at a time (clamped split index, so every
    // load is in range and none waits behind a select), added in order.
    float v = part[idx];
    for (int base = 1; base < splits; base += 16) {
        float t[16];
#pragma unroll
        for (int u = 0; u < 16; u++) t[u] = part[(size_t)min(base + u, splits - 1) * mn + idx];
#pragma unroll
        for (int u = 0; u < 16; u++)
            if (base + u < splits) v = add_rn(v, t[u]);
    }
    if (bias) v = add_rn(v, bias[idx / N]);
    c[idx] = v;
}

// splitk_reduce_kernel for 2-4 splits and N % 4 == 0: one float4 of outputs
// per thread, every read (partials, bias, gamma, residual) issued before the
// arithmetic.  Per element exactly epilogue_store<EPI> of the split-order sum.
template <Epi EPI, int SPLITS>
__global__ __launch_bounds__(256) void splitk_reduce4_kernel(int M, int N, EpiArgs ep) {
    const size_t mn4 = (size_t)M * N / 4;
    const size_t i4 = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i4 >= mn4) return;
    const f32x4 *part = reinterpret_cast<const f32x4 *>(ep.partial);
    const int col = (int)((i4 * 4) % N);
    f32x4 p[SPLITS];
#pragma unroll
    for (int sp = 0; sp < SPLITS; sp++) p[sp] = part[(size_t)sp * mn4 + i4];
    const f32x4 b = load_or(reinterpret_cast<const f32x4 *>(ep.bias), part, col / 4, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
    const f32x4 g = load_or(reinterpret_cast<const f32x4 *>(ep.gamma), part, col / 4, f32x4{1.0f, 1.0f, 1.0f, 1.0f});
    f32x4 *c4 = reinterpret_cast<f32x4 *>(ep.c) + i4;
    f32x4 x = EPI == Epi::Residual ? *c4 : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 v = p[0];
#pragma unroll
    for (int sp = 1; sp < SPLITS; sp++)
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] = add_rn(v[e], p[sp][e]);
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        float t = v[e];
        if (ep.bias) t = add_rn(t, b[e]);
        if constexpr (EPI == Epi::Gelu) {
            o[e] = gelu_fast_form(t);
        } else {
            if (ep.gamma) t = mul_rn(t, g[e]);
            o[e] = EPI == Epi::Residual ? add_rn(x[e], t) : t;
        }
    }
    *c4 = o;
}

// Split-K reduction fused with the residual update and the LayerNorm of the
// updated rows: one wave per row (N % 4 == 0, N <= 1024).  Each element is
// computed exactly as by splitk_reduce_kernel<Residual>, and each row is
// normalised exactly as by layernorm_kernel, in one pass over the row.  All
// reads of a lane are issued before any arithmetic (chunks past the row end
// read chunk 0 and are dropped), so they are in flight together.
template <int SPLITS>
__global__ __launch_bounds__(256) void splitk_residual_ln_kernel(int M, int N, EpiArgs ep,
                                                                 const float *__restrict__ ln_g,
                                                                 const float *__restrict__ ln_b,
                                                                 float *__restrict__ ln_out,
                                                                 float eps) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= M) return;
    const int n4 = N >> 2;
    const size_t mn4 = (size_t)M * n4;
    const f32x4 *part = reinterpret_cast<const f32x4 *>(ep.partial);
    f32x4 *c4 = reinterpret_cast<f32x4 *>(ep.c + (size_t)row * N);
    const f32x4 *bias4 = reinterpret_cast<const f32x4 *>(ep.bias);
    const f32x4 *gamma4 = reinterpret_cast<const f32x4 *>(ep.gamma);
    f32x4 p[4][SPLITS], x[4], b[4], g[4], lg[4], lb[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int idx = lane + j * 64 < n4 ? lane + j * 64 : 0;
        const size_t i4 = (size_t)row * n4 + idx;
#pragma unroll
        for (int sp = 0; sp < SPLITS; sp++) p[j][sp] = part[(size_t)sp * mn4 + i4];
        x[j] = c4[idx];
        b[j] = load_or(bias4, (const f32x4 *)c4, idx, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
        g[j] = load_or(gamma4, (const f32x4 *)c4, idx, f32x4{1.0f, 1.0f, 1.0f, 1.0f});
        lg[j] = reinterpret_cast<const f32x4 *>(ln_g)[idx];
        lb[j] = reinterpret_cast<const f32x4 *>(ln_b)[idx];
    }
    wait_vmem_all();  // one wait for all of them; the stores below then need none
    f32x4 r[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const bool live = lane + j * 64 < n4;
        f32x4 v = p[j][0];
#pragma unroll
        for (int sp = 1; sp < SPLITS; sp++)
#pragma unroll
            for (int e = 0; e < 4; e++) v[e] = add_rn(v[e], p[j][sp][e]);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            if (ep.bias) v[e] = add_rn(v[e], b[j][e]);
            if (ep.gamma) v[e] = mul_rn(v[e], g[j][e]);
            x[j][e] = add_rn(x[j][e], v[e]);
        }
        r[j] = live ? x[j] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (live) c4[lane + j * 64] = x[j];
    }
    float mean, inv;
    ln_row_stats(r, lane, n4, N, eps, mean, inv);
    f32x4 *y4 = reinterpret_cast<f32x4 *>(ln_out + (size_t)row * N);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int idx = lane + j * 64;
        if (idx < n4) y4[idx] = ln_apply(r[j], mean, inv, lg[j], lb[j]);
    }
}

struct Tile {
    int bm, bn, bk, wm, wn;
};

// XCD-grouped tile order (tile_of_block), by shape, from FETCH_SIZE /
// WRITE_SIZE counters and kernel traces on MI355X:
// - past 1024 rows, where the operand panels outgrow what the XCDs' L2s
//   share (fc2 at M = 3460: 148 -> 140 us);
// - long K (fc2 at 865 tokens, split K): 105 -> 50 MB fetched and written,
//   time unchanged;
// and not for the other launches at 865 tokens: QKV and the out-projection
// fetch less with it but ran 0.3-0.4 us slower, and fc1's 48 column tiles
// in launch order already give each XCD one strip of columns for its whole
// and tail tiles alike (38 MB fetched against 44 MB with it, at the same
// time).  The convolution and patch-scatter
// GEMMs keep the row rule.  VESTRA_HIP_GEMM_XCD=0|1 forces it off or on (A/B
// studies).
int use_xcd_order(const GemmArgs &g) {
    static const char *env = std::getenv("VESTRA_HIP_GEMM_XCD");
    if (env && (env[0] == '0' || env[0] == '1') && env[1] == 0) return env[0] - '0';
    if (g.conv_in_c || g.scatter_kw) return g.m > 1024;
    return g.m > 1024 || g.k >= 2048;
}

template <int BM, int BN, int BK, int WM, int WN, Epi EPI, bool SPLIT, bool EXACT, int CONV = 0,
          int LNF = 0>
hipError_t launch_tile(hipStream_t s, const GemmArgs &g, const EpiArgs &ep, int splits, int kps) {
    constexpr size_t lds = gemm_lds_bytes<BM, BN, BK>();
    auto kernel = gemm_nt_kernel<BM, BN, BK, WM, WN, EPI, SPLIT, EXACT, CONV, false, LNF>;
    static std::atomic<uint64_t> configured{0};
    if (hipError_t e = ensure_dynamic_lds(kernel, lds, configured); e != hipSuccess) return e;
    dim3 grid((unsigned)((g.n + BN - 1) / BN), (unsigned)((g.m + BM - 1) / BM), (unsigned)splits);
    const int xcd_order = use_xcd_order(g);
    kernel<<<grid, WM * WN * 64, lds, s>>>(g.a, g.bt, (int)g.m, (int)g.n, (int)g.k, kps, xcd_order, ep);
    return hipGetLastError();
}

template <int BM, int BN, int BK, int WM, int WN, Epi EPI, bool SPLIT>
hipError_t run_tile(hipStream_t s, const GemmArgs &g, const EpiArgs &ep, int splits) {
    const int kps = (int)(((g.k + splits - 1) / splits + BK - 1) / BK * BK);
    // K == 0 takes the masked path: the whole-slice loads would touch empty operands.
    const bool exact = g.k > 0 && g.k % BK == 0 && (size_t)kps * splits == g.k;
    if (exact) return launch_tile<BM, BN, BK, WM, WN, EPI, SPLIT, true>(s, g, ep, splits, kps);
    return launch_tile<BM, BN, BK, WM, WN, EPI, SPLIT, false>(s, g, ep, splits, kps);
}

template <Epi EPI, bool SPLIT>
hipError_t run_cfg(hipStream_t s, const GemmArgs &g, const EpiArgs &ep, const Tile &t, int splits) {
#define VH_TILE(BM, BN, BK, WM, WN)                                                    \
    if constexpr (EPI != Epi::Qkv || (BN) / (WN) == 64 || (BN) / (WN) == 32) {           \
        if (t.bm == BM && t.bn == BN && t.bk == BK && t.wm == WM && t.wn == WN)        \
            return run_tile<BM, BN, BK, WM, WN, EPI, SPLIT>(s, g, ep, splits);          \
    }
    VH_TILE(64, 128, 32, 2, 2)
    VH_TILE(64, 64, 32, 2, 2)
    VH_TILE(64, 128, 32, 2, 4)
    VH_TILE(32, 128, 32, 1, 4)
    VH_TILE(128, 128, 32, 2, 4)
    VH_TILE(64, 128, 64, 2, 4)
    VH_TILE(32, 128, 64, 1, 4)
    VH_TILE(128, 128, 64, 2, 4)
    VH_TILE(64, 64, 64, 2, 2)
    VH_TILE(64, 256, 32, 2, 4)
    VH_TILE(128, 64, 32, 4, 2)
#undef VH_TILE
    return hipErrorInvalidValue;
}

// VESTRA_HIP_GEMM_TILE="BMxBNxBKxWMxWNxSPLIT" overrides the per-shape choice
// (A/B studies); unknown tiles fall back to the default.
bool tile_override(Tile *t, int *splits) {
    const char *e = std::getenv("VESTRA_HIP_GEMM_TILE");
    if (!e || !*e) return false;
    Tile o{};
    int sp = 1;
    if (std::sscanf(e, "%dx%dx%dx%dx%dx%d", &o.bm, &o.bn, &o.bk, &o.wm, &o.wn, &sp) < 5) return false;
    *t = o;
    *splits = sp > 0 ? sp : 1;
    return true;
}

// Per-shape defaults from the kernel-trace tile sweep on MI355X (DA3
// projections at 865 and 4 x 865 tokens).  Only the long-K narrow projection
// (fc2: K = 3072, N = 768) splits K: with K = 768 the 64x64 grid already
// keeps every CU busy for less time than a separate reduction costs.  Where
// the 64x64 grid of such a split launch has fewer tiles than CUs, dispatch
// runs it as the balanced tail instead (K pieces summed by the last piece).
void default_tile(const GemmArgs &g, Tile *t, int *splits) {
    *splits = 1;
    const bool narrow = g.n <= 1024;
    const bool long_k = g.k >= 2048;
    if (g.m <= 1024) {
        if (narrow && long_k) {
            *t = Tile{64, 128, 64, 2, 4};
            *splits = 3;
        } else if (narrow || g.n >= 3072) {
            *t = Tile{64, 64, 32, 2, 2};
        } else {
            *t = Tile{64, 128, 64, 2, 4};
        }
    } else {
        // QKV at 4 x 865 tokens: 107.1 us against 108.8 for 128 x 128 x 32.
        // fc2 (narrow, long K) at 4 x 865 tokens: 132.7 us unsplit (with the
        // balanced tail for its last round) against 137.3 for 128 x 128 x 32
        // split-K 3 with its reduction, and its Residual epilogue then writes
        // the row statistics the next layer's QKV takes (the 12-layer
        // encoder 6.51 -> 6.37 ms).
        *t = Tile{64, 64, 32, 2, 2};
    }
}

int cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        cache[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

struct TailPlan {
    int full, splits, count;
};

// Balanced tail for the 64 x 64 x 32 tile.  With T tiles on C CUs the
// workgroup-per-tile grid ends with a partial round (at M = 865, N = 3072:
// 672 tiles, 3 on some CUs and 2 on others), and the kernel lasts as long as
// the busiest CU.  Running the whole rounds as they are and the T % C tiles
// after them as S pieces of K / S each brings the busiest CU's load from
// ceil(T / C) tiles to T / C rounded down plus ceil(S (T % C) / C) / S.  S is
// the smallest of 2..4 with the lowest load (pieces of at least 4 slices).
// With fewer tiles than CUs there is no whole round and every tile runs as
// pieces (the 865 x 768 x 768 projection: 168 tiles, 504 pieces).
// VESTRA_HIP_GEMM_TAIL=0 turns the tail off and =1 takes it whenever it
// lowers the load at all (A/B studies and tests).  only_splits, if set, is
// the one piece count allowed.
bool tail_plan(const GemmArgs &g, const Tile &t, TailPlan *plan, int only_splits = 0) {
    if (t.bm != 64 || t.bn != 64 || t.bk != 32 || t.wm != 2 || t.wn != 2) return false;
    if (!g.tail_ws || !g.tail_cnt || g.k == 0 || g.k % 32 != 0) return false;
    const char *env = std::getenv("VESTRA_HIP_GEMM_TAIL");
    if (env && env[0] == '0') return false;
    const bool forced = env && env[0] == '1';
    const long cus = cu_count();
    if (cus <= 0) return false;
    const long tiles = (long)((g.m + 63) / 64) * (long)((g.n + 63) / 64);
    const long full = tiles / cus * cus, rem = tiles - full;
    const long count8 = (rem + 7) / 8 * 8;
    if (rem == 0 || full % 8 != 0) return false;
    const long ktiles = (long)(g.k / 32);
    // Measured on MI355X (fc1-shaped, N = 3072, K = 768, per-launch events,
    // tail off -> on): M = 512 38.5 -> 32.6 us, 832 51.8 -> 46.1, 865 52.4 ->
    // 50.1, 1730 98.7 -> 91.8, 3460 175.9 -> 171.8 (predicted loads -25%,
    // -17%, -11%, -12%, -6%).  The fix-up's partial reads are all in flight
    // at once; when each waited for the one before, the tail lost at M = 865
    // and 3460.  Hence a tail for any predicted cut of 5% or more.
    const double whole = (double)(full / cus + 1);
    double best = forced ? whole : whole * 0.95;
    int pick = 0;
    for (int sp = 2; sp <= 4; sp++) {
        if (ktiles % sp != 0 || ktiles / sp < 4 || (only_splits && sp != only_splits)) continue;
        if ((size_t)count8 > g.tail_cnt_n || (size_t)(count8 * sp) * 64 * 64 > g.tail_ws_floats) continue;
        const double load = (double)(full / cus) + (double)((rem * sp + cus - 1) / cus) / sp;
        if (load < best) {
            best = load;
            pick = sp;
        }
    }
    if (!pick || full + pick * count8 > INT32_MAX) return false;
    *plan = TailPlan{(int)full, pick, (int)rem};
    return true;
}

template <Epi EPI, int LNF = 0, int CONV = 0>
hipError_t launch_tail(hipStream_t s, const GemmArgs &g, EpiArgs ep, const TailPlan &p) {
    constexpr int BM = 64, BN = 64, BK = 32, WM = 2, WN = 2;
    constexpr size_t lds = gemm_lds_bytes<BM, BN, BK>();
    auto kernel = gemm_nt_kernel<BM, BN, BK, WM, WN, EPI, false, true, CONV, true, LNF>;
    static std::atomic<uint64_t> configured{0};
    if (hipError_t e = ensure_dynamic_lds(kernel, lds, configured); e != hipSuccess) return e;
    ep.partial = g.tail_ws;
    ep.tail_stats = g.tail_stats;
    ep.tail_cnt = g.tail_cnt;
    ep.tail_full = p.full;
    ep.tail_splits = p.splits;
    ep.tail_count = p.count;
    ep.tail_kps = (int)g.k / p.splits;
    const unsigned blocks = (unsigned)(p.full + p.splits * ((p.count + 7) / 8 * 8));
    const int xcd_order = use_xcd_order(g);
    kernel<<<blocks, WM * WN * 64, lds, s>>>(g.a, g.bt, (int)g.m, (int)g.n, (int)g.k, (int)g.k, xcd_order, ep);
    return hipGetLastError();
}

// The in-workgroup split-K Residual and Store GEMM (gemm_kgroup_kernel, 32 x 96 tiles,
// 2 K groups of 2 x 2 waves, 64-wide k-slices when each group has at least
// two of them, else 32-wide): taken for M, K, N <= 1024 (the out-
// projection at 865 tokens: 15.6 us as the balanced tail's 504 pieces), when
// N % 96 == 0 and each group has at least two whole 32-wide slices.  A sweep
// of tiles, wave shapes and group counts at 865 x 768 x 768 (lab, 200-launch
// bursts): 13.3 us here with 32-wide slices, 13.7 for 32 x 48 with two
// groups of 2 x 1, 15.0 for 64 x 48 with four groups of 2 x 1, 15.9 for
// 64 x 64 with two groups.  In the block (per-launch events, two alternating
// runs): 32-wide slices 17.3 us, three K groups 16.7, four 16.8, 64-wide
// slices (half the barriers) 16.6-16.7.
// VESTRA_HIP_GEMM_KGROUP=0 never takes it, =1 whenever the shape allows.
bool use_kgroup(const GemmArgs &g) {
    constexpr size_t KG = 2, BK = 32;
    if (g.n % 96 != 0 || g.k % (KG * BK) != 0 || g.k / KG < 2 * BK || g.m > INT32_MAX) return false;
    const char *env = std::getenv("VESTRA_HIP_GEMM_KGROUP");  // per call (tests switch it)
    if (env && env[0] == '0') return false;
    if (env && env[0] == '1') return true;
    return g.m <= 1024 && g.k <= 1024 && g.n <= 1024;
}

template <Epi EPI, int BM, int BN, int BK, int WM, int WN, int KG>
hipError_t launch_kgroup_t(hipStream_t s, const GemmArgs &g, EpiArgs ep) {
    constexpr size_t lds = (size_t)KG * 2 * (BM + BN) * BK * sizeof(float);
    auto kernel = gemm_kgroup_kernel<BM, BN, BK, WM, WN, KG, EPI>;
    static std::atomic<uint64_t> configured{0};
    if (hipError_t e = ensure_dynamic_lds(kernel, lds, configured); e != hipSuccess) return e;
    if (EPI == Epi::Residual && g.stats_out) {
        ep.stats_out = reinterpret_cast<float2 *>(g.stats_out);
        ep.stats_chunks = (int)(g.n / (BN / WN));
        if (g.stats_out_chunks) *g.stats_out_chunks = ep.stats_chunks;
    }
    dim3 grid((unsigned)(g.n / BN), (unsigned)((g.m + BM - 1) / BM));
    kernel<<<grid, WM * WN * KG * 64, lds, s>>>(g.a, g.bt, (int)g.m, (int)g.n, (int)g.k, ep);
    return hipGetLastError();
}

template <Epi EPI>
hipError_t launch_kgroup(hipStream_t s, const GemmArgs &g, EpiArgs ep) {
    if (g.k % (2 * 64) == 0 && g.k / 2 >= 2 * 64) return launch_kgroup_t<EPI, 32, 96, 64, 2, 2, 2>(s, g, ep);
    return launch_kgroup_t<EPI, 32, 96, 32, 2, 2, 2>(s, g, ep);
}

// LayerNorm-folded Gelu / Qkv GEMM (ln_fold_c set): whole slices and no K
// split, on the 64x128x64 tile where the per-shape table picks it and the
// 64x64x32 tile otherwise (with the balanced tail for Gelu when tail_plan
// takes it).  The row statistics come from the producer's chunk statistics
// (stats_in) when given in a shape the tile takes, else from the A slices.
template <Epi EPI, int LNF>
hipError_t launch_lnf(hipStream_t s, const GemmArgs &g, const EpiArgs &ep, bool wide) {
    if constexpr (EPI == Epi::Gelu) {
        TailPlan p;
        if (!wide && g.tail_stats && tail_plan(g, Tile{64, 64, 32, 2, 2}, &p))
            return launch_tail<EPI, LNF>(s, g, ep, p);
    }
    if (wide) return launch_tile<64, 128, 64, 2, 4, EPI, false, true, 0, LNF>(s, g, ep, 1, (int)g.k);
    return launch_tile<64, 64, 32, 2, 2, EPI, false, true, 0, LNF>(s, g, ep, 1, (int)g.k);
}

template <Epi EPI>
hipError_t dispatch_lnf(hipStream_t s, const GemmArgs &g, EpiArgs ep) {
    Tile t;
    int splits;
    if (!tile_override(&t, &splits)) default_tile(g, &t, &splits);
    const bool wide = t.bm == 64 && t.bn == 128 && t.bk == 64 && t.wm == 2 && t.wn == 4;
    const int bk = wide ? 64 : 32;
    if (g.k == 0 || g.k % bk != 0 || !g.bias) return hipErrorInvalidValue;
    const size_t tpr = wide ? 8 : 4;  // threads per tile row (NT / BM)
    const size_t ch = g.stats_in_chunks;
    // VESTRA_HIP_LN_STATS=0 ignores the producer's statistics (A/B studies
    // and tests of both forms; read per call).
    const char *env = std::getenv("VESTRA_HIP_LN_STATS");
    const bool use_in = !(env && env[0] == '0');
    if (use_in && g.stats_in && ch && g.k % ch == 0 && ch % tpr == 0 && ch / tpr <= 8) {
        ep.stats_in = reinterpret_cast<const float2 *>(g.stats_in);
        ep.stats_chunks = (int)ch;
        return launch_lnf<EPI, 2>(s, g, ep, wide);
    }
    return launch_lnf<EPI, 1>(s, g, ep, wide);
}

template <Epi EPI>
hipError_t dispatch(hipStream_t s, const GemmArgs &g, EpiArgs ep) {
    if (g.ln_fold_c) {
        if constexpr (EPI == Epi::Gelu || EPI == Epi::Qkv) return dispatch_lnf<EPI>(s, g, ep);
        return hipErrorInvalidValue;
    }
    Tile t;
    int splits;
    const bool overridden = tile_override(&t, &splits);
    if (!overridden) default_tile(g, &t, &splits);
    if (EPI == Epi::Qkv) splits = 1;
    const int table_splits = !overridden && splits > 1 ? splits : 0;
    if (splits > 1 && (g.ws == nullptr || g.ws_floats < (size_t)splits * g.m * g.n)) splits = 1;
    // Residual with stats_out: the 64-wide tiles of the tail and of the
    // unsplit 64 x 64 x 32 launch (32-column wave tiles) also write the row
    // statistics of the updated rows (chunks per row in stats_out_chunks).
    auto with_stats = [&](EpiArgs e) {
        if (EPI == Epi::Residual && g.stats_out && g.n % 32 == 0) {
            e.stats_out = reinterpret_cast<float2 *>(g.stats_out);
            e.stats_chunks = (int)(g.n / 32);
            if (g.stats_out_chunks) *g.stats_out_chunks = e.stats_chunks;
        }
        return e;
    };
    if (g.stats_out_chunks) *g.stats_out_chunks = 0;
    if constexpr (EPI == Epi::Residual) {
        if (!overridden && use_kgroup(g)) return launch_kgroup<EPI>(s, g, ep);
    } else if constexpr (EPI == Epi::Store) {
        // A Store GEMM keeps whole K per tile when the balanced tail is
        // switched off (VESTRA_HIP_GEMM_TAIL=0: the summation order of an
        // unsplit tile, which the direct convolution reproduces bit for bit).
        const char *tail = std::getenv("VESTRA_HIP_GEMM_TAIL");
        if (!overridden && !(tail && tail[0] == '0') && use_kgroup(g)) return launch_kgroup<EPI>(s, g, ep);
    }
    if constexpr (EPI != Epi::Qkv) {
        // Store, GELU and Residual: the last piece of a tail tile runs the
        // epilogue once (a Residual tile adds its residual exactly once).
        TailPlan p;
        if (splits == 1 && tail_plan(g, t, &p)) return launch_tail<EPI>(s, g, with_stats(ep), p);
        // A long-K launch that the table splits, whose 64 x 64 grid has
        // fewer tiles than CUs (fc2 at 865 tokens: 168 tiles): every tile as
        // K pieces, the last piece of each summing them in order and running
        // the epilogue, saves the separate reduction launch (fc2 41.3 against
        // 42.1 us for split-K 3 of 64 x 128 tiles plus the reduction).  The
        // pieces are the table's K ranges, so each output is the same sum of
        // the same partials as split-K with its reduction (the encoder's
        // fused fc2 reduction and LayerNorm still splits K that way).
        if (table_splits && g.k % ((size_t)table_splits * t.bk) == 0 &&
            tail_plan(g, Tile{64, 64, 32, 2, 2}, &p, table_splits) && p.full == 0)
            return launch_tail<EPI>(s, g, with_stats(ep), p);
    }
    if (splits == 1) {
        const bool narrow_wave = t.bm == 64 && t.bn == 64 && t.bk == 32 && t.wm == 2 && t.wn == 2;
        hipError_t e = run_cfg<EPI, false>(s, g, narrow_wave ? with_stats(ep) : ep, t, 1);
        if (e == hipErrorInvalidValue) {
            if (g.stats_out_chunks) *g.stats_out_chunks = 0;
            default_tile(g, &t, &splits);
            e = run_cfg<EPI, false>(s, g, ep, t, 1);
        }
        return e;
    }
    if constexpr (EPI == Epi::Qkv) {
        return hipErrorInvalidValue;
    } else {
        ep.partial = g.ws;
        hipError_t e = run_cfg<EPI, true>(s, g, ep, t, splits);
        if (e != hipSuccess) return e;
        size_t mn = g.m * g.n;
        if (g.n % 4 == 0 && splits >= 2 && splits <= 4) {
            const unsigned blocks = (unsigned)((mn / 4 + 255) / 256);
            const int m = (int)g.m, n = (int)g.n;
            if (splits == 2) splitk_reduce4_kernel<EPI, 2><<<blocks, 256, 0, s>>>(m, n, ep);
            else if (splits == 3) splitk_reduce4_kernel<EPI, 3><<<blocks, 256, 0, s>>>(m, n, ep);
            else splitk_reduce4_kernel<EPI, 4><<<blocks, 256, 0, s>>>(m, n, ep);
            return hipGetLastError();
        }
        unsigned blocks = (unsigned)std::min<size_t>((mn / 4 + 255) / 256, 4096);
        if (blocks == 0) blocks = 1;
        splitk_reduce_kernel<EPI><<<blocks, 256, 0, s>>>(splits, (int)g.m, (int)g.n, ep);
        return hipGetLastError();
    }
}

// Implicit convolution: Store epilogue, whole slices, no K split.  The tile
// comes from the per-shape table; its BK must divide the channel count.
hipError_t dispatch_conv(hipStream_t s, const GemmArgs &g, const EpiArgs &ep) {
    Tile t;
    int splits;
    if (!tile_override(&t, &splits)) default_tile(g, &t, &splits);
    if (g.conv_in_c % t.bk != 0) t = Tile{64, 64, 32, 2, 2};
    if (g.conv_in_c % t.bk != 0 || g.k % t.bk != 0 || g.k == 0) return hipErrorInvalidValue;
    const int kps = (int)g.k;
#define VH_CONV_TILE(BM, BN, BK, WM, WN)                                                    \
    if (t.bm == BM && t.bn == BN && t.bk == BK && t.wm == WM && t.wn == WN)                 \
        return launch_tile<BM, BN, BK, WM, WN, Epi::Store, false, true, 1>(s, g, ep, 1, kps);
    VH_CONV_TILE(64, 64, 32, 2, 2)
    VH_CONV_TILE(128, 128, 32, 2, 4)
    VH_CONV_TILE(64, 128, 64, 2, 4)
    VH_CONV_TILE(64, 128, 32, 2, 4)
#undef VH_CONV_TILE
    return launch_tile<64, 64, 32, 2, 2, Epi::Store, false, true, 1>(s, g, ep, 1, kps);
}

// Direct convolution of a CHW image: the 64 x 64 x 32 tile (one pixel and
// 8 channels per thread in the loader), with the balanced tail when the
// tiles leave a partial last round over the CUs (tail_plan; the DPT 3x3
// 128 -> 128 convolution on 144 x 96: 432 tiles, the last 176 as 4 K
// pieces).
hipError_t dispatch_conv_direct(hipStream_t s, const GemmArgs &g, const EpiArgs &ep) {
    if (g.conv_in_c % 32 != 0 || g.k % 32 != 0 || g.k == 0) return hipErrorInvalidValue;
    // Grids of fewer than a quarter as many tiles as CUs (small outputs,
    // long K: 768 -> 128 over 12 x 18 is 8 tiles of K = 6912) split K over
    // up to CUs / tiles workgroups of at least 4 slices, into the
    // balanced tail's workspace (at most CUs x 64 x 64 floats), and a second
    // launch sums the splits in order and adds the bias; the tail's 4 pieces
    // would leave most CUs idle.
    // VESTRA_HIP_GEMM_TAIL=0 keeps every tile whole (A/B runs and tests).
    const char *tail_env = std::getenv("VESTRA_HIP_GEMM_TAIL");
    const long cus = cu_count();
    const long tiles = (long)((g.m + 63) / 64) * (long)((g.n + 63) / 64);
    const long ks = (long)(g.k / 32);
    if (!(tail_env && tail_env[0] == '0') && cus > 0 && g.tail_ws && tiles * 4 < cus) {
        long sp = std::min(cus / tiles, ks / 4);
        while (sp > 4 && ks % sp != 0) sp--;
        if (sp > 4 && (size_t)sp * g.m * g.n <= g.tail_ws_floats) {
            EpiArgs e2 = ep;
            e2.partial = g.tail_ws;
            hipError_t e = launch_tile<64, 64, 32, 2, 2, Epi::Store, true, true, 3>(s, g, e2, (int)sp,
                                                                                   (int)(g.k / sp));
            if (e != hipSuccess) return e;
            const size_t mn = g.m * g.n;
            conv_splitk_reduce_kernel<<<(unsigned)((mn + 255) / 256), 256, 0, s>>>(
                (int)sp, (int)g.m, (int)g.n, g.tail_ws, ep.bias, ep.c);
            return hipGetLastError();
        }
    }
    TailPlan p;
    if (tail_plan(g, Tile{64, 64, 32, 2, 2}, &p)) return launch_tail<Epi::Store, 0, 3>(s, g, ep, p);
    return launch_tile<64, 64, 32, 2, 2, Epi::Store, false, true, 3>(s, g, ep, 1, (int)g.k);
}

// Patch-scatter GEMM (k % 32 == 0): one 64 x 64 x 32 tile shape, since the
// row count (out_c * kh * kw) and the pixel count are both moderate.
hipError_t dispatch_scatter(hipStream_t s, const GemmArgs &g, const EpiArgs &ep) {
    if (g.k % 32 != 0 || g.k == 0) return hipErrorInvalidValue;
    if (g.scatter_chw) return launch_tile<64, 64, 32, 2, 2, Epi::Store, false, true, 4>(s, g, ep, 1, (int)g.k);
    return launch_tile<64, 64, 32, 2, 2, Epi::Store, false, true, 2>(s, g, ep, 1, (int)g.k);
}

}  // namespace

// Residual GEMM followed by the LayerNorm of the updated rows: split K and
// fuse the reduction with the normalisation when the shape allows, else run
// the GEMM and a separate LayerNorm.
static hipError_t residual_ln(hipStream_t s, const GemmArgs &g, EpiArgs ep) {
    Tile t;
    int splits;
    if (!tile_override(&t, &splits)) {
        default_tile(g, &t, &splits);
        // The out-projection shape (K <= 1024) splits K at M <= 1024, where its
        // 168 tiles would leave CUs idle (865 tokens: 20.4 us fused against
        // 25.4 unsplit plus LayerNorm); past 1024 rows the tiles fill the GPU
        // and the unsplit GEMM plus a LayerNorm launch is faster (4 x 865
        // tokens: 47.9 against 53.5 us).
        if (splits < 2 && g.m <= 1024) {
            t = Tile{64, 64, 32, 2, 2};
            splits = 3;
        }
    }
    const bool fused = splits >= 2 && splits <= 4 && g.k >= 64 * (size_t)splits && g.n % 4 == 0 && g.n <= 1024 &&
                       g.ws != nullptr && g.ws_floats >= (size_t)splits * g.m * g.n;
    if (!fused) {
        hipError_t e = dispatch<Epi::Residual>(s, g, ep);
        if (e != hipSuccess) return e;
        return launch_layernorm(s, g.c, g.ln_gamma, g.ln_beta, g.ln_out, g.m, g.n, g.ln_eps);
    }
    ep.partial = g.ws;
    hipError_t e = run_cfg<Epi::Residual, true>(s, g, ep, t, splits);
    if (e == hipErrorInvalidValue) {
        t = Tile{64, 64, 32, 2, 2};
        e = run_cfg<Epi::Residual, true>(s, g, ep, t, splits);
    }
    if (e != hipSuccess) return e;
    // One wave per row; up to 2048 rows, one row per workgroup spreads the
    // rows over every CU.
    const unsigned wpb = g.m <= 2048 ? 1 : 4;
    const dim3 grid((unsigned)((g.m + wpb - 1) / wpb));
    const int m = (int)g.m, n = (int)g.n, nt = (int)(64 * wpb);
    switch (splits) {
        case 2: splitk_residual_ln_kernel<2><<<grid, nt, 0, s>>>(m, n, ep, g.ln_gamma, g.ln_beta, g.ln_out, g.ln_eps); break;
        case 3: splitk_residual_ln_kernel<3><<<grid, nt, 0, s>>>(m, n, ep, g.ln_gamma, g.ln_beta, g.ln_out, g.ln_eps); break;
        default: splitk_residual_ln_kernel<4><<<grid, nt, 0, s>>>(m, n, ep, g.ln_gamma, g.ln_beta, g.ln_out, g.ln_eps); break;
    }
    return hipGetLastError();
}

hipError_t launch_gemm(hipStream_t s, const GemmArgs &g) {
    if (g.m == 0 || g.n == 0) return hipSuccess;
    EpiArgs ep{};
    ep.c = g.c;
    ep.bias = g.bias;
    ep.gamma = g.gamma;
    ep.q = g.q;
    ep.k = g.k_out;
    ep.v = g.v;
    ep.tokens = (int)g.tokens;
    ep.heads = (int)g.heads;
    ep.rot = g.rot;
    ep.ln_c = g.ln_fold_c;
    ep.ln_eps = g.ln_fold_eps;
    if (g.conv_in_c && g.conv_ih) {
        if (g.epi != Epi::Store || g.conv_kw == 0 || g.conv_ow == 0 || g.conv_iw == 0 ||
            g.conv_stride == 0 || g.n % g.conv_ow != 0 || g.k % (g.conv_in_c * g.conv_kw) != 0)
            return hipErrorInvalidValue;
        ep.conv_in_c = (int)g.conv_in_c;
        ep.conv_kw = (int)g.conv_kw;
        ep.conv_ow = (int)g.conv_ow;
        ep.conv_plane = g.n;
        ep.cd_ih = (int)g.conv_ih;
        ep.cd_iw = (int)g.conv_iw;
        ep.cd_stride = (int)g.conv_stride;
        ep.cd_pad = (int)g.conv_pad;
        ep.cd_relu = g.conv_relu ? 1 : 0;
        return dispatch_conv_direct(s, g, ep);
    }
    if (g.conv_in_c) {
        if (g.epi != Epi::Store) return hipErrorInvalidValue;
        if (g.conv_ow == 0 || g.conv_ow > g.conv_wp || g.n % g.conv_wp != 0)
            return hipErrorInvalidValue;
        ep.conv_in_c = (int)g.conv_in_c;
        ep.conv_kw = (int)g.conv_kw;
        ep.conv_wp = (int)g.conv_wp;
        ep.conv_ow = (int)g.conv_ow;
        ep.conv_plane = g.n / g.conv_wp * g.conv_ow;
        return dispatch_conv(s, g, ep);
    }
    if (g.scatter_kw) {
        if (g.epi != Epi::Store || g.scatter_kh == 0 || g.scatter_iw == 0 ||
            g.m % (g.scatter_kh * g.scatter_kw) != 0 || g.n % g.scatter_iw != 0)
            return hipErrorInvalidValue;
        ep.scat_kh = (int)g.scatter_kh;
        ep.scat_kw = (int)g.scatter_kw;
        ep.scat_iw = (int)g.scatter_iw;
        if (g.scatter_chw) {
            // The direct loader as a 1 x 1 convolution over the CHW input:
            // column n is input pixel (n / iw, n % iw), channel k its row.
            ep.conv_in_c = (int)g.k;
            ep.conv_kw = 1;
            ep.conv_ow = (int)g.scatter_iw;
            ep.cd_ih = (int)(g.n / g.scatter_iw);
            ep.cd_iw = (int)g.scatter_iw;
            ep.cd_stride = 1;
            ep.cd_pad = 0;
            ep.cd_relu = 0;
        }
        return dispatch_scatter(s, g, ep);
    }
    switch (g.epi) {
        case Epi::Store: return dispatch<Epi::Store>(s, g, ep);
        case Epi::Gelu: return dispatch<Epi::Gelu>(s, g, ep);
        case Epi::Residual:
            return g.ln_out ? residual_ln(s, g, ep) : dispatch<Epi::Residual>(s, g, ep);
        case Epi::Qkv: return dispatch<Epi::Qkv>(s, g, ep);
    }
    return hipErrorInvalidValue;
}

}  // namespace vh
