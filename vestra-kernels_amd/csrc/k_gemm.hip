// fp32-MFMA projection GEMM for gfx950 with fused epilogues.
//
// C[m,n] = sum_k A[m,k] * Bt[n,k]; A is the activation (row-major), Bt the
// weight prepared once in [out, in] order so both operands stream k-contiguous
// rows.  A 256-thread workgroup (4 wave64s) owns a BM x BN tile; BK = 32
// slices of A and Bt are double-buffered in LDS with rows padded to 36 floats
// (16-byte fragment reads of 16 consecutive rows then touch 64 distinct
// banks).  Each wave computes a (BM/WM) x (BN/WN) sub-tile with
// v_mfma_f32_16x16x4_f32: one ds_read_b128 per 16-row fragment feeds four
// MFMA k-steps (lane group h supplies k = kk+4h+s at step s).
//
// Epilogues (all separately rounded, as the reference's):
//   Store    : c = (acc + bias) * gamma          (CudaLinearF32::run)
//   Gelu     : c = gelu(acc + bias)              (fc1, Kernels::gelu forms)
//   Residual : c = c + (acc + bias) * gamma      (out-proj / fc2 + residual)
//   Qkv      : head-major Q/K/V with bias and the 2-D RoPE rotation of Q, K
#include "common.h"
#include "kernels.h"

namespace vh {
namespace {

constexpr int BK = 32;
constexpr int LDK = BK + 4;

struct EpiArgs {
    float *c;
    const float *bias;
    const float *gamma;
    float *q, *k, *v;
    int tokens, heads;
    const float *rot;
    size_t tail_start;
};

template <int BM, int BN, int WM, int WN, Epi EPI>
__global__ __launch_bounds__(256) void gemm_nt_kernel(const float *__restrict__ A,
                                                      const float *__restrict__ Bt, int M, int N,
                                                      int K, EpiArgs ep) {
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 16, FN = TN / 16;
    constexpr int ACH = BM * BK / 4 / 256;
    constexpr int BCH = BN * BK / 4 / 256;
    static_assert(WM * WN == 4, "four waves");
    static_assert(ACH >= 1 && BCH >= 1, "tile too small for 256 threads");
    static_assert(EPI != Epi::Qkv || TN == 64, "QKV epilogue needs one head per wave tile");

    __shared__ __attribute__((aligned(16))) float As[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) float Bs[2][BN * LDK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lh = lane >> 4;
    const int wm = wave / WN, wn = wave % WN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const bool vec = (K & 3) == 0;

    f32x4 ra[ACH], rb[BCH];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            int c = tid + i * 256, row = c >> 3, kq = (c & 7) * 4;
            int gm = m0 + row, gk = k0 + kq;
            const float *p = A + (size_t)gm * K + gk;
            if (vec && gm < M && gk < K) {
                ra[i] = *reinterpret_cast<const f32x4 *>(p);
            } else {
                f32x4 t;
#pragma unroll
                for (int e = 0; e < 4; e++) t[e] = (gm < M && gk + e < K) ? p[e] : 0.0f;
                ra[i] = t;
            }
        }
#pragma unroll
        for (int i = 0; i < BCH; i++) {
            int c = tid + i * 256, row = c >> 3, kq = (c & 7) * 4;
            int gn = n0 + row, gk = k0 + kq;
            const float *p = Bt + (size_t)gn * K + gk;
            if (vec && gn < N && gk < K) {
                rb[i] = *reinterpret_cast<const f32x4 *>(p);
            } else {
                f32x4 t;
#pragma unroll
                for (int e = 0; e < 4; e++) t[e] = (gn < N && gk + e < K) ? p[e] : 0.0f;
                rb[i] = t;
            }
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            int c = tid + i * 256, row = c >> 3, kq = (c & 7) * 4;
            *reinterpret_cast<f32x4 *>(&As[buf][row * LDK + kq]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < BCH; i++) {
            int c = tid + i * 256, row = c >> 3, kq = (c & 7) * 4;
            *reinterpret_cast<f32x4 *>(&Bs[buf][row * LDK + kq]) = rb[i];
        }
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](int buf) {
        const float *as = As[buf];
        const float *bs = Bs[buf];
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            f32x4 a[FM], b[FN];
#pragma unroll
            for (int i = 0; i < FM; i++)
                a[i] = *reinterpret_cast<const f32x4 *>(
                    &as[(wm * TM + i * 16 + li) * LDK + kk + 4 * lh]);
#pragma unroll
            for (int j = 0; j < FN; j++)
                b[j] = *reinterpret_cast<const f32x4 *>(
                    &bs[(wn * TN + j * 16 + li) * LDK + kk + 4 * lh]);
#pragma unroll
            for (int s = 0; s < 4; s++)
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++) acc[i][j] = mfma16x16x4(a[i][s], b[j][s], acc[i][j]);
        }
    };

    const int ktiles = (K + BK - 1) / BK;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int t = 0; t < ktiles; t++) {
        const int cur = t & 1;
        const bool next = t + 1 < ktiles;
        if (next) gload((t + 1) * BK);
        compute(cur);
        if (next) lstore(cur ^ 1);
        __syncthreads();
    }

    // C fragment layout: register r of lane l holds row 4*(l/16)+r, column l%16.
    const int rbase = m0 + wm * TM + 4 * lh;
    if constexpr (EPI == Epi::Qkv) {
        const int colw = n0 + wn * TN;  // first column of this wave's head
        if (colw >= N) return;
        const int per = ep.heads * 64;
        const int group = colw / per, head = (colw % per) / 64;
        float *dst = group == 0 ? ep.q : (group == 1 ? ep.k : ep.v);
        const bool rope = ep.rot != nullptr && group < 2;
        float bias[FN];
#pragma unroll
        for (int j = 0; j < FN; j++) bias[j] = ep.bias[colw + j * 16 + li];
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = rbase + i * 16 + r;
                if (row >= M) continue;
                const int img = row / ep.tokens, t = row % ep.tokens;
                float vals[FN];
#pragma unroll
                for (int j = 0; j < FN; j++) vals[j] = add_rn(acc[i][j][r], bias[j]);
                if (rope) {
                    // rope::rotate_half (src/rope.rs:84-93): dims (i, i+16) of
                    // each 32-wide axis half sit in fragments (2a, 2a+1).
#pragma unroll
                    for (int axis = 0; axis < 2; axis++) {
                        const float *rr = ep.rot + (((size_t)t * 2 + axis) * 16 + li) * 2;
                        const float sn = rr[0], cs = rr[1];
                        const float a = vals[2 * axis], b = vals[2 * axis + 1];
                        vals[2 * axis] = sub_rn(mul_rn(a, cs), mul_rn(b, sn));
                        vals[2 * axis + 1] = add_rn(mul_rn(b, cs), mul_rn(a, sn));
                    }
                }
                float *orow = dst + (((size_t)img * ep.heads + head) * ep.tokens + t) * 64;
#pragma unroll
                for (int j = 0; j < FN; j++) orow[j * 16 + li] = vals[j];
            }
    } else {
        const int cbase = n0 + wn * TN + li;
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int col = cbase + j * 16;
            if (col >= N) continue;
            const float b = ep.bias ? ep.bias[col] : 0.0f;
            const float g = ep.gamma ? ep.gamma[col] : 1.0f;
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = rbase + i * 16 + r;
                    if (row >= M) continue;
                    const size_t idx = (size_t)row * N + col;
                    float v = acc[i][j][r];
                    if (ep.bias) v = add_rn(v, b);
                    if constexpr (EPI == Epi::Store) {
                        if (ep.gamma) v = mul_rn(v, g);
                        ep.c[idx] = v;
                    } else if constexpr (EPI == Epi::Gelu) {
                        ep.c[idx] = idx < ep.tail_start ? gelu_avx512_form(v) : gelu_scalar_form(v);
                    } else {
                        if (ep.gamma) v = mul_rn(v, g);
                        ep.c[idx] = add_rn(ep.c[idx], v);
                    }
                }
        }
    }
}

template <int BM, int BN, int WM, int WN, Epi EPI>
hipError_t run(hipStream_t s, const GemmArgs &g, const EpiArgs &ep) {
    dim3 grid((unsigned)((g.n + BN - 1) / BN), (unsigned)((g.m + BM - 1) / BM));
    gemm_nt_kernel<BM, BN, WM, WN, EPI>
        <<<grid, 256, 0, s>>>(g.a, g.bt, (int)g.m, (int)g.n, (int)g.k, ep);
    return hipGetLastError();
}

template <Epi EPI>
hipError_t dispatch(hipStream_t s, const GemmArgs &g, const EpiArgs &ep) {
    if (g.n >= 2048) return run<64, 128, 2, 2, EPI>(s, g, ep);
    return run<64, 64, 2, 2, EPI>(s, g, ep);
}

}  // namespace

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
    size_t total = g.m * g.n;
    ep.tail_start = total - total % 16;
    switch (g.epi) {
        case Epi::Store: return dispatch<Epi::Store>(s, g, ep);
        case Epi::Gelu: return dispatch<Epi::Gelu>(s, g, ep);
        case Epi::Residual: return dispatch<Epi::Residual>(s, g, ep);
        case Epi::Qkv: return run<64, 128, 2, 2, Epi::Qkv>(s, g, ep);
    }
    return hipErrorInvalidValue;
}

}  // namespace vh
