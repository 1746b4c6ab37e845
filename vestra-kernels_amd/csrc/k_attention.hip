// Online-softmax attention for gfx950.
//
// flash_kernel: DA3 head_dim 64, scale 1/8, fp32 MFMA.  A workgroup of four
// wave64s owns 64 queries of one (image, head); wave w owns queries
// q0+16w..q0+16w+15.  Key/value panels of 64 keys stream through LDS
// (double-buffered; K rows padded to 68 floats, V stored transposed and
// swizzled).  Per panel each wave computes
//     S^T[key][query] = K[key][:] . Q[query][:]     (v_mfma_f32_16x16x4_f32)
// so that register r of lane l holds key 16g+4(l/16)+r of query l%16 --
// exactly the B-operand layout of the second contraction
//     O^T[d][query] += V^T[d][key] . P^T[key][query]
// and no register transpose or LDS round trip of P is needed.  The running
// max and sum live in registers; a query's 64 keys are spread over the four
// 16-lane groups, so the max takes two cross-group shuffles per panel and
// the sum is reduced once at the end.  Exponentials run in base 2 with the
// 1/8 * log2(e) scale folded into one multiply.
//
// flash_direct_kernel: the same work split for one key stream per
// workgroup, with K/V panels copied straight from global memory into LDS
// and V kept row-major (P is the A operand of the second contraction); it
// is the default for one-stream layouts, flash_kernel serves two-stream
// layouts.
//
// Head dims below 64 (the generic online-attention contract of
// src/cuda.rs:868-922) run through the same MFMA kernel: pad_rows64_kernel
// widens Q, K and V rows to 64 with zeros (the zero dims add nothing to a
// score and give zero output columns), the softmax takes a runtime scale of
// 1/sqrt(head_dim), and unpad_rows_kernel keeps the first head_dim columns.
#include <algorithm>
#include <cstdlib>

#include "common.h"
#include "kernels.h"

namespace vh {
namespace {

constexpr int D = 64;
constexpr int BQ = 64;
constexpr int BKV = 64;
constexpr int LDP = D + 4;  // padded LDS row of a K/V panel
constexpr float kLog2e = 1.4426950408889634f;

struct FlashArgs {
    const float *q, *k, *v;
    float *out;
    int T, heads, bh, qtiles;
    int xcd_map;  // 1: place all q-tiles of a head on one XCD's L2
    // Key split across workgroups: split z takes keys [z*split_keys, ...).
    int splits, split_keys;
    float scale_log2;  // softmax scale times log2(e): 1/8 * log2(e) for DA3
    float *po;    // [splits][bh][T][64] unnormalised outputs
    float2 *pml;  // [splits][bh][T] (running max in the base-2 domain, sum)
    // Token-major split runs only: when q8_qs is set, the merge writes the
    // output rows as block-major Q8_0 (quantize_row_q8_0) instead of f32.
    int8_t *q8_qs;
    uint16_t *q8_d;
    // Fused merge (flash_direct_kernel<.., FUSED>): the splits of query
    // group g = bh * qtiles + qt publish thread-major partials at
    // pt + (g * splits + z) * kFusedPartial (16 output values per thread,
    // then m and l of the thread's query), and cnt[g] counts them in; it is
    // zero on entry and the split that merges leaves it zero.
    float *pt;
    unsigned *cnt;
};
constexpr int kFusedValues = 18;  // per thread: o[4][4], m, l
constexpr size_t kFusedPartial = (size_t)kFusedValues * 256;

// Stores the merged output dims d4..d4+3 of query `query` of head-row bh:
// token-major f32, token-major block-major Q8_0 (fa.q8_qs), or head-major
// f32.  For Q8_0 the eight consecutive lanes of a 16-lane row that hold
// one 32-column block take its absmax with three DPP steps, so all eight
// must be active.
template <bool TOKEN_MAJOR>
__device__ __forceinline__ void store_merged(const FlashArgs &fa, int bh, int query, int d4, f32x4 o) {
    float *dst;
    if constexpr (TOKEN_MAJOR) {
        const int img = bh / fa.heads, head = bh % fa.heads;
        if (fa.q8_qs) {
            // Row img*T + query of the token-major [images*T][heads*64]
            // output, quantised as quantize_row_q8_0 does.
            float amax = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; e++) amax = q8_absmax(amax, o[e]);
            amax = q8_absmax(amax, dpp_f32<0xb1>(amax));
            amax = q8_absmax(amax, dpp_f32<0x4e>(amax));
            amax = q8_absmax(amax, dpp_f32<0x141>(amax));
            float d, qinv;
            q8_scale(amax, d, qinv);
            uint32_t w = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float qv = roundf(mul_rn(o[e], qinv));  // f32::round: half away from zero
                int qi;
                if (isnan(qv)) {
                    qi = 0;  // `NaN as i8` saturates to 0
                } else {
                    qv = fminf(fmaxf(qv, -127.0f), 127.0f);
                    qi = (int)qv;
                }
                w |= ((uint32_t)(qi & 0xff)) << (8 * e);
            }
            const size_t M = (size_t)(fa.bh / fa.heads) * fa.T;
            const size_t slot = (size_t)(head * 2 + (d4 >> 5)) * M + (size_t)img * fa.T + query;
            reinterpret_cast<uint32_t *>(fa.q8_qs + slot * 32)[(d4 & 31) >> 2] = w;
            if ((d4 & 31) == 0) fa.q8_d[slot] = __builtin_bit_cast(uint16_t, (_Float16)d);
            return;
        }
        dst = fa.out + ((size_t)img * fa.T + query) * ((size_t)fa.heads * D) + (size_t)head * D;
    } else {
        dst = fa.out + ((size_t)bh * fa.T + query) * D;
    }
    *reinterpret_cast<f32x4 *>(dst + d4) = o;
}

// V panels are stored transposed, Vt[d][key], so that the four keys a lane
// feeds to one PV k-step are one 16-byte read.  Key column k of row d sits
// at k ^ vswz(d): the XOR moves whole aligned 4-key groups, and it spreads
// both the transposing stores (a wave writes 16 d-rows x 4 keys) and the
// fragment reads (a 16-lane group reads 16 d-rows) over all 64 banks.
__device__ __forceinline__ int vswz(int d) { return 4 * ((d & 15) ^ ((d >> 2) & 15)); }

// KVS key-panel streams per workgroup: waves [s*4, s*4+4) take the panels
// p = s (mod KVS) for the same 64 queries, so a SIMD runs KVS waves whose
// MFMA and softmax phases overlap; the streams merge through LDS at the end.
// LDS holds one workgroup per CU at KVS = 2 (two at KVS = 1), i.e. two waves
// per SIMD either way; telling the compiler so lets it keep a panel's
// fragments in registers instead of trading latency for occupancy.
//
// SPLIT: the workgroup covers only the keys of split z and writes its
// unnormalised output and (max, sum) for flash_merge_kernel.
template <bool TOKEN_MAJOR, int KVS, bool SPLIT>
__global__ __launch_bounds__(256 * KVS) __attribute__((amdgpu_waves_per_eu(1, 2))) void flash_kernel(
    FlashArgs fa) {
    constexpr int NT = 256 * KVS;
    constexpr int KSTAGE = KVS * BKV * LDP;  // floats of one K stage
    constexpr int VSTAGE = KVS * D * BKV;    // floats of one V^T stage
    extern __shared__ __attribute__((aligned(16))) float smem[];
    float *Ks = smem;               // [2][KVS][BKV*LDP]
    float *Vs = smem + 2 * KSTAGE;  // [2][KVS][D*BKV], transposed and swizzled

    // Hardware deals workgroups round-robin over the 8 XCDs; with xcd_map the
    // items are renumbered so that the q-tiles (and key splits) of one head
    // share an XCD.
    const int splits = SPLIT ? fa.splits : 1;
    const int total = fa.bh * fa.qtiles * splits;
    int item = blockIdx.x;
    if (fa.xcd_map) {
        const int per_xcd = (total + 7) / 8;
        item = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
        if (item >= total) return;
    }
    const int z = item % splits;
    const int qt = (item / splits) % fa.qtiles;
    const int bh = item / splits / fa.qtiles;
    const int T = fa.T;
    // This workgroup's keys [kb, ke).
    const int kb = SPLIT ? z * fa.split_keys : 0;
    const int ke = SPLIT ? min(T, kb + fa.split_keys) : T;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lh = lane >> 4;
    const int qgroup = wave & 3, stream = wave >> 2;
    const int q0 = qt * BQ;
    const size_t head_off = (size_t)bh * T * D;
    const float *Qh = fa.q + head_off;
    const float *Kh = fa.k + head_off;
    const float *Vh = fa.v + head_off;

    // This lane's query (column of S^T) and its Q fragment for all 64 dims:
    // qf[c][s] = Q[query][16c + 4*lh + s].
    const int query = q0 + qgroup * 16 + li;
    f32x4 qf[4];
#pragma unroll
    for (int c = 0; c < 4; c++)
        qf[c] = query < T ? *reinterpret_cast<const f32x4 *>(Qh + (size_t)query * D + 16 * c + 4 * lh)
                          : f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // One step stages KVS consecutive panels: KVS x 64 keys x 16 float4.
    // Keys past T load the last key's row (no branch, no select on the
    // loaded value, so the loads stay in flight across the MFMAs); their
    // scores are masked to -inf and their V rows are zeroed when stored.
    constexpr int CH = KVS * BKV * 16 / NT;  // float4 chunks per thread (= 4)
    f32x4 rk[CH], rv[CH];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int c = tid + i * NT, key = c >> 4, d4 = (c & 15) * 4;
            const size_t row = (size_t)min(k0 + key, ke - 1) * D + d4;
            rk[i] = *reinterpret_cast<const f32x4 *>(Kh + row);
            rv[i] = *reinterpret_cast<const f32x4 *>(Vh + row);
        }
    };
    auto lstore = [&](int buf, int k0) {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int c = tid + i * NT, key = c >> 4, d4 = (c & 15) * 4;
            *reinterpret_cast<f32x4 *>(&Ks[buf * KSTAGE + key * LDP + d4]) = rk[i];
            // Rows past T become +0 through an all-zero bit mask (a select
            // here is turned into a branch around one of the stores).
            const unsigned keep = k0 + key < ke ? 0xffffffffu : 0u;
            float *vt = Vs + buf * VSTAGE + (key / BKV) * D * BKV;
            const int kin = key % BKV;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int d = d4 + e;
                vt[d * BKV + (kin ^ vswz(d))] = __uint_as_float(__float_as_uint(rv[i][e]) & keep);
            }
        }
    };

    const float scale = fa.scale_log2;
    float m = -INFINITY;  // running max (base-2 domain) of this lane's query
    float l = 0.0f;       // partial running sum over this lane's keys
    f32x4 o[4];           // o[df][r] = O[query][16*df + 4*lh + r] (unnormalised)
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    int vcol[4];          // swizzle of this lane's V^T rows 16*df + li
#pragma unroll
    for (int df = 0; df < 4; df++) vcol[df] = vswz(16 * df + li);

    const int steps = (ke - kb + KVS * BKV - 1) / (KVS * BKV);
    gload(kb);
    lstore(0, kb);
    __syncthreads();
    // Branch-free step loop: the last step reloads its own keys into the idle
    // buffer, which is never read again.
    for (int step = 0; step < steps; step++) {
        const int cur = step & 1;
        const int k0 = kb + step * KVS * BKV + stream * BKV;  // this stream's panel
        const int kn = kb + min(step + 1, steps - 1) * KVS * BKV;
        gload(kn);

        // All K and V fragments of the panel are read up front; the MFMAs
        // consume them in issue order.
        const float *ks = Ks + cur * KSTAGE + stream * BKV * LDP + li * LDP + 4 * lh;
        const float *vt = Vs + cur * VSTAGE + stream * D * BKV;
        f32x4 kf[4][4], vf[4][4];
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                kf[g][c] = *reinterpret_cast<const f32x4 *>(&ks[16 * g * LDP + 16 * c]);
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
            for (int df = 0; df < 4; df++)
                vf[g][df] = *reinterpret_cast<const f32x4 *>(
                    &vt[(16 * df + li) * BKV + ((16 * g + 4 * lh) ^ vcol[df])]);

        // S^T fragments: s[g][r] = S[key 16g+4lh+r][query li].  The four key
        // groups are independent accumulation chains; interleaving them keeps
        // consecutive MFMAs independent (each chain's order is unchanged).
        f32x4 s[4];
#pragma unroll
        for (int g = 0; g < 4; g++) s[g] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int st = 0; st < 4; st++)
#pragma unroll
                for (int g = 0; g < 4; g++) s[g] = mfma16x16x4(kf[g][c][st], qf[c][st], s[g]);
        // Issue order of this region: the K fragments, the next step's global
        // loads, then the QK MFMAs with one V fragment read after every four.
        __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, 2 * CH, 0);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        // Online softmax for this lane's query over its 16 keys of the panel.
        float mx = -INFINITY;
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int key = k0 + 16 * g + 4 * lh + r;
                float t = key < ke ? s[g][r] * scale : -INFINITY;
                s[g][r] = t;
                mx = fmaxf(mx, t);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mnew = fmaxf(m, mx);
        // A stream whose panels so far hold no valid key keeps m = -inf; use
        // 0 as the reference so exp2 sees -inf (giving 0), never NaN.
        const float mref = mnew == -INFINITY ? 0.0f : mnew;
        const float corr = __builtin_amdgcn_exp2f(m - mref);
        float psum = 0.0f;
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float pv = __builtin_amdgcn_exp2f(s[g][r] - mref);
                s[g][r] = pv;
                psum += pv;
            }
        l = l * corr + psum;
        m = mnew;
#pragma unroll
        for (int df = 0; df < 4; df++) o[df] *= corr;
        __builtin_amdgcn_sched_barrier(0);
        // O^T[d][query] += V^T[d][key] P^T[key][query]: lane supplies
        // V[16g+4lh+st][16df+li] (A, from vf) and s[g][st] (B).
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
            for (int st = 0; st < 4; st++)
#pragma unroll
                for (int df = 0; df < 4; df++) o[df] = mfma16x16x4(vf[g][df][st], s[g][st], o[df]);

        lstore(cur ^ 1, kn);
        // The next stage's LDS stores (4 K + 16 transposed V per thread) go
        // out between the PV MFMAs.
#pragma unroll
        for (int i = 0; i < 5 * CH; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 64 - 15 * CH, 0);
        __syncthreads();
    }

    if constexpr (KVS > 1) {
        // Streams 1.. publish (m, l, o) through LDS; stream 0 merges them in
        // stream order.  The staging buffers are free after the last barrier.
        constexpr int REC = 18;  // m, l, 16 outputs per lane
        float *xbuf = smem;
        if (stream > 0) {
            float *rec = xbuf + (((stream - 1) * 4 + qgroup) * 64 + lane) * REC;
            rec[0] = m;
            rec[1] = l;
#pragma unroll
            for (int df = 0; df < 4; df++)
#pragma unroll
                for (int r = 0; r < 4; r++) rec[2 + 4 * df + r] = o[df][r];
        }
        __syncthreads();
        if (stream > 0) return;
        float mm = m;
#pragma unroll
        for (int sidx = 1; sidx < KVS; sidx++)
            mm = fmaxf(mm, xbuf[(((sidx - 1) * 4 + qgroup) * 64 + lane) * REC]);
        const float w0 = __builtin_amdgcn_exp2f(m - mm);
        l *= w0;
#pragma unroll
        for (int df = 0; df < 4; df++) o[df] *= w0;
#pragma unroll
        for (int sidx = 1; sidx < KVS; sidx++) {
            const float *rec = xbuf + (((sidx - 1) * 4 + qgroup) * 64 + lane) * REC;
            const float w = __builtin_amdgcn_exp2f(rec[0] - mm);
            l += w * rec[1];
#pragma unroll
            for (int df = 0; df < 4; df++)
#pragma unroll
                for (int r = 0; r < 4; r++) o[df][r] += w * rec[2 + 4 * df + r];
        }
    }

    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (query >= T) return;
    if constexpr (SPLIT) {
        const size_t prow = ((size_t)z * fa.bh + bh) * T + query;
        float *orow = fa.po + prow * D;
#pragma unroll
        for (int df = 0; df < 4; df++) *reinterpret_cast<f32x4 *>(orow + 16 * df + 4 * lh) = o[df];
        if (lh == 0) fa.pml[prow] = make_float2(m, l);
        return;
    }
    const float inv = 1.0f / l;
    float *orow;
    if constexpr (TOKEN_MAJOR) {
        const int img = bh / fa.heads, head = bh % fa.heads;
        orow = fa.out + ((size_t)img * T + query) * ((size_t)fa.heads * D) + (size_t)head * D;
    } else {
        orow = fa.out + head_off + (size_t)query * D;
    }
#pragma unroll
    for (int df = 0; df < 4; df++)
        *reinterpret_cast<f32x4 *>(orow + 16 * df + 4 * lh) = o[df] * inv;
}

// Direct-to-LDS form for one key stream per workgroup (two workgroups per
// CU).  Panels of K and V go from global memory straight into LDS with
// global_load_lds_dwordx4 (no register staging, no LDS stores): instruction
// i of wave w copies keys 4c..4c+3 (c = 4i + w), lane L writing the 16-byte
// granule L%16 of key 4c + L/16.  The wave picks which global granule each
// lane fetches, so K is XOR-swizzled on the way in (global granule g of key
// r lands at granule g ^ (r & 15)) and a 16-lane group reading one granule
// column of 16 keys hits 16 distinct bank groups.
//
// V stays row-major, because the second contraction takes P as the A
// operand and V as B:
//     O[query][d] += P[query][key] . V[key][d]   (d = 4*li + df for output
//                                                 fragment df of lane li)
// The score registers of S^T = K.Q^T already hold P[query li][keys
// 16g+4lh+r], i.e. the A operand of k-step (g, r); lane (li, lh) feeds B
// with V[16g+4lh+r][4li+df] for df = 0..3 -- one 16-byte read per k-step
// serving four MFMAs.  The output fragment of lane (li, lh) then holds
// queries 4lh+r, whose softmax corrections live in lanes 4lh+r: four lane
// shuffles per panel carry them over.
//
// Per panel: one barrier (after which the panel's copies, issued one panel
// earlier, have landed and every wave is done with the buffer being
// refilled), the 16 K fragment reads, the copies of the next panel, then
// the QK MFMAs with one V fragment read after every four, the softmax, and
// the PV MFMAs.
using lds_ptr = __attribute__((address_space(3))) void *;
using global_ptr = __attribute__((address_space(1))) void *;
constexpr int PANEL = BKV * D;  // floats of one K or V panel (16 KB)

// Each lane copies the 16 bytes at src to lds_wave + 16 * lane.
__device__ __forceinline__ void copy_to_lds16(const float *src, float *lds_wave) {
    __builtin_amdgcn_global_load_lds((global_ptr)src, (lds_ptr)lds_wave, 16, 0, 0);
}

// max(v, value of the lane 16 (32) away) on the VALU: gfx950's
// v_permlane16_swap (v_permlane32_swap) of two copies of v leaves v in one
// and the partner lane's v in the other (in either order, and fmaxf does not
// depend on the order), without the LDS round trip of a shuffle.  Written
// out because the compiler's builtins for these instructions, given a value
// and its own copy, used one result twice; s_nop 1 on each side covers the
// VALU-write / permlane hazards.
__device__ __forceinline__ float max_xor16(float v) {
    float a = v, b = v;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return fmaxf(a, b);
}
__device__ __forceinline__ float max_xor32(float v) {
    float a = v, b = v;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return fmaxf(a, b);
}

// FUSED (with SPLIT): the split that finishes last in its query group
// merges the group's partials itself (flash_merge_kernel's arithmetic and
// order), so no merge launch follows.
template <bool TOKEN_MAJOR, bool SPLIT, bool FUSED = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void flash_direct_kernel(
    FlashArgs fa) {
    static_assert(SPLIT || !FUSED, "the fused merge is for key splits");
    extern __shared__ __attribute__((aligned(16))) float smem[];
    float *Ks = smem;              // [2][64 keys][64], swizzled granules
    float *Vs = smem + 2 * PANEL;  // [2][64 keys][64]

    const int splits = SPLIT ? fa.splits : 1;
    const int total = fa.bh * fa.qtiles * splits;
    int item = blockIdx.x;
    if (fa.xcd_map) {
        const int per_xcd = (total + 7) / 8;
        item = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
        if (item >= total) return;
    }
    const int z = item % splits;
    const int qt = (item / splits) % fa.qtiles;
    const int bh = item / splits / fa.qtiles;
    const int T = fa.T;
    const int kb = SPLIT ? z * fa.split_keys : 0;
    const int ke = SPLIT ? min(T, kb + fa.split_keys) : T;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lh = lane >> 4;
    const size_t head_off = (size_t)bh * T * D;
    const float *Qh = fa.q + head_off;
    const float *Kh = fa.k + head_off;
    const float *Vh = fa.v + head_off;
    const int qw = qt * BQ + wave * 16;  // this wave's first query
    const int query = qw + li;
    f32x4 qf[4];
#pragma unroll
    for (int c = 0; c < 4; c++)
        qf[c] = query < T ? *reinterpret_cast<const f32x4 *>(Qh + (size_t)query * D + 16 * c + 4 * lh)
                          : f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Keys past ke copy key ke - 1: finite values whose scores are masked.
    auto copy_panel = [&](int buf, int k0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = 4 * i + wave;
            const int key = 4 * c + lh;
            const size_t row = (size_t)min(k0 + key, ke - 1) * D;
            copy_to_lds16(Kh + row + 4 * (li ^ (key & 15)), Ks + buf * PANEL + c * 256);
            copy_to_lds16(Vh + row + 4 * li, Vs + buf * PANEL + c * 256);
        }
    };

    const float scale = fa.scale_log2;
    float m = -INFINITY;  // running max (base 2) of query li
    float l = 0.0f;       // partial running sum over this lane's keys
    f32x4 o[4];           // o[df][r] = O[query qw + 4lh + r][4li + df] (unnormalised)
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int n = (ke - kb + BKV - 1) / BKV;  // panels, >= 1
    copy_panel(0, kb);
    for (int j = 0; j < n; j++) {
        const int buf = j & 1;
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's copies of panel j
        __syncthreads();
        const float *ks = Ks + buf * PANEL;
        const float *vs = Vs + buf * PANEL + (4 * lh) * D + 4 * li;
        f32x4 kf[4][4], vf[4][4];  // kf[g][c] = K[16g + li][16c + 4lh ..]
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                kf[g][c] = *reinterpret_cast<const f32x4 *>(&ks[(16 * g + li) * D + 4 * ((4 * c + lh) ^ li)]);
        if (j + 1 < n) copy_panel(buf ^ 1, kb + (j + 1) * BKV);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
            for (int st = 0; st < 4; st++)
                vf[g][st] = *reinterpret_cast<const f32x4 *>(&vs[(16 * g + st) * D]);
        // S^T fragments: s[g][r] = S[key 16g+4lh+r][query li].
        f32x4 s[4];
#pragma unroll
        for (int g = 0; g < 4; g++) s[g] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int st = 0; st < 4; st++)
#pragma unroll
                for (int g = 0; g < 4; g++) s[g] = mfma16x16x4(kf[g][c][st], qf[c][st], s[g]);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_s_setprio(1);
        __builtin_amdgcn_sched_barrier(0);
        // The softmax runs at raised wave priority: it is the chain between
        // this wave's two contractions, and the SIMD's other wave keeps the
        // matrix core busy meanwhile (attention at 865 tokens 31.7 -> 31.0
        // us; priority over the QK MFMAs instead, or over the fragment reads
        // as well, took 33.3 us).
        // Online softmax of query li over its 16 keys of the panel.  The max
        // is taken on the raw scores (the scale is positive) and the scale
        // is folded into the exponent's FMA; full panels need no mask.
        const int k0 = kb + j * BKV;
        float mx = -INFINITY;
        if (k0 + BKV <= ke) {
#pragma unroll
            for (int g = 0; g < 4; g++)
                mx = fmaxf(mx, fmaxf(fmaxf(s[g][0], s[g][1]), fmaxf(s[g][2], s[g][3])));
        } else {
#pragma unroll
            for (int g = 0; g < 4; g++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int key = k0 + 16 * g + 4 * lh + r;
                    s[g][r] = key < ke ? s[g][r] : -INFINITY;
                    mx = fmaxf(mx, s[g][r]);
                }
        }
        mx = max_xor32(max_xor16(mx));
        const float mnew = fmaxf(m, mx * scale);
        // A range with no valid key yet keeps m = -inf; 0 as the reference
        // makes exp2 see -inf (giving 0), never NaN.
        const float mref = mnew == -INFINITY ? 0.0f : mnew;
        const float corr = __builtin_amdgcn_exp2f(m - mref);
        float psum = 0.0f;
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[g][r], scale, -mref));
                s[g][r] = p;
                psum += p;
            }
        l = l * corr + psum;
        m = mnew;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float cr = __shfl(corr, 4 * lh + r, 64);
#pragma unroll
            for (int df = 0; df < 4; df++) o[df][r] *= cr;
        }
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
        // O[q][4li + df] += P[q][key] V[key][4li + df], key = 16g + 4lh + st.
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
            for (int st = 0; st < 4; st++)
#pragma unroll
                for (int df = 0; df < 4; df++) o[df] = mfma16x16x4(s[g][st], vf[g][st][df], o[df]);
    }

    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if constexpr (FUSED) {
        // Publish this split's partial thread-major (each store instruction
        // writes 256 consecutive bytes per wave), then count it in; the
        // split that sees the last count merges.  Ordering as in the GEMM's
        // balanced tail: agent-scope atomic stores write through the XCD's
        // L2 to where every XCD reads; each thread waits for its stores'
        // acknowledgement (vmcnt counts stores; inline asm with a memory
        // clobber, so no store moves past it); the barrier orders those
        // waits before thread 0's agent-scope increment; the merging split
        // reads with agent-scope atomic loads, which bypass the L2.  No
        // split waits for another, so the grid drains at any residency.
        const int group = bh * fa.qtiles + qt;
        const float *grp = fa.pt + (size_t)group * fa.splits * kFusedPartial + tid;
        float *mine = fa.pt + ((size_t)group * fa.splits + z) * kFusedPartial + tid;
#pragma unroll
        for (int df = 0; df < 4; df++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                __hip_atomic_store(mine + (df * 4 + r) * 256, o[df][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(mine + 16 * 256, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(mine + 17 * 256, l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        __shared__ int merge_here;
        if (tid == 0)
            merge_here = __hip_atomic_fetch_add(fa.cnt + group, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                         (unsigned)(fa.splits - 1);
        __syncthreads();
        if (!merge_here) return;
        // Every split's values (this one's too) are loaded before the first
        // use, under a uniform branch per split.
        float pv[kMaxFlashSplits][kFusedValues];
#pragma unroll
        for (int p = 0; p < kMaxFlashSplits; p++) {
#pragma unroll
            for (int e = 0; e < kFusedValues; e++)
                pv[p][e] = p < fa.splits ? __hip_atomic_load(grp + (p * kFusedValues + e) * 256, __ATOMIC_RELAXED,
                                                             __HIP_MEMORY_SCOPE_AGENT)
                                         : 0.0f;
        }
        if (tid == 0) __hip_atomic_store(fa.cnt + group, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // Split weights and inverse sum of this lane's query li, then of
        // each output row (query qw + 4lh + r, held by lane 4lh + r).
        float mm = pv[0][16];
#pragma unroll
        for (int p = 1; p < kMaxFlashSplits; p++)
            if (p < fa.splits) mm = fmaxf(mm, pv[p][16]);
        float w[kMaxFlashSplits], lsum = 0.0f;
#pragma unroll
        for (int p = 0; p < kMaxFlashSplits; p++) {
            w[p] = 0.0f;
            if (p < fa.splits) {
                w[p] = __builtin_amdgcn_exp2f(pv[p][16] - mm);
                lsum += w[p] * pv[p][17];
            }
        }
        const float inv = 1.0f / lsum;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float wr[kMaxFlashSplits];
#pragma unroll
            for (int p = 0; p < kMaxFlashSplits; p++) wr[p] = __shfl(w[p], 4 * lh + r, 64);
            const float ir = __shfl(inv, 4 * lh + r, 64);
            f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int p = 0; p < kMaxFlashSplits; p++)
                if (p < fa.splits) acc += wr[p] * f32x4{pv[p][r], pv[p][4 + r], pv[p][8 + r], pv[p][12 + r]};
            const int qr = qw + 4 * lh + r;
            if (qr < T) store_merged<TOKEN_MAJOR>(fa, bh, qr, 4 * li, acc * ir);
        }
        return;
    }
    // Output row r of this lane is query qw + 4lh + r, whose (m, l) sit in
    // lane 4lh + r.
    float lr[4], mr[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        lr[r] = __shfl(l, 4 * lh + r, 64);
        mr[r] = __shfl(m, 4 * lh + r, 64);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int qr = qw + 4 * lh + r;
        if (qr >= T) continue;
        const f32x4 v = f32x4{o[0][r], o[1][r], o[2][r], o[3][r]};
        if constexpr (SPLIT) {
            const size_t prow = ((size_t)z * fa.bh + bh) * T + qr;
            *reinterpret_cast<f32x4 *>(fa.po + prow * D + 4 * li) = v;
            if (li == 0) fa.pml[prow] = make_float2(mr[r], lr[r]);
        } else {
            float *orow;
            if constexpr (TOKEN_MAJOR) {
                const int img = bh / fa.heads, head = bh % fa.heads;
                orow = fa.out + ((size_t)img * T + qr) * ((size_t)fa.heads * D) + (size_t)head * D;
            } else {
                orow = fa.out + head_off + (size_t)qr * D;
            }
            *reinterpret_cast<f32x4 *>(orow + 4 * li) = v * (1.0f / lr[r]);
        }
    }
}

// Combines the key splits of each (head, query) in split order:
// O = sum_z 2^(m_z - M) o_z / sum_z 2^(m_z - M) l_z with M = max_z m_z.
// One thread per four output dims; all reads are issued first.  The fused
// form inside flash_direct_kernel does the same arithmetic in the same order.
template <bool TOKEN_MAJOR, int S>
__global__ __launch_bounds__(256) void flash_merge_kernel(FlashArgs fa) {
    const size_t rows = (size_t)fa.bh * fa.T;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= rows * 16) return;
    const size_t row = idx >> 4;
    const int d4 = (int)(idx & 15) * 4;
    float2 ml[S];
    f32x4 po[S];
#pragma unroll
    for (int z = 0; z < S; z++) {
        ml[z] = fa.pml[z * rows + row];
        po[z] = *reinterpret_cast<const f32x4 *>(fa.po + (z * rows + row) * D + d4);
    }
    float mm = ml[0].x;
#pragma unroll
    for (int z = 1; z < S; z++) mm = fmaxf(mm, ml[z].x);
    float lsum = 0.0f;
    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int z = 0; z < S; z++) {
        const float w = __builtin_amdgcn_exp2f(ml[z].x - mm);
        lsum += w * ml[z].y;
        acc += w * po[z];
    }
    const float inv = 1.0f / lsum;
    store_merged<TOKEN_MAJOR>(fa, (int)(row / fa.T), (int)(row % fa.T), d4, acc * inv);
}

template <bool TOKEN_MAJOR, int KVS, bool SPLIT>
hipError_t run_flash(hipStream_t s, const FlashArgs &fa) {
    constexpr size_t lds = 2 * (size_t)KVS * (BKV * LDP + D * BKV) * sizeof(float);
    auto kernel = flash_kernel<TOKEN_MAJOR, KVS, SPLIT>;
    static std::atomic<uint64_t> configured{0};
    if (hipError_t e = ensure_dynamic_lds(kernel, lds, configured); e != hipSuccess) return e;
    const int total = fa.bh * fa.qtiles * (SPLIT ? fa.splits : 1);
    const int grid = fa.xcd_map ? (total + 7) / 8 * 8 : total;
    kernel<<<grid, 256 * KVS, lds, s>>>(fa);
    if constexpr (SPLIT) {
        const size_t threads = (size_t)fa.bh * fa.T * 16;
        const dim3 grid((unsigned)((threads + 255) / 256));
        static_assert(kMaxFlashSplits == 4, "merge instantiations");
        if (fa.splits == 2) flash_merge_kernel<TOKEN_MAJOR, 2><<<grid, 256, 0, s>>>(fa);
        else if (fa.splits == 3) flash_merge_kernel<TOKEN_MAJOR, 3><<<grid, 256, 0, s>>>(fa);
        else flash_merge_kernel<TOKEN_MAJOR, 4><<<grid, 256, 0, s>>>(fa);
    }
    return hipGetLastError();
}

template <bool TOKEN_MAJOR, bool SPLIT, bool FUSED = false>
hipError_t run_flash_direct(hipStream_t s, const FlashArgs &fa) {
    constexpr size_t lds = 2 * (size_t)(2 * PANEL) * sizeof(float);
    auto kernel = flash_direct_kernel<TOKEN_MAJOR, SPLIT, FUSED>;
    static std::atomic<uint64_t> configured{0};
    if (hipError_t e = ensure_dynamic_lds(kernel, lds, configured); e != hipSuccess) return e;
    const int total = fa.bh * fa.qtiles * (SPLIT ? fa.splits : 1);
    const int grid = fa.xcd_map ? (total + 7) / 8 * 8 : total;
    kernel<<<grid, 256, lds, s>>>(fa);
    if constexpr (SPLIT && !FUSED) {
        const size_t threads = (size_t)fa.bh * fa.T * 16;
        const dim3 mgrid((unsigned)((threads + 255) / 256));
        if (fa.splits == 2) flash_merge_kernel<TOKEN_MAJOR, 2><<<mgrid, 256, 0, s>>>(fa);
        else if (fa.splits == 3) flash_merge_kernel<TOKEN_MAJOR, 3><<<mgrid, 256, 0, s>>>(fa);
        else flash_merge_kernel<TOKEN_MAJOR, 4><<<mgrid, 256, 0, s>>>(fa);
    }
    return hipGetLastError();
}

// Rows of hd < 64 floats widened to 64 (zeros past hd); blockIdx.y picks
// one of the three operands, a thread writes one float4 of a padded row.
__global__ __launch_bounds__(256) void pad_rows64_kernel(const float *__restrict__ q,
                                                         const float *__restrict__ k,
                                                         const float *__restrict__ v,
                                                         float *__restrict__ pq,
                                                         float *__restrict__ pk,
                                                         float *__restrict__ pv, size_t rows,
                                                         int hd) {
    const float *src = blockIdx.y == 0 ? q : (blockIdx.y == 1 ? k : v);
    float *dst = blockIdx.y == 0 ? pq : (blockIdx.y == 1 ? pk : pv);
    const size_t n = rows * 16;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const size_t row = i >> 4;
        const int d0 = (int)(i & 15) * 4;
        const float *sr = src + row * hd;
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; e++) o[e] = d0 + e < hd ? sr[d0 + e] : 0.0f;
        *reinterpret_cast<f32x4 *>(dst + row * D + d0) = o;
    }
}

// The first hd columns of 64-wide rows, packed into hd-wide rows.
__global__ __launch_bounds__(256) void unpad_rows_kernel(const float *__restrict__ src,
                                                         float *__restrict__ dst, size_t rows,
                                                         int hd) {
    const size_t n = rows * hd;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const size_t row = i / hd;
        dst[i] = src[row * D + (i - row * hd)];
    }
}

unsigned stride_grid(size_t threads) {
    return (unsigned)std::min<size_t>((threads + 255) / 256, 16384);
}

}  // namespace

size_t flash_workspace_floats(size_t bh, size_t tokens) {
    return (size_t)kMaxFlashSplits * bh * tokens * (D + 2);
}

size_t flash_fused_workspace_floats(size_t bh, size_t tokens) {
    return (size_t)kMaxFlashSplits * flash_query_groups(bh, tokens) * kFusedPartial;
}

size_t flash_query_groups(size_t bh, size_t tokens) { return bh * ((tokens + BQ - 1) / BQ); }

hipError_t launch_flash_attention(hipStream_t s, const float *q, const float *k, const float *v,
                                  float *out, size_t bh, size_t tokens, size_t heads,
                                  bool token_major, float *ws, size_t ws_floats, int8_t *q8_qs,
                                  uint16_t *q8_d, bool *quantized, float softmax_scale,
                                  unsigned *cnt, size_t cnt_n) {
    if (quantized) *quantized = false;
    if (bh == 0 || tokens == 0) return hipSuccess;
    FlashArgs fa{};
    fa.scale_log2 = softmax_scale * kLog2e;
    fa.q = q;
    fa.k = k;
    fa.v = v;
    fa.out = out;
    fa.T = (int)tokens;
    fa.heads = (int)heads;
    fa.bh = (int)bh;
    fa.qtiles = (int)((tokens + BQ - 1) / BQ);
    fa.xcd_map = 1;
    if (const char *e = std::getenv("VESTRA_HIP_FLASH_XCD")) fa.xcd_map = std::atoi(e) != 0;

    // Layout choice by a per-SIMD load model, in 64-key panels: two key
    // streams in one workgroup per CU, or one stream with two workgroups per
    // CU, optionally splitting the keys across workgroups (plus a merge
    // pass) when the grid alone leaves CUs idle.
    const long items = (long)fa.bh * fa.qtiles;
    const long panels = ((long)tokens + BKV - 1) / BKV;
    auto rounds = [](long wgs, long slots) { return (wgs + slots - 1) / slots; };
    long best = rounds(items, 256) * panels;
    int streams = 2, splits = 1;
    if (rounds(items, 512) * 2 * panels < best) {
        best = rounds(items, 512) * 2 * panels;
        streams = 1;
    }
    auto split_keys = [&](int sp) { return (int)((panels + sp - 1) / sp) * BKV; };
    auto usable = [&](int sp) {
        const long pps = (panels + sp - 1) / sp;
        return sp >= 2 && sp <= kMaxFlashSplits && (panels + pps - 1) / pps == sp &&
               ws != nullptr && ws_floats >= (size_t)sp * bh * tokens * (D + 2);
    };
    for (int sp = 2; sp <= kMaxFlashSplits; sp++) {
        if (!usable(sp)) continue;
        const long cost = rounds(items * sp, 512) * 2 * (split_keys(sp) / BKV) + 1;
        if (cost < best) {
            best = cost;
            splits = sp;
            streams = 1;
        }
    }
    // Overrides for A/B runs: VESTRA_HIP_FLASH_SPLITS (1 = none) and
    // VESTRA_HIP_FLASH_STREAMS (1 or 2, unsplit only).
    if (const char *e = std::getenv("VESTRA_HIP_FLASH_SPLITS")) {
        const int sp = std::atoi(e);
        if (sp <= 1) splits = 1;
        else if (usable(sp)) splits = sp, streams = 1;
    }
    if (const char *e = std::getenv("VESTRA_HIP_FLASH_STREAMS"))
        if (splits == 1) streams = std::atoi(e) == 2 ? 2 : 1;

    // One-stream layouts run the direct-to-LDS kernel
    // (VESTRA_HIP_FLASH_DIRECT=0 selects the register-staged loop for A/B runs).
    bool direct = true;
    if (const char *e = std::getenv("VESTRA_HIP_FLASH_DIRECT")) direct = std::atoi(e) != 0;
    if (splits > 1) {
        fa.splits = splits;
        fa.split_keys = split_keys(splits);
        fa.po = ws;
        fa.pml = reinterpret_cast<float2 *>(ws + (size_t)splits * bh * tokens * D);
        if (token_major && q8_qs && q8_d) {
            fa.q8_qs = q8_qs;
            fa.q8_d = q8_d;
            if (quantized) *quantized = true;
        }
        // The last split of each query group merges in the kernel when the
        // caller gives the arrival counters and room for the thread-major
        // partials, and the grid is one round of workgroups (two per CU):
        // then every group's last split merges at the very end, where the
        // merge launch would add its own launch and first-load latency
        // (block at 865 tokens 152.5 -> 151.9 us).  Over several rounds the
        // merge launch is faster: it reads partials the L2 still holds,
        // where the in-kernel merge writes them through and reads them back
        // (12-layer encoder at 4 x 865 tokens 6.13 against 6.21 ms).
        // VESTRA_HIP_FLASH_FUSED=0 / 1 turns it off / on whenever possible.
        bool fused = direct && cnt != nullptr && cnt_n >= (size_t)items &&
                     ws_floats >= (size_t)splits * items * kFusedPartial;
        if (const char *e = std::getenv("VESTRA_HIP_FLASH_FUSED")) fused = fused && std::atoi(e) != 0;
        else fused = fused && items * splits <= 512;
        if (fused) {
            fa.pt = ws;
            fa.cnt = cnt;
            return token_major ? run_flash_direct<true, true, true>(s, fa)
                               : run_flash_direct<false, true, true>(s, fa);
        }
        if (direct)
            return token_major ? run_flash_direct<true, true>(s, fa) : run_flash_direct<false, true>(s, fa);
        return token_major ? run_flash<true, 1, true>(s, fa) : run_flash<false, 1, true>(s, fa);
    }
    fa.splits = 1;
    fa.split_keys = (int)tokens;
    if (streams == 2)
        return token_major ? run_flash<true, 2, false>(s, fa) : run_flash<false, 2, false>(s, fa);
    if (direct)
        return token_major ? run_flash_direct<true, false>(s, fa) : run_flash_direct<false, false>(s, fa);
    return token_major ? run_flash<true, 1, false>(s, fa) : run_flash<false, 1, false>(s, fa);
}

hipError_t launch_pad_rows64(hipStream_t s, const float *q, const float *k, const float *v,
                             float *pq, float *pk, float *pv, size_t rows, size_t hd) {
    if (rows == 0) return hipSuccess;
    pad_rows64_kernel<<<dim3(stride_grid(rows * 16), 3), 256, 0, s>>>(q, k, v, pq, pk, pv, rows,
                                                                     (int)hd);
    return hipGetLastError();
}

hipError_t launch_unpad_rows(hipStream_t s, const float *src, float *dst, size_t rows, size_t hd) {
    if (rows == 0) return hipSuccess;
    unpad_rows_kernel<<<stride_grid(rows * hd), 256, 0, s>>>(src, dst, rows, (int)hd);
    return hipGetLastError();
}

}  // namespace vh
