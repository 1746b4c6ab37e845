// HBM-bound elementwise, normalisation, RoPE and layout kernels (gfx950).
//
// Every kernel is a coalesced grid-stride loop or a wave64-per-row
// reduction.  Arithmetic that restates a reference op uses separately
// rounded adds and multiplies (add_rn/mul_rn) so the compiler cannot
// contract it into FMAs the reference never executes.
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace vh {

namespace {

constexpr int kThreads = 256;

// Launches that move at least this many bytes stream: non-temporal loads
// and stores (no L2 / Infinity Cache retention), four float4 per thread in
// flight.  On MI355X that lifts a 512 MiB copy from 5.6 to 6.4 TB/s; below
// the threshold the data is left cached for the kernel that consumes it.
constexpr size_t kStreamBytes = size_t(128) << 20;

template <bool NT, class T>
__device__ __forceinline__ T ld(const T *p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}
template <bool NT, class T>
__device__ __forceinline__ void st(T *p, T v) {
    if constexpr (NT) __builtin_nontemporal_store(v, p);
    else *p = v;
}

inline unsigned grid_for(size_t n, size_t per_thread = 1) {
    size_t blocks = (n + kThreads * per_thread - 1) / (kThreads * per_thread);
    if (blocks == 0) blocks = 1;
    // 256 CUs x 8 resident blocks is plenty for a grid-stride loop.
    return (unsigned)(blocks < 2048 * 8 ? blocks : 2048 * 8);
}

__global__ void add_kernel(float *__restrict__ dst, const float *__restrict__ src, size_t n) {
    size_t n4 = n / 4;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    bool aligned = ((((uintptr_t)dst) | ((uintptr_t)src)) & 15) == 0;
    if (aligned) {
        for (size_t j = i; j < n4; j += stride) {
            f32x4 a = reinterpret_cast<f32x4 *>(dst)[j];
            f32x4 b = reinterpret_cast<const f32x4 *>(src)[j];
            reinterpret_cast<f32x4 *>(dst)[j] = a + b;
        }
        for (size_t j = n4 * 4 + i; j < n; j += stride) dst[j] = dst[j] + src[j];
    } else {
        for (size_t j = i; j < n; j += stride) dst[j] = dst[j] + src[j];
    }
}

// Streaming copy: four float4 per thread loaded before any store,
// non-temporal accesses (n % 4 == 0, 16-byte aligned, no overlap).
__global__ __launch_bounds__(256) void stream_copy_kernel(float *__restrict__ dst,
                                                          const float *__restrict__ src, size_t n4) {
    f32x4 *d4 = reinterpret_cast<f32x4 *>(dst);
    const f32x4 *s4 = reinterpret_cast<const f32x4 *>(src);
    const size_t stride = (size_t)gridDim.x * 1024;
    for (size_t base = (size_t)blockIdx.x * 1024 + threadIdx.x; base < n4; base += stride) {
        f32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (base + 256 * u < n4) v[u] = ld<true>(s4 + base + 256 * u);
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (base + 256 * u < n4) st<true>(d4 + base + 256 * u, v[u]);
    }
}

// add_kernel's streaming form (16-byte aligned operands): four float4 of
// each operand loaded per thread before any add, non-temporal accesses.
__global__ __launch_bounds__(256) void add_stream_kernel(float *__restrict__ dst,
                                                         const float *__restrict__ src, size_t n) {
    const size_t n4 = n / 4;
    f32x4 *d4 = reinterpret_cast<f32x4 *>(dst);
    const f32x4 *s4 = reinterpret_cast<const f32x4 *>(src);
    const size_t stride = (size_t)gridDim.x * 1024;
    for (size_t base = (size_t)blockIdx.x * 1024 + threadIdx.x; base < n4; base += stride) {
        f32x4 a[4], b[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const size_t j = base + 256 * u;
            if (j < n4) {
                a[u] = ld<true>(d4 + j);
                b[u] = ld<true>(s4 + j);
            }
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const size_t j = base + 256 * u;
            if (j < n4) st<true>(d4 + j, a[u] + b[u]);
        }
    }
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (t < n - n4 * 4) dst[n4 * 4 + t] = dst[n4 * 4 + t] + src[n4 * 4 + t];
}

// src/cuda.rs:56-69: values = (values + bias[c]) * gamma[c]
__global__ void bias_scale_kernel(float *__restrict__ v, const float *__restrict__ bias,
                                  const float *__restrict__ gamma, size_t rows, size_t cols) {
    size_t n = rows * cols;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        size_t c = i % cols;
        v[i] = mul_rn(add_rn(v[i], bias[c]), gamma[c]);
    }
}

// Kernels::gelu (src/dispatch.rs:56-73): AVX-512 form on the first n - n%16
// values, scalar::gelu on the tail.
__global__ void gelu_kernel(float *__restrict__ v, size_t n) {
    size_t main = n - (n % 16);
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        float x = v[i];
        v[i] = i < main ? gelu_avx512_form(x) : gelu_scalar_form(x);
    }
}

// Four values per thread with 16-byte accesses (v 16-byte aligned, n % 4 ==
// 0); every element takes the same form as in gelu_kernel.
__global__ __launch_bounds__(256) void gelu4_kernel(float *__restrict__ v, size_t n4, size_t main) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    f32x4 *v4 = reinterpret_cast<f32x4 *>(v);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
        f32x4 x = v4[i];
#pragma unroll
        for (int e = 0; e < 4; e++)
            x[e] = 4 * i + e < main ? gelu_avx512_form(x[e]) : gelu_scalar_form(x[e]);
        v4[i] = x;
    }
}

// gelu4_kernel's streaming form: four float4 per thread loaded before any
// arithmetic, non-temporal accesses; the same form per element.
__global__ __launch_bounds__(256) void gelu4_stream_kernel(float *__restrict__ v, size_t n4,
                                                           size_t main) {
    const size_t stride = (size_t)gridDim.x * 1024;
    f32x4 *v4 = reinterpret_cast<f32x4 *>(v);
    for (size_t base = (size_t)blockIdx.x * 1024 + threadIdx.x; base < n4; base += stride) {
        f32x4 x[4];
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (base + 256 * u < n4) x[u] = ld<true>(v4 + base + 256 * u);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const size_t i = base + 256 * u;
            if (i >= n4) continue;
#pragma unroll
            for (int e = 0; e < 4; e++)
                x[u][e] = 4 * i + e < main ? gelu_avx512_form(x[u][e]) : gelu_scalar_form(x[u][e]);
            st<true>(v4 + i, x[u]);
        }
    }
}

// One wave64 per row; up to 4 float4 per lane stay in registers (cols <= 1024
// and cols % 4 == 0), otherwise the row is re-read.  Tree reductions differ
// from the sequential CPU sums only in rounding (tolerance-checked).
template <bool NT>
__global__ __launch_bounds__(256) void layernorm_kernel(const float *__restrict__ in,
                                                        const float *__restrict__ gamma,
                                                        const float *__restrict__ beta,
                                                        float *__restrict__ out, size_t rows,
                                                        size_t cols, float eps) {
    const int lane = threadIdx.x & 63;
    size_t row = (size_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *x = in + row * cols;
    float *y = out + row * cols;
    if ((cols & 3) == 0 && cols <= 1024 && ((((uintptr_t)x) | ((uintptr_t)y)) & 15) == 0) {
        const int n4 = (int)(cols >> 2);
        // Every read (the row, gamma, beta) is issued before the statistics:
        // gamma and beta come from clamped indices (chunks past the row end
        // read chunk 0 and are dropped), so that no load waits behind the
        // bounds branch of its store.
        f32x4 r[4], g[4], b[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int idx = lane + j * 64, ci = idx < n4 ? idx : 0;
            r[j] = idx < n4 ? ld<NT>(reinterpret_cast<const f32x4 *>(x) + idx) : f32x4{0, 0, 0, 0};
            g[j] = reinterpret_cast<const f32x4 *>(gamma)[ci];
            b[j] = reinterpret_cast<const f32x4 *>(beta)[ci];
        }
        float mean, inv;
        ln_row_stats(r, lane, n4, (int)cols, eps, mean, inv);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int idx = lane + j * 64;
            if (idx < n4) st<NT>(reinterpret_cast<f32x4 *>(y) + idx, ln_apply(r[j], mean, inv, g[j], b[j]));
        }
    } else {
        float s = 0.0f;
        for (size_t c = lane; c < cols; c += 64) s += x[c];
        float mean = div_rn(wave_sum(s), (float)cols);
        float q = 0.0f;
        for (size_t c = lane; c < cols; c += 64) {
            float d = x[c] - mean;
            q += d * d;
        }
        float var = div_rn(wave_sum(q), (float)cols);
        float inv = div_rn(1.0f, sqrt_rn(add_rn(var, eps)));
        for (size_t c = lane; c < cols; c += 64)
            y[c] = add_rn(mul_rn(mul_rn(sub_rn(x[c], mean), inv), gamma[c]), beta[c]);
    }
}

// scalar::layernorm_row (src/scalar.rs:99-114) verbatim, one thread per row:
// sequential sums from -0.0, every op separately rounded.
__global__ void layernorm_cpu_order_kernel(const float *__restrict__ in,
                                           const float *__restrict__ gamma,
                                           const float *__restrict__ beta,
                                           float *__restrict__ out, size_t rows, size_t cols,
                                           float eps) {
    size_t row = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    const float *x = in + row * cols;
    float *y = out + row * cols;
    float sum = -0.0f;
    for (size_t c = 0; c < cols; c++) sum = add_rn(sum, x[c]);
    float mean = div_rn(sum, (float)cols);
    float sq = -0.0f;
    for (size_t c = 0; c < cols; c++) {
        float d = sub_rn(x[c], mean);
        sq = add_rn(sq, mul_rn(d, d));
    }
    float var = div_rn(sq, (float)cols);
    float inv = div_rn(1.0f, sqrt_rn(add_rn(var, eps)));
    for (size_t c = 0; c < cols; c++)
        y[c] = add_rn(mul_rn(mul_rn(sub_rn(x[c], mean), inv), gamma[c]), beta[c]);
}

// src/cuda.rs:243-259 semantics.
__global__ void split_qkv_kernel(const float *__restrict__ qkv, float *__restrict__ q,
                                 float *__restrict__ k, float *__restrict__ v, size_t tokens,
                                 size_t heads, size_t hd) {
    size_t per = heads * hd, n = tokens * per;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        size_t t = i / per, w = i % per;
        size_t src = t * 3 * per + w;
        size_t hm = (w / hd) * tokens * hd + t * hd + (w % hd);
        q[hm] = qkv[src];
        k[hm] = qkv[src + per];
        v[hm] = qkv[src + 2 * per];
    }
}

// src/cuda.rs:263-276 semantics.
__global__ void hnd_to_token_kernel(const float *__restrict__ hnd, float *__restrict__ out,
                                    size_t tokens, size_t heads, size_t hd) {
    size_t per = heads * hd, n = tokens * per;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        size_t t = i / per, w = i % per;
        out[i] = hnd[(w / hd) * tokens * hd + t * hd + (w % hd)];
    }
}

// src/cuda.rs:281-291 semantics: [tokens, channels] -> [channels, tokens].
__global__ void token_to_chw_kernel(const float *__restrict__ tm, float *__restrict__ chw,
                                    size_t tokens, size_t channels) {
    size_t n = tokens * channels;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        size_t c = i / tokens, t = i % tokens;  // write-coalesced
        chw[i] = tm[t * channels + c];
    }
}

// src/cuda.rs:295-316 semantics: NCHW image -> rows of [channel, py, px].
__global__ void patchify_kernel(const float *__restrict__ image, float *__restrict__ patches,
                                size_t height, size_t width, size_t patch, size_t channels) {
    size_t area = patch * patch, row_w = channels * area;
    size_t gw = width / patch, count = (height / patch) * gw, n = count * row_w;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        size_t pi = i / row_w, wi = i % row_w;
        size_t ch = wi / area, sp = wi % area;
        size_t y = (pi / gw) * patch + sp / patch, x = (pi % gw) * patch + sp % patch;
        patches[i] = image[(ch * height + y) * width + x];
    }
}

// src/cuda.rs:321-334 semantics.
__global__ void prepend_cls_add_pos_kernel(const float *__restrict__ patches,
                                           const float *__restrict__ cls,
                                           const float *__restrict__ pos, float *__restrict__ out,
                                           size_t patch_count, size_t embed) {
    size_t n = (patch_count + 1) * embed;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        size_t t = i / embed, c = i % embed;
        float v = t == 0 ? cls[c] : patches[(t - 1) * embed + c];
        out[i] = add_rn(v, pos[i]);
    }
}

// rope::rope2d (src/rope.rs:30-93): one thread per rotation pair.
// rot: [n][2][quarter][sin, cos]
__global__ void rope2d_kernel(float *__restrict__ x, size_t heads, size_t n, size_t hd,
                              const float *__restrict__ rot) {
    size_t half = hd / 2, quarter = half / 2;
    size_t pairs = heads * n * 2 * quarter;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < pairs; i += stride) {
        size_t qi = i % quarter;
        size_t axis = (i / quarter) % 2;
        size_t row = i / (2 * quarter);  // h * n + p
        size_t p = row % n;
        float *base = x + row * hd + axis * half;
        size_t r = ((p * 2 + axis) * quarter + qi) * 2;
        float sn = rot[r], cs = rot[r + 1];
        float a = base[qi], b = base[qi + quarter];
        base[qi] = sub_rn(mul_rn(a, cs), mul_rn(b, sn));
        base[qi + quarter] = add_rn(mul_rn(b, cs), mul_rn(a, sn));
    }
}

// rope2d for head_dim 64 (the DA3 shape), the same arithmetic as
// rope2d_kernel: 16 lanes per 64-wide row, lane j holding dims 4j..4j+3
// (axis j / 8); the rotation partner (dim +/- 16) lives in lane j ^ 4.
// Rows are contiguous, so a wave reads and writes 1 KB at a time, and the
// [n][2][16][sin, cos] table is read as two float4 per lane.
template <bool NT>
__global__ __launch_bounds__(256) void rope2d_hd64_kernel(float *__restrict__ x, int rows, int n,
                                                          const float *__restrict__ rot) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    const int row = min(t >> 4, rows - 1);  // idle lanes shadow the last row
    const int j = t & 15;
    f32x4 *p = reinterpret_cast<f32x4 *>(x + (size_t)row * 64) + j;
    const f32x4 v = ld<NT>(p);
    f32x4 w;
#pragma unroll
    for (int e = 0; e < 4; e++) w[e] = __shfl_xor(v[e], 4, 16);
    const int pos = row % n, axis = j >> 3, q4 = (j & 3) * 4;
    const f32x4 *rp = reinterpret_cast<const f32x4 *>(rot + (((size_t)pos * 2 + axis) * 16 + q4) * 2);
    const f32x4 r0 = rp[0], r1 = rp[1];  // (sin, cos) of dims q4 .. q4 + 3
    const float sn[4] = {r0[0], r0[2], r1[0], r1[2]}, cs[4] = {r0[1], r0[3], r1[1], r1[3]};
    const bool first = (j & 4) == 0;  // holds the a values of (a, b) = (dim, dim + 16)
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; e++)
        o[e] = first ? sub_rn(mul_rn(v[e], cs[e]), mul_rn(w[e], sn[e]))
                     : add_rn(mul_rn(v[e], cs[e]), mul_rn(w[e], sn[e]));
    if ((t >> 4) < rows) st<NT>(p, o);
}

// qk_norm_rope (src/specialized.rs:412-454): 16 lanes per 64-wide row, lane j
// holds dims 4j..4j+3; the rotation partner (dim + 16) lives in lane j ^ 4.
// LayerNorm sums use a 16-lane tree (tolerance-checked against the CPU order).
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    float *__restrict__ q, float *__restrict__ k, const float *__restrict__ qg,
    const float *__restrict__ qb, const float *__restrict__ kg, const float *__restrict__ kb,
    const float *__restrict__ rot, size_t rows, size_t tokens, float eps) {
    size_t gid = (size_t)blockIdx.x * 16 + (threadIdx.x >> 4);  // row over [q rows | k rows]
    const int j = threadIdx.x & 15;
    bool valid = gid < 2 * rows;
    size_t row = valid ? (gid < rows ? gid : gid - rows) : 0;
    float *data = (gid < rows ? q : k) + row * 64;
    const float *g = gid < rows ? qg : kg;
    const float *b = gid < rows ? qb : kb;
    f32x4 v = valid ? reinterpret_cast<f32x4 *>(data)[j] : f32x4{0, 0, 0, 0};
    float s = (v.x + v.y) + (v.z + v.w);
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) s += __shfl_xor(s, o, 16);
    float mean = div_rn(s, 64.0f);
    f32x4 d = v - mean;
    float sq = (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) sq += __shfl_xor(sq, o, 16);
    float inv = div_rn(1.0f, sqrt_rn(add_rn(div_rn(sq, 64.0f), eps)));
    f32x4 gv = reinterpret_cast<const f32x4 *>(g)[j];
    f32x4 bv = reinterpret_cast<const f32x4 *>(b)[j];
    f32x4 nrm;
    nrm.x = add_rn(mul_rn(mul_rn(sub_rn(v.x, mean), inv), gv.x), bv.x);
    nrm.y = add_rn(mul_rn(mul_rn(sub_rn(v.y, mean), inv), gv.y), bv.y);
    nrm.z = add_rn(mul_rn(mul_rn(sub_rn(v.z, mean), inv), gv.z), bv.z);
    nrm.w = add_rn(mul_rn(mul_rn(sub_rn(v.w, mean), inv), gv.w), bv.w);
    f32x4 other;
    other.x = __shfl_xor(nrm.x, 4, 16);
    other.y = __shfl_xor(nrm.y, 4, 16);
    other.z = __shfl_xor(nrm.z, 4, 16);
    other.w = __shfl_xor(nrm.w, 4, 16);
    if (!valid) return;
    size_t token = row % tokens;
    int axis = j >> 3;
    bool first = (j & 4) == 0;  // dims [0,16) of the axis half
    f32x4 outv;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        int i = ((j & 3) * 4 + c);  // index within the quarter
        const float *rr = rot + ((token * 2 + axis) * 16 + i) * 2;
        float sn = rr[0], cs = rr[1];
        float mine = nrm[c], part = other[c];
        outv[c] = first ? sub_rn(mul_rn(mine, cs), mul_rn(part, sn))
                        : add_rn(mul_rn(mine, cs), mul_rn(part, sn));
    }
    reinterpret_cast<f32x4 *>(data)[j] = outv;
}

// Rotation table from device positions (f32 [tokens][2]) with the device
// libm, as the reference's device kernel computes its angles
// (src/cuda.rs:222-236): rot[((t*2 + axis)*16 + i)*2 + {sin, cos}],
// theta_i = freq^(-2i/32).
__global__ void rope_table_kernel(const float *__restrict__ pos, size_t tokens, float freq,
                                  float *__restrict__ rot) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= tokens * 32) return;
    size_t t = i / 32, axis = (i / 16) % 2, qi = i % 16;
    float inv = powf(freq, div_rn(mul_rn(-2.0f, (float)qi), 32.0f));
    float arg = mul_rn(pos[2 * t + axis], inv);
    rot[i * 2] = sinf(arg);
    rot[i * 2 + 1] = cosf(arg);
}

// 32x32 tile transpose through LDS: out[c][r] = in[r][c].
__global__ __launch_bounds__(256) void transpose_kernel(const float *__restrict__ in,
                                                        float *__restrict__ out, size_t rows,
                                                        size_t cols) {
    __shared__ float tile[32][33];
    size_t c0 = (size_t)blockIdx.x * 32, r0 = (size_t)blockIdx.y * 32;
    int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int j = ty; j < 32; j += 8) {
        size_t r = r0 + j, c = c0 + tx;
        if (r < rows && c < cols) tile[j][tx] = in[r * cols + c];
    }
    __syncthreads();
    for (int j = ty; j < 32; j += 8) {
        size_t c = c0 + j, r = r0 + tx;
        if (r < rows && c < cols) out[c * rows + r] = tile[tx][j];
    }
}

}  // namespace

bool stream_copy_applies(float *dst, const float *src, size_t n) {
    const uintptr_t d = reinterpret_cast<uintptr_t>(dst), r = reinterpret_cast<uintptr_t>(src);
    const size_t bytes = n * sizeof(float);
    const bool disjoint = d + bytes <= r || r + bytes <= d;
    return n % 4 == 0 && ((d | r) & 15) == 0 && disjoint && 2 * bytes >= kStreamBytes;
}

hipError_t launch_stream_copy(hipStream_t s, float *dst, const float *src, size_t n) {
    if (n == 0) return hipSuccess;
    const size_t blocks = std::min<size_t>((n / 4 + 1023) / 1024, 16384);
    stream_copy_kernel<<<(unsigned)std::max<size_t>(blocks, 1), 256, 0, s>>>(dst, src, n / 4);
    return hipGetLastError();
}

hipError_t launch_add(hipStream_t s, float *dst, const float *src, size_t n) {
    if (n == 0) return hipSuccess;
    const bool aligned = ((((uintptr_t)dst) | ((uintptr_t)src)) & 15) == 0;
    if (aligned && 12 * n >= kStreamBytes) {
        const size_t blocks = std::min<size_t>((n / 4 + 1023) / 1024, 16384);
        add_stream_kernel<<<(unsigned)std::max<size_t>(blocks, 1), 256, 0, s>>>(dst, src, n);
    } else {
        add_kernel<<<grid_for(n, 4), kThreads, 0, s>>>(dst, src, n);
    }
    return hipGetLastError();
}

hipError_t launch_bias_scale(hipStream_t s, float *v, const float *bias, const float *gamma,
                             size_t rows, size_t cols) {
    if (rows * cols == 0) return hipSuccess;
    bias_scale_kernel<<<grid_for(rows * cols), kThreads, 0, s>>>(v, bias, gamma, rows, cols);
    return hipGetLastError();
}

hipError_t launch_gelu(hipStream_t s, float *v, size_t n) {
    if (n == 0) return hipSuccess;
    if (n % 4 == 0 && (reinterpret_cast<uintptr_t>(v) & 15) == 0 && 8 * n >= kStreamBytes)
        gelu4_stream_kernel<<<(unsigned)std::min<size_t>((n / 4 + 1023) / 1024, 16384), 256, 0, s>>>(
            v, n / 4, n - n % 16);
    else if (n % 4 == 0 && (reinterpret_cast<uintptr_t>(v) & 15) == 0)
        gelu4_kernel<<<grid_for(n / 4), 256, 0, s>>>(v, n / 4, n - n % 16);
    else
        gelu_kernel<<<grid_for(n), kThreads, 0, s>>>(v, n);
    return hipGetLastError();
}

hipError_t launch_layernorm(hipStream_t s, const float *in, const float *gamma,
                            const float *beta, float *out, size_t rows, size_t cols, float eps) {
    if (rows == 0 || cols == 0) return hipSuccess;
    // Up to 2048 rows, one row per workgroup spreads the rows over every CU.
    const unsigned wpb = rows <= 2048 ? 1 : 4;  // waves (rows) per workgroup
    const dim3 grid((unsigned)((rows + wpb - 1) / wpb));
    if (8 * rows * cols >= kStreamBytes)
        layernorm_kernel<true><<<grid, 64 * wpb, 0, s>>>(in, gamma, beta, out, rows, cols, eps);
    else
        layernorm_kernel<false><<<grid, 64 * wpb, 0, s>>>(in, gamma, beta, out, rows, cols, eps);
    return hipGetLastError();
}

hipError_t launch_layernorm_cpu_order(hipStream_t s, const float *in, const float *gamma,
                                      const float *beta, float *out, size_t rows, size_t cols,
                                      float eps) {
    if (rows == 0 || cols == 0) return hipSuccess;
    layernorm_cpu_order_kernel<<<(unsigned)((rows + 63) / 64), 64, 0, s>>>(in, gamma, beta, out,
                                                                            rows, cols, eps);
    return hipGetLastError();
}

hipError_t launch_split_qkv(hipStream_t s, const float *qkv, float *q, float *k, float *v,
                            size_t tokens, size_t heads, size_t head_dim) {
    size_t n = tokens * heads * head_dim;
    if (n == 0) return hipSuccess;
    split_qkv_kernel<<<grid_for(n), kThreads, 0, s>>>(qkv, q, k, v, tokens, heads, head_dim);
    return hipGetLastError();
}

hipError_t launch_hnd_to_token(hipStream_t s, const float *hnd, float *out, size_t tokens,
                               size_t heads, size_t head_dim) {
    size_t n = tokens * heads * head_dim;
    if (n == 0) return hipSuccess;
    hnd_to_token_kernel<<<grid_for(n), kThreads, 0, s>>>(hnd, out, tokens, heads, head_dim);
    return hipGetLastError();
}

hipError_t launch_token_to_chw(hipStream_t s, const float *tm, float *chw, size_t tokens,
                               size_t channels) {
    size_t n = tokens * channels;
    if (n == 0) return hipSuccess;
    token_to_chw_kernel<<<grid_for(n), kThreads, 0, s>>>(tm, chw, tokens, channels);
    return hipGetLastError();
}

hipError_t launch_patchify(hipStream_t s, const float *image, float *patches, size_t height,
                           size_t width, size_t patch, size_t channels) {
    size_t n = (height / patch) * (width / patch) * channels * patch * patch;
    if (n == 0) return hipSuccess;
    patchify_kernel<<<grid_for(n), kThreads, 0, s>>>(image, patches, height, width, patch,
                                                     channels);
    return hipGetLastError();
}

hipError_t launch_prepend_cls_add_pos(hipStream_t s, const float *patches, const float *cls,
                                      const float *pos, float *out, size_t patch_count,
                                      size_t embed) {
    size_t n = (patch_count + 1) * embed;
    if (n == 0) return hipSuccess;
    prepend_cls_add_pos_kernel<<<grid_for(n), kThreads, 0, s>>>(patches, cls, pos, out,
                                                                patch_count, embed);
    return hipGetLastError();
}

hipError_t launch_rope2d(hipStream_t s, float *x, size_t heads, size_t n, size_t head_dim,
                         const float *rot) {
    size_t pairs = heads * n * (head_dim / 2);
    if (pairs == 0) return hipSuccess;
    const size_t rows = heads * n;
    if (head_dim == 64 && rows <= (size_t)INT32_MAX / 16) {
        const unsigned blocks = (unsigned)((rows * 16 + 255) / 256);
        if (rows * 64 * 8 >= kStreamBytes)
            rope2d_hd64_kernel<true><<<blocks, 256, 0, s>>>(x, (int)rows, (int)n, rot);
        else
            rope2d_hd64_kernel<false><<<blocks, 256, 0, s>>>(x, (int)rows, (int)n, rot);
        return hipGetLastError();
    }
    rope2d_kernel<<<grid_for(pairs), kThreads, 0, s>>>(x, heads, n, head_dim, rot);
    return hipGetLastError();
}

hipError_t launch_qk_norm_rope(hipStream_t s, float *q, float *k, const float *qg,
                               const float *qb, const float *kg, const float *kb,
                               const float *rot, size_t rows, size_t tokens, float eps) {
    if (rows == 0) return hipSuccess;
    size_t blocks = (2 * rows + 15) / 16;
    qk_norm_rope_kernel<<<(unsigned)blocks, 256, 0, s>>>(q, k, qg, qb, kg, kb, rot, rows, tokens,
                                                         eps);
    return hipGetLastError();
}

hipError_t launch_rope_table_device(hipStream_t s, const float *pos, size_t tokens, float freq,
                                    float *rot) {
    if (tokens == 0) return hipSuccess;
    rope_table_kernel<<<(unsigned)((tokens * 32 + 255) / 256), 256, 0, s>>>(pos, tokens, freq, rot);
    return hipGetLastError();
}

hipError_t launch_transpose(hipStream_t s, const float *in, float *out, size_t rows,
                            size_t cols) {
    if (rows == 0 || cols == 0) return hipSuccess;
    dim3 grid((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32));
    transpose_kernel<<<grid, 256, 0, s>>>(in, out, rows, cols);
    return hipGetLastError();
}

}  // namespace vh
