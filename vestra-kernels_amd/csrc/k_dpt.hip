// DPT-head building blocks for gfx950: convolution operand staging,
// transposed-convolution scatter and bilinear resampling.
//
// A convolution runs as one fp32-MFMA GEMM (k_gemm.hip): the input patches
// are gathered into colT [oh*ow][in_c*kh*kw] (one row per output pixel,
// k-contiguous like the GEMM's A operand), the OIHW weight is already
// [out_c][in_c*kh*kw] (the GEMM's Bt operand), and the GEMM's bias epilogue
// adds the per-channel bias.  Its [pixel][out_c] result is transposed to CHW.
// A non-overlapping transposed convolution (kernel == stride) is the same
// GEMM over [pixel][in_c] against the filter packed as [out_c*kh*kw][in_c],
// followed by a scatter of each pixel's kh x kw patch.
//
// The resize kernels restate src/resample.rs op for op (separately rounded
// f32 ops, the same coordinate formulas), so they are bit-exact.
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace vh {
namespace {

// colT[p][k] for a 64-pixel x 64-k tile: read with pixels fastest (adjacent
// output columns read adjacent input columns), transpose through LDS, write
// with k fastest.  k = (ic * kh + ky) * kw + kx, the OIHW flattening.
__global__ __launch_bounds__(256) void im2col_t_kernel(const float *__restrict__ in,
                                                       float *__restrict__ col, int in_c, int ih,
                                                       int iw, int kh, int kw, int stride,
                                                       int pad, int oh, int ow, int relu) {
    __shared__ float tile[64][65];
    const int npix = oh * ow, K = in_c * kh * kw;
    const int p0 = blockIdx.x * 64, k0 = blockIdx.y * 64;
    const int t = threadIdx.x;
    {
        const int pl = t & 63, kr = t >> 6;
        const int p = p0 + pl;
        const int oy = p / ow, ox = p % ow;
#pragma unroll 4
        for (int r = 0; r < 16; r++) {
            const int kl = kr * 16 + r, k = k0 + kl;
            float v = 0.0f;
            if (p < npix && k < K) {
                const int ic = k / (kh * kw), kk = k % (kh * kw);
                const int iy = oy * stride + kk / kw - pad, ix = ox * stride + kk % kw - pad;
                if (iy >= 0 && iy < ih && ix >= 0 && ix < iw) {
                    v = in[((size_t)ic * ih + iy) * iw + ix];
                    if (relu) v = fmaxf(v, 0.0f);
                }
            }
            tile[kl][pl] = v;
        }
    }
    __syncthreads();
    {
        const int kl = t & 63, pr = t >> 6;
        const int k = k0 + kl;
        if (k >= K) return;
#pragma unroll 4
        for (int r = 0; r < 16; r++) {
            const int pl = pr * 16 + r, p = p0 + pl;
            if (p < npix) col[(size_t)p * K + k] = tile[kl][pl];
        }
    }
}

// colT[p][(ky*kw + kx)*in_c + ic] from a channel-last input xh [ih*iw][in_c]
// (in_c % 4 == 0): each tap of a pixel is one contiguous run of in_c values,
// copied as float4, zeros where the tap falls in the padding.  One workgroup
// walks whole pixels, so the writes of a row are contiguous.
__global__ __launch_bounds__(256) void im2col_hwc_kernel(const float *__restrict__ xh,
                                                         float *__restrict__ col, int in_c, int ih,
                                                         int iw, int kh, int kw, int stride,
                                                         int pad, int oh, int ow, int relu) {
    const int c4n = in_c / 4, K4 = c4n * kh * kw, npix = oh * ow;
    for (int p = blockIdx.x; p < npix; p += gridDim.x) {
        const int oy = p / ow, ox = p % ow;
        f32x4 *dst = reinterpret_cast<f32x4 *>(col + (size_t)p * K4 * 4);
        for (int j = threadIdx.x; j < K4; j += blockDim.x) {
            const int tap = j / c4n, c4 = j - tap * c4n;
            const int iy = oy * stride + tap / kw - pad, ix = ox * stride + tap % kw - pad;
            f32x4 v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            if (iy >= 0 && iy < ih && ix >= 0 && ix < iw) {
                v = reinterpret_cast<const f32x4 *>(xh + ((size_t)iy * iw + ix) * in_c)[c4];
                if (relu) {
#pragma unroll
                    for (int e = 0; e < 4; e++) v[e] = fmaxf(v[e], 0.0f);
                }
            }
            dst[j] = v;
        }
    }
}

// CHW -> zero-padded channel-last image xp [rows][c]: row r is padded pixel
// (r / wp, r % wp) of the (ih + 2 pad) x wp grid; rows past the grid (the
// implicit GEMM's overrun) and the border are zeros.  32 x 32 tiles through
// LDS: reads run along x, writes along channels.
__global__ __launch_bounds__(256) void chw_to_padded_hwc_kernel(const float *__restrict__ in,
                                                                float *__restrict__ xp, int c,
                                                                int ih, int iw, int pad, int wp,
                                                                int rows, int relu) {
    __shared__ float tile[32][33];
    const int r0 = blockIdx.x * 32, c0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    const int hp = ih + 2 * pad;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int ch = c0 + ty + 8 * k, r = r0 + tx;
        float v = 0.0f;
        if (ch < c && r < rows) {
            const int py = r / wp, px = r - py * wp;
            const int y = py - pad, x = px - pad;
            if (py < hp && y >= 0 && y < ih && x >= 0 && x < iw) {
                v = in[((size_t)ch * ih + y) * iw + x];
                if (relu) v = fmaxf(v, 0.0f);
            }
        }
        tile[ty + 8 * k][tx] = v;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int r = r0 + ty + 8 * k, ch = c0 + tx;
        if (r < rows && ch < c) xp[(size_t)r * c + ch] = tile[tx][ty + 8 * k];
    }
}

// out[oc][iy*kh+ky][ix*kw+kx] = c[iy*iw+ix][(oc*kh+ky)*kw+kx]: one thread per
// output element, so the writes are coalesced.
__global__ __launch_bounds__(256) void patch_scatter_kernel(const float *__restrict__ c,
                                                            float *__restrict__ out, int out_c,
                                                            int ih, int iw, int kh, int kw) {
    const int oh = ih * kh, ow = iw * kw;
    const size_t total = (size_t)out_c * oh * ow;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (size_t)gridDim.x * blockDim.x) {
        const int ox = (int)(e % ow);
        const size_t r = e / ow;
        const int oy = (int)(r % oh), oc = (int)(r / oh);
        const int iy = oy / kh, ky = oy % kh, ix = ox / kw, kx = ox % kw;
        out[e] = c[((size_t)iy * iw + ix) * ((size_t)out_c * kh * kw) + (oc * kh + ky) * kw + kx];
    }
}

// General transposed convolution (any kernel and stride), gathered per
// output element: for each input channel the taps that land on (oy, ox), in
// (ic, ky, kx) order, then the bias.
__global__ __launch_bounds__(256) void conv_transpose_gather_kernel(
    const float *__restrict__ in, const float *__restrict__ w, const float *__restrict__ bias,
    float *__restrict__ out, int in_c, int ih, int iw, int out_c, int kh, int kw, int stride) {
    const int oh = (ih - 1) * stride + kh, ow = (iw - 1) * stride + kw;
    const size_t total = (size_t)out_c * oh * ow;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (size_t)gridDim.x * blockDim.x) {
        const int ox = (int)(e % ow);
        const size_t r = e / ow;
        const int oy = (int)(r % oh), oc = (int)(r / oh);
        float acc = 0.0f;
        for (int ic = 0; ic < in_c; ic++) {
            for (int ky = oy % stride; ky < kh; ky += stride) {
                const int iy = (oy - ky) / stride;
                if (iy < 0 || iy >= ih) continue;
                for (int kx = ox % stride; kx < kw; kx += stride) {
                    const int ix = (ox - kx) / stride;
                    if (ix < 0 || ix >= iw) continue;
                    acc = add_rn(acc, mul_rn(in[((size_t)ic * ih + iy) * iw + ix],
                                             w[(((size_t)ic * out_c + oc) * kh + ky) * kw + kx]));
                }
            }
        }
        if (bias) acc = add_rn(acc, bias[oc]);
        out[e] = acc;
    }
}

struct Tap {
    int i0, i1;
    float frac;
};

// resample::src_coord (src/resample.rs:82-95): half-pixel centres.
__device__ __forceinline__ Tap half_pixel_tap(int dst, float scale, int len_in) {
    const float src = sub_rn(mul_rn(add_rn((float)dst, 0.5f), scale), 0.5f);
    const float sc = fmaxf(src, 0.0f);
    int i0 = (int)floorf(sc);
    i0 = min(i0, len_in - 1);
    const int i1 = min(i0 + 1, len_in - 1);
    float frac = i1 == i0 ? 0.0f : sub_rn(sc, (float)i0);
    frac = fminf(fmaxf(frac, 0.0f), 1.0f);
    return Tap{i0, i1, frac};
}

// resample::src_coord_align_corners (src/resample.rs:151-166).
__device__ __forceinline__ Tap align_corners_tap(int dst, int len_in, int len_out) {
    if (len_in <= 1) return Tap{0, 0, 0.0f};
    float src = len_out <= 1 ? 0.0f
                             : div_rn(mul_rn((float)dst, (float)(len_in - 1)), (float)(len_out - 1));
    src = fminf(fmaxf(src, 0.0f), (float)(len_in - 1));
    int i0 = min((int)floorf(src), len_in - 1);
    const int i1 = min(i0 + 1, len_in - 1);
    float frac = i1 == i0 ? 0.0f : sub_rn(src, (float)i0);
    frac = fminf(fmaxf(frac, 0.0f), 1.0f);
    return Tap{i0, i1, frac};
}

// A thread owns one output position (oy, ox) of a group of channels: the two
// taps are computed once (the row tap is uniform across the workgroup's row)
// and reused for every channel.  top = r0[x0]*(1-fx) + r0[x1]*fx, the same
// for the lower row, out = top*(1-fy) + bot*fy (+ add), as
// src/resample.rs:72-76 rounds them.
constexpr int kResizeChannels = 8;  // channels per thread
template <bool ALIGN>
__global__ __launch_bounds__(256) void bilinear_kernel(const float *__restrict__ in,
                                                       const float *__restrict__ add,
                                                       float *__restrict__ out, int c, int ih,
                                                       int iw, int oh, int ow, float scale_y,
                                                       float scale_x) {
    const int ox = blockIdx.x * 64 + (threadIdx.x & 63);
    const int oy = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (ox >= ow || oy >= oh) return;
    const Tap ty = ALIGN ? align_corners_tap(oy, ih, oh) : half_pixel_tap(oy, scale_y, ih);
    const Tap tx = ALIGN ? align_corners_tap(ox, iw, ow) : half_pixel_tap(ox, scale_x, iw);
    const float gx = sub_rn(1.0f, tx.frac), gy = sub_rn(1.0f, ty.frac);
    const size_t in_plane = (size_t)ih * iw, out_plane = (size_t)oh * ow;
    const size_t o00 = (size_t)ty.i0 * iw + tx.i0, o01 = (size_t)ty.i0 * iw + tx.i1;
    const size_t o10 = (size_t)ty.i1 * iw + tx.i0, o11 = (size_t)ty.i1 * iw + tx.i1;
    const size_t opos = (size_t)oy * ow + ox;
    const int c0 = blockIdx.z * kResizeChannels, c1 = min(c, c0 + kResizeChannels);
    for (int ch = c0; ch < c1; ch++) {
        const float *plane = in + (size_t)ch * in_plane;
        const float top = add_rn(mul_rn(plane[o00], gx), mul_rn(plane[o01], tx.frac));
        const float bot = add_rn(mul_rn(plane[o10], gx), mul_rn(plane[o11], tx.frac));
        float v = add_rn(mul_rn(top, gy), mul_rn(bot, ty.frac));
        const size_t e = (size_t)ch * out_plane + opos;
        if (add) v = add_rn(v, add[e]);
        out[e] = v;
    }
}

__global__ __launch_bounds__(256) void fill_kernel(float *__restrict__ p, size_t n, float v) {
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
         e += (size_t)gridDim.x * blockDim.x)
        p[e] = v;
}

unsigned grid_for(size_t total) {
    const size_t blocks = (total + 255) / 256;
    return (unsigned)(blocks < 65536 ? (blocks ? blocks : 1) : 65536);
}

}  // namespace

hipError_t launch_im2col_t(hipStream_t s, const float *in, float *col, size_t in_c, size_t ih,
                           size_t iw, size_t kh, size_t kw, size_t stride, size_t pad, size_t oh,
                           size_t ow, bool relu) {
    const size_t npix = oh * ow, K = in_c * kh * kw;
    if (npix == 0 || K == 0) return hipSuccess;
    dim3 grid((unsigned)((npix + 63) / 64), (unsigned)((K + 63) / 64));
    if (grid.y > 65535) return hipErrorInvalidValue;
    im2col_t_kernel<<<grid, 256, 0, s>>>(in, col, (int)in_c, (int)ih, (int)iw, (int)kh, (int)kw,
                                         (int)stride, (int)pad, (int)oh, (int)ow, relu ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_im2col_hwc(hipStream_t s, const float *xh, float *col, size_t in_c, size_t ih,
                             size_t iw, size_t kh, size_t kw, size_t stride, size_t pad,
                             size_t oh, size_t ow, bool relu) {
    const size_t npix = oh * ow;
    if (npix == 0 || in_c == 0) return hipSuccess;
    if (in_c % 4 != 0) return hipErrorInvalidValue;
    const unsigned blocks = (unsigned)std::min<size_t>(npix, 65536);
    im2col_hwc_kernel<<<blocks, 256, 0, s>>>(xh, col, (int)in_c, (int)ih, (int)iw, (int)kh,
                                             (int)kw, (int)stride, (int)pad, (int)oh, (int)ow,
                                             relu ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_chw_to_padded_hwc(hipStream_t s, const float *in, float *xp, size_t c,
                                    size_t ih, size_t iw, size_t pad, size_t rows, bool relu) {
    if (rows == 0 || c == 0) return hipSuccess;
    const dim3 grid((unsigned)((rows + 31) / 32), (unsigned)((c + 31) / 32));
    if (grid.y > 65535) return hipErrorInvalidValue;
    chw_to_padded_hwc_kernel<<<grid, 256, 0, s>>>(in, xp, (int)c, (int)ih, (int)iw, (int)pad,
                                                  (int)(iw + 2 * pad), (int)rows, relu ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_patch_scatter(hipStream_t s, const float *c, float *out, size_t out_c,
                                size_t ih, size_t iw, size_t kh, size_t kw) {
    const size_t total = out_c * ih * kh * iw * kw;
    if (total == 0) return hipSuccess;
    patch_scatter_kernel<<<grid_for(total), 256, 0, s>>>(c, out, (int)out_c, (int)ih, (int)iw,
                                                         (int)kh, (int)kw);
    return hipGetLastError();
}

hipError_t launch_conv_transpose_gather(hipStream_t s, const float *in, const float *w,
                                        const float *bias, float *out, size_t in_c, size_t ih,
                                        size_t iw, size_t out_c, size_t kh, size_t kw,
                                        size_t stride) {
    const size_t total = out_c * ((ih - 1) * stride + kh) * ((iw - 1) * stride + kw);
    if (total == 0 || ih == 0 || iw == 0) return hipSuccess;
    conv_transpose_gather_kernel<<<grid_for(total), 256, 0, s>>>(
        in, w, bias, out, (int)in_c, (int)ih, (int)iw, (int)out_c, (int)kh, (int)kw, (int)stride);
    return hipGetLastError();
}

hipError_t launch_bilinear(hipStream_t s, const float *in, const float *add, float *out,
                           size_t c, size_t ih, size_t iw, size_t oh, size_t ow,
                           bool align_corners) {
    const size_t total = c * oh * ow;
    if (total == 0 || ih == 0 || iw == 0) return hipSuccess;
    const dim3 grid((unsigned)((ow + 63) / 64), (unsigned)((oh + 3) / 4),
                    (unsigned)((c + kResizeChannels - 1) / kResizeChannels));
    if (grid.y > 65535 || grid.z > 65535) return hipErrorInvalidValue;
    if (align_corners) {
        bilinear_kernel<true><<<grid, 256, 0, s>>>(in, add, out, (int)c, (int)ih, (int)iw,
                                                   (int)oh, (int)ow, 0.0f, 0.0f);
    } else {
        // scale = len_in / len_out in f32 (src/resample.rs:26-27), correctly
        // rounded on the host.
        const float sy = (float)ih / (float)oh, sx = (float)iw / (float)ow;
        bilinear_kernel<false><<<grid, 256, 0, s>>>(in, add, out, (int)c, (int)ih, (int)iw,
                                                    (int)oh, (int)ow, sy, sx);
    }
    return hipGetLastError();
}

hipError_t launch_fill(hipStream_t s, float *p, size_t n, float v) {
    if (n == 0) return hipSuccess;
    fill_kernel<<<grid_for(n), 256, 0, s>>>(p, n, v);
    return hipGetLastError();
}

}  // namespace vh
