// Host-side launchers of the gfx950 kernels.  Shapes are validated by the
// C ABI layer (runtime.hip) before any of these is called; each launcher
// only maps a validated shape onto a grid and returns the launch status.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace vh {

// ---- elementwise / layout (k_elementwise.hip) ----------------------------
hipError_t launch_add(hipStream_t s, float *dst, const float *src, size_t n);
hipError_t launch_bias_scale(hipStream_t s, float *v, const float *bias, const float *gamma,
                             size_t rows, size_t cols);
hipError_t launch_gelu(hipStream_t s, float *v, size_t n);
hipError_t launch_layernorm(hipStream_t s, const float *in, const float *gamma,
                            const float *beta, float *out, size_t rows, size_t cols, float eps);
hipError_t launch_layernorm_cpu_order(hipStream_t s, const float *in, const float *gamma,
                                      const float *beta, float *out, size_t rows, size_t cols,
                                      float eps);
hipError_t launch_split_qkv(hipStream_t s, const float *qkv, float *q, float *k, float *v,
                            size_t tokens, size_t heads, size_t head_dim);
hipError_t launch_hnd_to_token(hipStream_t s, const float *hnd, float *out, size_t tokens,
                               size_t heads, size_t head_dim);
hipError_t launch_token_to_chw(hipStream_t s, const float *tm, float *chw, size_t tokens,
                               size_t channels);
hipError_t launch_patchify(hipStream_t s, const float *image, float *patches, size_t height,
                           size_t width, size_t patch, size_t channels);
hipError_t launch_prepend_cls_add_pos(hipStream_t s, const float *patches, const float *cls,
                                      const float *pos, float *out, size_t patch_count,
                                      size_t embed);
// rot: [n][2][head_dim/4][sin, cos]
hipError_t launch_rope2d(hipStream_t s, float *x, size_t heads, size_t n, size_t head_dim,
                         const float *rot);
// rot: [tokens][2][16][sin, cos]; rows = heads*tokens rows of 64
hipError_t launch_qk_norm_rope(hipStream_t s, float *q, float *k, const float *qg,
                               const float *qb, const float *kg, const float *kb,
                               const float *rot, size_t rows, size_t tokens, float eps);
// Table for qk_norm_rope from device f32 positions [tokens][2].
hipError_t launch_rope_table_device(hipStream_t s, const float *pos, size_t tokens, float freq,
                                    float *rot);
hipError_t launch_transpose(hipStream_t s, const float *in, float *out, size_t rows,
                            size_t cols);
// Streaming copy of n floats (non-temporal, four float4 per thread in
// flight) for 16-byte-aligned, non-overlapping runs of at least 128 MiB.
bool stream_copy_applies(float *dst, const float *src, size_t n);
hipError_t launch_stream_copy(hipStream_t s, float *dst, const float *src, size_t n);

// ---- attention (k_attention.hip) ----------------------------------------
// Head dims below 64 through the flash kernel: q/k/v rows of hd floats
// widened to 64 with zeros (pq/pk/pv [rows][64]), and the first hd columns
// of [rows][64] packed back into [rows][hd].
hipError_t launch_pad_rows64(hipStream_t s, const float *q, const float *k, const float *v,
                             float *pq, float *pk, float *pv, size_t rows, size_t hd);
hipError_t launch_unpad_rows(hipStream_t s, const float *src, float *dst, size_t rows, size_t hd);
// fp32-MFMA flash attention, head_dim 64, softmax scale 1/8 by default
// (1/sqrt(hd) for zero-padded rows of hd < 64).  q/k/v [bh][tokens][64]
// with bh = images*heads; out head-major or token-major [img][tokens][heads*64].
// Key splits across workgroups need a workspace of flash_workspace_floats()
// floats; with ws == nullptr (or too small) the kernel runs unsplit.
constexpr int kMaxFlashSplits = 4;
size_t flash_workspace_floats(size_t bh, size_t tokens);
// With cnt (flash_query_groups() counters, zero on entry, left zero) and a
// workspace of flash_fused_workspace_floats() floats, the split that ends
// last in each 64-query group merges the group in the kernel (bit-identical
// to the merge launch that runs otherwise).
size_t flash_query_groups(size_t bh, size_t tokens);
size_t flash_fused_workspace_floats(size_t bh, size_t tokens);
// With q8_qs / q8_d (token-major only) a run that splits the keys writes its
// output as block-major Q8_0 rows [images*tokens][heads*64] from the merge
// (bit-identical to the f32 output quantised) and sets *quantized; otherwise
// the f32 output is written and *quantized is false.
hipError_t launch_flash_attention(hipStream_t s, const float *q, const float *k, const float *v,
                                  float *out, size_t bh, size_t tokens, size_t heads,
                                  bool token_major, float *ws, size_t ws_floats,
                                  int8_t *q8_qs = nullptr, uint16_t *q8_d = nullptr,
                                  bool *quantized = nullptr, float softmax_scale = 0.125f,
                                  unsigned *cnt = nullptr, size_t cnt_n = 0);

// ---- DPT head (k_dpt.hip) ------------------------------------------------
// colT [oh*ow][in_c*kh*kw] of a CHW input (zero padding; ReLU on the input
// values when relu).
hipError_t launch_im2col_t(hipStream_t s, const float *in, float *col, size_t in_c, size_t ih,
                           size_t iw, size_t kh, size_t kw, size_t stride, size_t pad, size_t oh,
                           size_t ow, bool relu);
// colT [oh*ow][kh*kw*in_c] from a channel-last input xh [ih*iw][in_c]
// (in_c % 4 == 0), k ordered (ky, kx, ic); ReLU on the input when relu.
hipError_t launch_im2col_hwc(hipStream_t s, const float *xh, float *col, size_t in_c, size_t ih,
                             size_t iw, size_t kh, size_t kw, size_t stride, size_t pad,
                             size_t oh, size_t ow, bool relu);
// CHW -> zero-padded channel-last xp [rows][c] on the (ih + 2 pad) x
// (iw + 2 pad) grid (rows past the grid are zeros; ReLU when relu).
hipError_t launch_chw_to_padded_hwc(hipStream_t s, const float *in, float *xp, size_t c,
                                    size_t ih, size_t iw, size_t pad, size_t rows, bool relu);
// c [ih*iw][out_c*kh*kw] -> out [out_c][ih*kh][iw*kw] (kernel == stride).
hipError_t launch_patch_scatter(hipStream_t s, const float *c, float *out, size_t out_c,
                                size_t ih, size_t iw, size_t kh, size_t kw);
// Transposed convolution of any kernel and stride (IOHW weight), gathered
// per output element; bias may be null.
hipError_t launch_conv_transpose_gather(hipStream_t s, const float *in, const float *w,
                                        const float *bias, float *out, size_t in_c, size_t ih,
                                        size_t iw, size_t out_c, size_t kh, size_t kw,
                                        size_t stride);
// Bilinear resize of c CHW planes (half-pixel centres or align-corners), then
// + add (same shape as out) when add is non-null.
hipError_t launch_bilinear(hipStream_t s, const float *in, const float *add, float *out,
                           size_t c, size_t ih, size_t iw, size_t oh, size_t ow,
                           bool align_corners);
// p[0..n) = v (a kernel, so that it may sit in a captured graph).
hipError_t launch_fill(hipStream_t s, float *p, size_t n, float v);

// ---- GEMM (k_gemm.hip) ----------------------------------------------------
enum class Epi : int { Store = 0, Gelu = 1, Residual = 2, Qkv = 3 };

struct GemmArgs {
    const float *a;  // [m][k] row-major
    const float *bt; // [n][k] row-major (weights pre-transposed)
    size_t m, n, k;
    Epi epi;
    float *c;            // Store / Gelu / Residual: [m][n]
    const float *bias;   // [n] or null
    const float *gamma;  // [n] or null (Store, Residual)
    // Qkv: outputs [images][heads][tokens][64]; rot [tokens][2][16][2] or null
    float *q, *k_out, *v;
    size_t tokens, heads;
    const float *rot;
    // split-K workspace (>= splits * m * n floats) or null (no split)
    float *ws;
    size_t ws_floats;
    // Balanced-tail workspace (Store / Gelu on the 64 x 64 tile): when the
    // tiles do not divide evenly over the CUs, the tiles past the last whole
    // round run as K pieces summed by the last piece to finish.  tail_ws holds
    // their partials (kTailTiles * 4 * 4096 floats), tail_cnt one counter per
    // tail tile (kTailTiles, zero on entry and on return).  Null: no tail.
    // Launches sharing one tail_cnt must not overlap in time.
    float *tail_ws = nullptr;
    size_t tail_ws_floats = 0;
    unsigned *tail_cnt = nullptr;
    size_t tail_cnt_n = 0;
    // Per-row LayerNorm sums of LayerNorm-folded tail pieces (kTailStatFloats).
    float *tail_stats = nullptr;
    // Gelu / Qkv only: a is the raw input of a pre-norm sub-layer and the
    // GEMM computes LayerNorm(a) . W^T + b as rstd * (a . bt^T - mean * c) +
    // bias, with bt = W diag(ln gamma), ln_fold_c = c[n] = sum_k bt[n][k] and
    // bias = b + W . ln beta prepared by the caller; the row statistics are
    // taken inside the GEMM (epsilon ln_fold_eps).  K % 64 == 0.
    const float *ln_fold_c = nullptr;
    float ln_fold_eps = 0.0f;
    // Row statistics per chunk of equal-width column ranges, (mean, M2)
    // float pairs [m][chunks]: a Residual GEMM with stats_out (room for
    // m * n / 16 pairs) writes them for the rows it updates when its tile
    // allows, and reports the chunks per row in *stats_out_chunks (0: none
    // written); a LayerNorm-folded GEMM with stats_in (stats_in_chunks per
    // row, k a multiple of it) takes its row statistics from them instead of
    // from its A slices.
    float *stats_out = nullptr;
    int *stats_out_chunks = nullptr;
    const float *stats_in = nullptr;
    size_t stats_in_chunks = 0;
    // Residual only: also write LayerNorm(c) row by row to ln_out (the next
    // sub-layer's input), fused into the split-K reduction when possible.
    const float *ln_gamma = nullptr, *ln_beta = nullptr;
    float *ln_out = nullptr;
    float ln_eps = 0.0f;
    // Implicit stride-1 convolution (Store only): a is the weight
    // [out_c][kh][kw][conv_in_c] (m = out_c, k = tap * conv_in_c + ic, tap =
    // ky * conv_kw + kx), bt is a zero-padded channel-last image
    // [rows][conv_in_c] of row width conv_wp, and n counts output positions
    // on that padded grid (n = oh * conv_wp); Bt row n of tap (ky, kx) is
    // image row n + ky * conv_wp + kx, so the image needs (kh - 1) * conv_wp
    // + conv_kw - 1 rows past n.  c receives the CHW output [m][oh][conv_ow]
    // (bias per output channel; the conv_wp - conv_ow junk columns are not
    // stored).  conv_in_c must be a multiple of 32.
    size_t conv_in_c = 0, conv_kw = 0, conv_wp = 0, conv_ow = 0;
    // Direct convolution of a CHW image (Store only, set conv_ih): bt is the
    // image [conv_in_c][conv_ih][conv_iw] itself, n = oh * conv_ow output
    // pixels, k = kh * conv_kw * conv_in_c (conv_in_c % 32 == 0), stride
    // conv_stride, zero padding conv_pad, ReLU on the image when conv_relu;
    // a and c as above (c = CHW [m][oh][conv_ow], no junk columns).
    size_t conv_ih = 0, conv_iw = 0, conv_stride = 0, conv_pad = 0;
    bool conv_relu = false;
    // Patch scatter of a kernel == stride transposed convolution (Store
    // only, k % 32 == 0): a is the weight [out_c * kh * kw][k], bt the
    // channel-last input [ih * iw][k] (n = ih * iw), and C[(oc * kh + ky) * kw
    // + kx][iy * iw + ix] + bias[row] goes to the CHW output
    // c[oc][iy * kh + ky][ix * kw + kx].  With scatter_chw, bt is the CHW
    // input [k][ih * iw] itself, read in place (no channel-last copy).
    size_t scatter_kh = 0, scatter_kw = 0, scatter_iw = 0;
    bool scatter_chw = false;
};
hipError_t launch_gemm(hipStream_t s, const GemmArgs &g);
// Sizes of the balanced-tail workspace (GemmArgs::tail_ws / tail_cnt).
constexpr size_t kTailTiles = 512;
constexpr size_t kTailFloats = kTailTiles * 4 * 64 * 64;
constexpr size_t kTailStatFloats = kTailTiles * 4 * 4 * 256;

// ---- Q8_0 (k_q8.hip) --------------------------------------------------------
// x [rows][k] -> block-major Q8_0: qs [k/32][rows][32] int8, d [k/32][rows] f16 bits
hipError_t launch_quantize_q8_0(hipStream_t s, const float *x, int8_t *qs, uint16_t *d,
                                size_t rows, size_t k);
// LayerNorm of each row straight into block-major Q8_0 (bit-identical to
// launch_layernorm then launch_quantize_q8_0); cols % 32 == 0, cols <= 1024.
hipError_t launch_layernorm_q8_0(hipStream_t s, const float *x, const float *gamma,
                                 const float *beta, int8_t *qs, uint16_t *d, size_t rows,
                                 size_t cols, float eps);
// c = a . b^T block by block (exact int sums, block-order f32 fold), then the
// epilogue (Store / Gelu / Residual, see k_q8.hip); bias / gamma may be null.
hipError_t launch_gemm_q8_0(hipStream_t s, const int8_t *a_qs, const uint16_t *a_d,
                            const int8_t *b_qs, const uint16_t *b_d, float *c, size_t m,
                            size_t n, size_t k, Epi epi = Epi::Store, const float *bias = nullptr,
                            const float *gamma = nullptr, int8_t *q8_qs = nullptr,
                            uint16_t *q8_d = nullptr, bool *quantized = nullptr);
// (Gelu with q8_qs / q8_d: when the tile allows, the GELU output is written
// as block-major Q8_0 rows, bit-identical to the f32 output quantised, and
// *quantized is set; otherwise c receives f32 and *quantized is false.)
// The QKV projection in Q8_0 (n = 3*heads*64): bias, then q/k/v head-major
// [img][head][token][64] with the 2-D RoPE of q and k when rot is non-null
// (rot [tokens][2][16][sin, cos]); m must be a multiple of tokens.
hipError_t launch_gemm_q8_0_qkv(hipStream_t s, const int8_t *a_qs, const uint16_t *a_d,
                                const int8_t *b_qs, const uint16_t *b_d, size_t m, size_t k,
                                const float *bias, float *q, float *kk, float *v, size_t tokens,
                                size_t heads, const float *rot);

}  // namespace vh
