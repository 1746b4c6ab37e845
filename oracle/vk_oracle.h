/*
 * vk_oracle.h -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of the hoppworks/vestra-kernels hot-path kernels (scalar
 * oracles and the AVX-512 production CPU path) used as the parity checker
 * for the HIP backend and as the reported CPU baseline.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library.  The HIP product path never links or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative
 * to the reference crate root).  Arithmetic is restated op for op: the file
 * is compiled with -ffp-contract=off, FMAs appear only where the reference
 * uses _mm512_fmadd_ps / fnmadd, and libm calls (expf, sinf, cosf, powf,
 * sqrtf) are the platform glibc ones that Rust's std calls on Linux.
 */
#ifndef VK_ORACLE_H
#define VK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/lib.rs:29-38: #[repr(C)] struct BlockQ8_0 { d: f16, qs: [i8; 32] } (34 bytes). */
#define VKO_QK8_0 32
typedef struct vko_block_q8_0 {
    uint16_t d; /* IEEE binary16 bits */
    int8_t qs[VKO_QK8_0];
} vko_block_q8_0;

/* ---- capability / threading ------------------------------------------- */
int vko_has_avx512(void);        /* avx512f+bw+vnni+fma, src/dispatch.rs:34-48 */
void vko_set_threads(int n);     /* <=0 restores the default (all cores) */
void vko_force_scalar(int on);   /* 1: take the reference's non-AVX-512 paths */
int vko_get_threads(void);
/* Rust f32::max: the other operand when one is NaN (any NaN). */
float vko_rust_max(float a, float b);

/* ---- f16 (half 2.7.1 from_f32/to_f32: IEEE round-to-nearest-even) ------ */
uint16_t vko_f32_to_f16(float x);
float vko_f16_to_f32(uint16_t h);
uint16_t vko_f32_to_f16_hw(float x); /* F16C vcvtps2ph imm 0 (RNE); pins the software path */
uint64_t vko_f16_sweep(uint32_t step);  /* mismatches of software vs F16C over a sweep */

/* ---- scalar oracles (src/scalar.rs) ------------------------------------ */
void vko_gemm_f32(size_t m, size_t n, size_t k, const float *a, const float *b, float *c);
void vko_gemm_q8_0(size_t m, size_t n, size_t k, const vko_block_q8_0 *a_q,
                   const vko_block_q8_0 *b_q, float *c);
void vko_add(float *dst, const float *src, size_t n);
void vko_add_bias_rows(float *x, size_t rows, size_t cols, const float *bias);
void vko_layernorm(float *x, size_t rows, size_t cols, const float *gamma, const float *beta,
                   float eps);
float vko_erf(float x);
void vko_gelu(float *x, size_t n);
void vko_layerscale(float *x, size_t rows, size_t cols, const float *gamma);
void vko_softmax_rows(float *x, size_t rows, size_t cols);

/* ---- Q8_0 (src/q8_0_dot.rs, src/lib.rs) -------------------------------- */
void vko_quantize_row_q8_0(const float *x, size_t nblocks, vko_block_q8_0 *out);
void vko_dequantize_q8_0(const vko_block_q8_0 *blocks, size_t nblocks, float *out);
void vko_gemm_q8_0_avx512(size_t m, size_t n, size_t k, const vko_block_q8_0 *a_q,
                          const vko_block_q8_0 *b_q, float *c);
/* Kernels::gemm_q8_0 dispatch (src/dispatch.rs:91-105). */
void vko_kernels_gemm_q8_0(size_t m, size_t n, size_t k, const vko_block_q8_0 *a_q,
                           const vko_block_q8_0 *b_q, float *c);

/* Cephes exp of src/simd_avx512.rs:22-69, one lane in scalar code. */
float vko_cephes_exp(float x);

/* ---- AVX-512 elementwise (src/simd_avx512.rs) + Kernels dispatch -------- */
void vko_gelu_avx512(float *x, size_t n);
void vko_gelu_avx512_lanes(float *x, size_t n); /* same arithmetic in scalar code */
void vko_kernels_gelu(float *x, size_t n); /* src/dispatch.rs:56-73 */
void vko_kernels_add(float *dst, const float *src, size_t n);

/* ---- RoPE (src/rope.rs, src/specialized.rs:273-454) --------------------- */
void vko_rope2d(float *x, size_t heads, size_t n, size_t head_dim, const int64_t *pos_yx,
                float freq);
/* rotations[(token*2*16 + axis*16 + i)*2 + {0: sin, 1: cos}], src/specialized.rs:389-410 */
void vko_rope_rotations(const int64_t *pos_yx, size_t tokens, float freq, float *rotations);
void vko_qk_norm_rope(float *q, float *k, size_t heads, size_t tokens, const float *q_gamma,
                      const float *q_beta, const float *k_gamma, const float *k_beta,
                      const int64_t *pos_yx, float freq, float eps);

/* ---- attention (src/attention.rs, src/specialized.rs:1302-2744) --------- */
void vko_attention_naive(const float *q, const float *k, const float *v, size_t heads, size_t n,
                         size_t head_dim, float *out);
/* attention_serial: every row through attention_row with use_avx512=false. */
void vko_attention_serial(const float *q, const float *k, const float *v, size_t heads, size_t n,
                          size_t head_dim, float *out);
/* attention(): DA3 flash gate, else rows with the AVX-512 helpers when present. */
void vko_attention(const float *q, const float *k, const float *v, size_t heads, size_t n,
                   size_t head_dim, float *out);
/* The DA3 flash arithmetic, one row at a time in scalar code (strict form). */
void vko_flash_attention_scalar(const float *q, const float *k, const float *v, size_t heads,
                                size_t tokens, float *out);
/* The production QT8 / 8x32 AVX-512 flash path (src/specialized.rs:1906-2258). */
int vko_flash_attention_avx512(const float *q, const float *k, const float *v, size_t heads,
                               size_t tokens, float *out);

/* ---- DA3 projections (src/specialized.rs:770-1300) ---------------------- */
/* C = A.B, FMA chain over k ascending; scalar fmaf form and AVX-512 form. */
void vko_linear_fma_scalar(size_t m, size_t n, size_t k, const float *a, const float *b,
                           float *c);
void vko_linear(size_t m, size_t n, size_t k, const float *a, const float *b, float *c);
void vko_linear_bias_scale(size_t m, size_t n, size_t k, const float *a, const float *b,
                           const float *bias, const float *scale, float *c);
/* QKV projection with bias, written head-major into q/k/v[heads][m][64]. */
void vko_qkv(size_t m, const float *a, const float *w, const float *bias, float *q, float *k,
             float *v);

/* ---- layout helpers (src/cuda.rs:243-334 semantics) -------------------- */
void vko_split_qkv_hnd(const float *qkv, size_t tokens, size_t heads, size_t head_dim, float *q,
                       float *k, float *v);
void vko_hnd_to_token(const float *hnd, size_t tokens, size_t heads, size_t head_dim,
                      float *token_major);

/* ---- DA3-BASE ViT block / encoder (engine composition, reconstructed) --- */
typedef struct vko_block_weights {
    const float *ln1_gamma, *ln1_beta;  /* [768] */
    const float *w_qkv, *b_qkv;         /* [768*2304], [2304] */
    const float *w_proj, *b_proj;       /* [768*768], [768] */
    const float *ls1;                   /* [768] */
    const float *ln2_gamma, *ln2_beta;  /* [768] */
    const float *w_fc1, *b_fc1;         /* [768*3072], [3072] */
    const float *w_fc2, *b_fc2;         /* [3072*768], [768] */
    const float *ls2;                   /* [768] */
    /* DA3 late blocks: LayerNorm of each 64-wide Q and K head row before the
     * RoPE (qk_norm_rope_f32_da3_base, src/specialized.rs:278-316); all NULL
     * for a plain block. */
    const float *q_norm_gamma, *q_norm_beta, *k_norm_gamma, *k_norm_beta; /* [64] */
} vko_block_weights;

/* x: [images*tokens*768] token-major, updated in place.  pos_yx: [tokens*2]
 * (shared by all images) or NULL for no RoPE.  The optional taps (each may be
 * NULL) receive intermediates for every image, token-major:
 * tap_ln1 [images*tokens*768] = LayerNorm-1 output, tap_attn [same] = the
 * attention output before the out-projection, tap_gelu
 * [images*tokens*3072] = the fc1 output after bias and GELU.  They let a
 * parity test check the branches before LayerScale (1e-5) shrinks them. */
void vko_vit_block(float *x, size_t images, size_t tokens, const vko_block_weights *w,
                   const int64_t *pos_yx, float rope_freq, float eps, float *tap_ln1,
                   float *tap_attn, float *tap_gelu);
/* The same block with Q8_0 projections: every projection input is quantised
 * with quantize_row_q8_0 (src/q8_0_dot.rs:27-46), each weight W [k][n] as the
 * rows of W^T, the product is Kernels::gemm_q8_0 (src/dispatch.rs:91-105),
 * and bias / LayerScale / GELU follow as separate f32 passes
 * (add_bias_rows, layerscale, Kernels::gelu).  The QKV product gets its bias
 * and is then split head-major.  The engine-level composition is this
 * backend's own; the crate has no Q8_0 block. */
void vko_vit_block_q8_0(float *x, size_t images, size_t tokens, const vko_block_weights *w,
                        const int64_t *pos_yx, float rope_freq, float eps, float *tap_ln1,
                        float *tap_attn, float *tap_gelu);

/* glibc 2.35's expf algorithm restated (the device's gelu_scalar_form uses
 * the same arithmetic): the value, one entry of its 2^(i/32) table, and the
 * number of sampled inputs (every step-th bit pattern) where it differs from
 * the host's expf. */
float vko_expf_glibc_form(float x);
uint64_t vko_exp2f_table_entry(int i);
uint64_t vko_expf_form_mismatches(uint32_t step);

/* ---- DPT head (src/conv.rs, src/resample.rs); batch-1 CHW ------------- */
/* conv2d_naive (src/conv.rs:950-998): weight OIHW, bias [out_c] or NULL,
 * oh = (ih + 2*pad - kh)/stride + 1. */
void vko_conv2d_naive(const float *input, size_t in_c, size_t ih, size_t iw, const float *weight,
                      size_t out_c, size_t kh, size_t kw, size_t stride, size_t pad,
                      const float *bias, float *out);
/* Winograd F(2x2, 3x3), the crate's CPU route for 3x3 stride-1 pad-1
 * convolutions (conv::conv2d, src/conv.rs:897-900): the filter transform
 * (src/conv.rs:121-173) into u [16][in_c][out_c], then the tiled convolution
 * (src/conv.rs:681-829) with the AVX-512 product of src/specialized.rs:597-633
 * (or the crate's scalar product).  out [out_c][ih][iw]. */
void vko_winograd_f2_filter(const float *weight, size_t in_c, size_t out_c, float *u);
void vko_conv3x3_winograd_f2(const float *input, size_t in_c, size_t ih, size_t iw,
                             const float *u, size_t out_c, const float *bias, int relu_input,
                             float *out);
/* 1: the AVX-512 product restated lane by lane with fmaf (bitwise check). */
void vko_winograd_use_lanes(int on);
/* conv_transpose2d (src/conv.rs:1009-1098) with its three routes; weight
 * IOHW, oh = (ih-1)*stride + kh. */
void vko_conv_transpose2d(const float *input, size_t in_c, size_t ih, size_t iw,
                          const float *weight, size_t out_c, size_t kh, size_t kw, size_t stride,
                          const float *bias, float *out);
/* The gather-form test oracle of src/conv.rs:1646-1704. */
void vko_conv_transpose2d_naive(const float *input, size_t in_c, size_t ih, size_t iw,
                                const float *weight, size_t out_c, size_t kh, size_t kw,
                                size_t stride, const float *bias, float *out);
/* src/resample.rs: half-pixel (table and per-element forms) and align-corners. */
void vko_bilinear_resize(const float *input, size_t c, size_t ih, size_t iw, size_t oh, size_t ow,
                         float *out);
void vko_bilinear_resize_naive(const float *input, size_t c, size_t ih, size_t iw, size_t oh,
                               size_t ow, float *out);
void vko_bilinear_resize_align_corners(const float *input, size_t c, size_t ih, size_t iw,
                                       size_t oh, size_t ow, float *out);

#ifdef __cplusplus
}
#endif
#endif
