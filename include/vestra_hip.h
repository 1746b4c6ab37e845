/*
 * vestra_hip.h -- C ABI of the MI355X (gfx950) HIP backend for the DA3-BASE
 * ViT encoder hot path of hoppworks/vestra-kernels.
 *
 * The surface mirrors the crate's device API (`src/cuda.rs`): a runtime that
 * owns one device and one ordered stream (CudaRuntime), opaque device-resident
 * f32 tensors (CudaTensorF32), prepared projection weights (CudaLinearF32) and
 * a status code per CudaError variant.  Every entry point cites the reference
 * item it replaces.  Signatures use plain pointers and sizes only.
 *
 * Conventions
 *  - Every call validates its arguments before any HIP call; on failure it
 *    returns a non-zero vh_status, leaves outputs untouched and records a
 *    thread-local message readable with vh_last_error().
 *  - All device work is ordered on the runtime's stream and asynchronous;
 *    vh_download_f32 / vh_q8_0_download / vh_runtime_synchronize synchronise.
 *  - A runtime may be shared between host threads only with external
 *    synchronisation (the reference's `&self` methods have the same rule).
 *  - Tensors created by an entry point (out-parameters) are owned by the
 *    caller and released with vh_tensor_free.
 *  - Sizes are size_t end to end: there is no 2^32-element limit.
 */
#ifndef VESTRA_HIP_H
#define VESTRA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* CudaError (src/cuda.rs:337-354), one code per variant. */
typedef enum vh_status {
    VH_OK = 0,
    VH_ERR_INITIALIZE = 1,      /* CudaError::Initialize { device, detail } */
    VH_ERR_UPLOAD = 2,          /* CudaError::Upload(String) */
    VH_ERR_DOWNLOAD = 3,        /* CudaError::Download(String) */
    VH_ERR_LENGTH_MISMATCH = 4, /* CudaError::LengthMismatch { destination, source_len } */
    VH_ERR_KERNEL = 5,          /* CudaError::Kernel(String): bad shape or launch failure */
    VH_ERR_BLAS = 6,            /* CudaError::Blas(String): GEMM / linear shape errors */
    VH_ERR_INVALID_ARGUMENT = 7 /* null handle or pointer (unrepresentable in the Rust API) */
} vh_status;

typedef struct vh_runtime vh_runtime;     /* CudaRuntime (src/cuda.rs:357-379) */
typedef struct vh_tensor vh_tensor;       /* CudaTensorF32 (src/cuda.rs:1283-1286) */
typedef struct vh_linear vh_linear;       /* CudaLinearF32 (src/cuda.rs:1291-1298) */
typedef struct vh_q8_tensor vh_q8_tensor; /* device rows of BlockQ8_0 (src/lib.rs:33-38) */
typedef struct vh_block vh_block;         /* prepared DA3-BASE encoder block */
typedef struct vh_linear_q8 vh_linear_q8; /* projection with BlockQ8_0 weights */
typedef struct vh_conv2d vh_conv2d;       /* prepared 2-D convolution (DPT head) */
typedef struct vh_conv_transpose2d vh_conv_transpose2d; /* prepared transposed convolution */

/* ---- errors --------------------------------------------------------------- */
/* Message of the calling thread's last failure ("" if none). */
const char *vh_last_error(void);
/* The two lengths carried by the last VH_ERR_LENGTH_MISMATCH
 * (CudaError::LengthMismatch { destination, source_len }). */
void vh_last_length_mismatch(size_t *destination, size_t *source_len);

/* ---- runtime: CudaRuntime::new / device / stream / Clone / Drop ----------- */
/* src/cuda.rs:383-465: binds `device`, creates its ordered stream. */
vh_status vh_runtime_new(size_t device, vh_runtime **out);
/* src/cuda.rs:357 #[derive(Clone)]: shares the same device and stream. */
vh_status vh_runtime_clone(const vh_runtime *rt, vh_runtime **out);
void vh_runtime_free(vh_runtime *rt);
/* src/cuda.rs:467-470 */
size_t vh_runtime_device(const vh_runtime *rt);
/* src/cuda.rs:1276-1279 stream(): the hipStream_t every operation uses. */
void *vh_runtime_stream(const vh_runtime *rt);
/* Blocks until all work queued on the runtime's stream has finished. */
vh_status vh_runtime_synchronize(const vh_runtime *rt);

/* ---- tensors -------------------------------------------------------------- */
/* src/cuda.rs:474-483 upload_f32 */
vh_status vh_upload_f32(const vh_runtime *rt, const float *values, size_t len, vh_tensor **out);
/* src/cuda.rs:487-491 download_f32: synchronising; out_len must equal len. */
vh_status vh_download_f32(const vh_runtime *rt, const vh_tensor *tensor, float *out,
                          size_t out_len);
/* Uninitialised device tensor of `len` floats (caller-provided output buffers). */
vh_status vh_tensor_alloc(const vh_runtime *rt, size_t len, vh_tensor **out);
void vh_tensor_free(vh_tensor *tensor);
/* src/cuda.rs:1349-1356 len / is_empty */
size_t vh_tensor_len(const vh_tensor *tensor);
int vh_tensor_is_empty(const vh_tensor *tensor);
/* Raw device address, for interop with other device libraries. */
float *vh_tensor_device_ptr(const vh_tensor *tensor);

/* ---- copies / residual (src/cuda.rs:496-654) ------------------------------ */
vh_status vh_copy_f32(const vh_runtime *rt, const vh_tensor *source, vh_tensor **out);
vh_status vh_copy_segment_f32(const vh_runtime *rt, const vh_tensor *source, size_t source_offset,
                              size_t len, vh_tensor **out);
vh_status vh_copy_segment_into_f32(const vh_runtime *rt, vh_tensor *destination,
                                   size_t destination_offset, const vh_tensor *source,
                                   size_t source_offset, size_t len);
vh_status vh_overwrite_prefix_f32(const vh_runtime *rt, vh_tensor *destination,
                                  const vh_tensor *source, size_t len);
/* src/cuda.rs:630-654 add_f32_in_place: destination += source. */
vh_status vh_add_f32_in_place(const vh_runtime *rt, vh_tensor *destination,
                              const vh_tensor *source);

/* ---- GEMM and epilogues --------------------------------------------------- */
/* src/cuda.rs:661-704 gemm_row_major_f32: C[m,n] = A[m,k] x B[k,n], row-major.
 * fp32 MFMA kernel (replaces cublasSgemm). */
vh_status vh_gemm_row_major_f32(const vh_runtime *rt, const vh_tensor *a, const vh_tensor *b,
                                size_t m, size_t k, size_t n, vh_tensor **out);
/* src/cuda.rs:708-742 bias_scale_f32_in_place: v = (v + bias[c]) * gamma[c]. */
vh_status vh_bias_scale_f32_in_place(const vh_runtime *rt, vh_tensor *values,
                                     const vh_tensor *bias, const vh_tensor *gamma, size_t rows,
                                     size_t columns);
/* src/cuda.rs:747-759 gelu_f32_in_place (arithmetic of Kernels::gelu,
 * src/dispatch.rs:56-73: AVX-512 erf/exp form, scalar form on the n%16 tail). */
vh_status vh_gelu_f32_in_place(const vh_runtime *rt, vh_tensor *values);

/* ---- LayerNorm ------------------------------------------------------------ */
/* src/cuda.rs:764-810 layernorm_f32 (one wave64 per row). */
vh_status vh_layernorm_f32(const vh_runtime *rt, const vh_tensor *input, const vh_tensor *gamma,
                           const vh_tensor *beta, size_t rows, size_t columns, float epsilon,
                           vh_tensor **out);
/* src/cuda.rs:815-863 layernorm_f32_cpu_order: the scalar::layernorm order,
 * bit-exact with src/scalar.rs:99-114. */
vh_status vh_layernorm_f32_cpu_order(const vh_runtime *rt, const vh_tensor *input,
                                     const vh_tensor *gamma, const vh_tensor *beta, size_t rows,
                                     size_t columns, float epsilon, vh_tensor **out);

/* ---- attention ------------------------------------------------------------ */
/* src/cuda.rs:868-922 attention_online_f32: head-major [heads,tokens,head_dim]
 * in and out, 1 <= head_dim <= 64, scale 1/sqrt(head_dim). */
vh_status vh_attention_online_f32(const vh_runtime *rt, const vh_tensor *q, const vh_tensor *k,
                                  const vh_tensor *v, size_t heads, size_t tokens,
                                  size_t head_dim, vh_tensor **out);
/* flash_attention_f32_da3_base (src/lib.rs:82-91, src/specialized.rs:730-765):
 * head_dim 64, scale 1/8, fp32-MFMA online softmax.  Any token count is
 * accepted (the reference's tokens % 865 gate is a CPU-kernel limit).
 * token_major = 0 writes head-major [heads,tokens,64]; 1 writes token-major
 * [tokens, heads*64] (the fused hnd_to_token of src/cuda.rs:984-1036). */
vh_status vh_flash_attention_f32_da3_base(const vh_runtime *rt, const vh_tensor *q,
                                          const vh_tensor *k, const vh_tensor *v, size_t heads,
                                          size_t tokens, int token_major, vh_tensor **out);
/* No counterpart in the reference.  vh_flash_attention_f32_da3_base for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc): it calls no
 * allocator.  The caller passes `out` (heads*tokens*64 floats, layout as
 * above).  The key-split partials live in a 64 MiB device array of the
 * library, one per GPU, reserved until the process ends; heads*tokens above
 * 63550 is rejected with VH_ERR_KERNEL before any launch.  Every call on a
 * GPU shares that GPU's array, and the library orders the calls in the order
 * they are made: each launch waits (hipStreamWaitEvent) for the previous
 * call's launch, on whatever runtime or stream it ran, so runtimes on
 * different streams and host threads may call it freely.  Under stream
 * capture that wait is not recorded: replays of such a graph are ordered
 * only by the caller against other uses of the array.  Results are
 * bit-identical to the allocating entry point's. */
vh_status vh_flash_attention_f32_da3_base_into(const vh_runtime *rt, const vh_tensor *q,
                                               const vh_tensor *k, const vh_tensor *v,
                                               size_t heads, size_t tokens, int token_major,
                                               vh_tensor *out);

/* ---- layout (src/cuda.rs:927-1175) ---------------------------------------- */
vh_status vh_split_qkv_hnd_f32(const vh_runtime *rt, const vh_tensor *qkv, size_t tokens,
                               size_t heads, size_t head_dim, vh_tensor **q, vh_tensor **k,
                               vh_tensor **v);
vh_status vh_hnd_to_token_f32(const vh_runtime *rt, const vh_tensor *hnd, size_t tokens,
                              size_t heads, size_t head_dim, vh_tensor **out);
vh_status vh_token_to_chw_f32(const vh_runtime *rt, const vh_tensor *token_major, size_t tokens,
                              size_t channels, vh_tensor **out);
vh_status vh_patchify_nchw_f32(const vh_runtime *rt, const vh_tensor *image, size_t height,
                               size_t width, size_t patch, size_t channels, vh_tensor **out);
vh_status vh_prepend_cls_add_pos_f32(const vh_runtime *rt, const vh_tensor *patches,
                                     const vh_tensor *cls, const vh_tensor *position,
                                     size_t patch_count, size_t embed, vh_tensor **out);

/* ---- RoPE ----------------------------------------------------------------- */
/* rope::rope2d (src/rope.rs:30-80) on a device [heads, n, head_dim] tensor.
 * pos_yx is host int64 [n*2]; the sin/cos table is built on the host with
 * the same libm calls as the reference and cached on the runtime. */
vh_status vh_rope2d_f32_in_place(const vh_runtime *rt, vh_tensor *x, size_t heads, size_t n,
                                 size_t head_dim, const int64_t *pos_yx, float frequency);
/* src/cuda.rs:1178-1228 qk_norm_rope_f32_da3_base: 64-wide rows, device
 * positions_yx f32 [tokens*2], rotation table as src/specialized.rs:389-410. */
vh_status vh_qk_norm_rope_f32_da3_base(const vh_runtime *rt, vh_tensor *q, vh_tensor *k,
                                       const vh_tensor *q_gamma, const vh_tensor *q_beta,
                                       const vh_tensor *k_gamma, const vh_tensor *k_beta,
                                       const vh_tensor *positions_yx, size_t heads,
                                       size_t tokens, float frequency, float epsilon);

/* ---- prepared projections (CudaLinearF32) --------------------------------- */
/* src/cuda.rs:1230-1268 prepare_linear_f32: weight row-major [K, N], bias [N],
 * gamma [N] or NULL (unit).  Weights are repacked once for the MFMA kernel. */
vh_status vh_prepare_linear_f32(const vh_runtime *rt, size_t input_features,
                                size_t output_features, const float *weight, const float *bias,
                                const float *gamma, vh_linear **out);
void vh_linear_free(vh_linear *linear);
size_t vh_linear_input_features(const vh_linear *linear);  /* src/cuda.rs:1301-1304 */
size_t vh_linear_output_features(const vh_linear *linear); /* src/cuda.rs:1306-1309 */
/* src/cuda.rs:1312-1334 run: (input x W + bias) * gamma, one fused launch. */
vh_status vh_linear_run(const vh_linear *linear, const vh_tensor *input, size_t rows,
                        vh_tensor **out);
/* src/cuda.rs:1340-1344 run_chw: run, then token-major -> CHW. */
vh_status vh_linear_run_chw(const vh_linear *linear, const vh_tensor *input, size_t rows,
                            vh_tensor **out);
/* run + gelu_f32_in_place fused (the fc1 step; src/gemm.rs:70-96 order:
 * GEMM, + bias, then GELU).  gamma must be unit (prepared with NULL). */
vh_status vh_linear_run_gelu(const vh_linear *linear, const vh_tensor *input, size_t rows,
                             vh_tensor **out);
/* run + add_f32_in_place fused (out-projection / fc2 with LayerScale and the
 * residual, src/specialized.rs:811-929 then src/dispatch.rs:77-83):
 * residual += (input x W + bias) * gamma. */
vh_status vh_linear_run_residual(const vh_linear *linear, const vh_tensor *input, size_t rows,
                                 vh_tensor *residual);
/* qkv_f32_da3_base (src/specialized.rs:996-1167) as a device op on a linear
 * with N = 3*heads*64: Q/K/V written head-major [images][heads][tokens][64]
 * with bias; when pos_yx (host int64 [tokens*2]) is non-NULL the 2-D RoPE of
 * src/rope.rs:30-93 is applied to Q and K in the same launch.  rows must be
 * images * tokens. */
vh_status vh_linear_run_qkv_hnd(const vh_linear *linear, const vh_tensor *input, size_t images,
                                size_t tokens, size_t heads, const int64_t *pos_yx,
                                float frequency, vh_tensor **q, vh_tensor **k, vh_tensor **v);

/* ---- Q8_0 ------------------------------------------------------------------ */
/* Rows of BlockQ8_0 ({f16 d; i8 qs[32]}, 34 bytes, src/lib.rs:33-38) held on
 * the device as separate qs and d arrays. */
vh_status vh_q8_0_upload(const vh_runtime *rt, const void *blocks, size_t rows, size_t k,
                         vh_q8_tensor **out);
/* Writes rows*k/32 BlockQ8_0 values (AoS) to `blocks`; synchronising. */
vh_status vh_q8_0_download(const vh_runtime *rt, const vh_q8_tensor *tensor, void *blocks,
                           size_t nblocks);
void vh_q8_tensor_free(vh_q8_tensor *tensor);
size_t vh_q8_tensor_rows(const vh_q8_tensor *tensor);
size_t vh_q8_tensor_k(const vh_q8_tensor *tensor);
/* quantize_row_q8_0 (src/q8_0_dot.rs:27-46) over each row of a device
 * [rows, k] f32 tensor, k % 32 == 0.  Bit-exact. */
vh_status vh_quantize_q8_0(const vh_runtime *rt, const vh_tensor *x, size_t rows, size_t k,
                           vh_q8_tensor **out);
/* quantize_row_q8_0(x, out) (src/q8_0_dot.rs:27-46) into an existing
 * [rows, k] Q8_0 tensor, as the reference writes a caller's block slice:
 * VH_ERR_LENGTH_MISMATCH ("x.len() must be out.len()*QK8_0", the reference's
 * assert) unless out holds rows x k / 32 blocks and x rows * k floats. */
vh_status vh_quantize_q8_0_into(const vh_runtime *rt, const vh_tensor *x, size_t rows, size_t k,
                                vh_q8_tensor *out);
/* Kernels::gemm_q8_0 (src/dispatch.rs:91-105, oracle src/scalar.rs:25-56):
 * C[m,n] = sum_b (d_a*d_b)*isum_b with a_q [m,k] and b_q [n,k]; int8 MFMA
 * block sums, f32 combine in block order.  Bit-exact. */
vh_status vh_gemm_q8_0(const vh_runtime *rt, const vh_q8_tensor *a_q, const vh_q8_tensor *b_q,
                       size_t m, size_t n, size_t k, vh_tensor **out);
/* Kernels::gemm_q8_0(m, n, k, a_q, b_q, c) (src/dispatch.rs:91-105) into a
 * caller's [m, n] f32 tensor, as the reference writes c: VH_ERR_LENGTH_MISMATCH
 * ("c.len() must be m * n", the reference's debug assertion,
 * src/scalar.rs:37) unless c holds m * n floats.  Bit-exact, the same kernel
 * as vh_gemm_q8_0. */
vh_status vh_gemm_q8_0_into(const vh_runtime *rt, const vh_q8_tensor *a_q, const vh_q8_tensor *b_q,
                            size_t m, size_t n, size_t k, vh_tensor *c);

/* ---- Q8_0 projections -------------------------------------------------------- */
/* A projection whose weights are GGUF-style BlockQ8_0 (src/lib.rs:33-38): the
 * pre-transposed row blocks that Kernels::gemm_q8_0 takes as its b operand
 * (src/dispatch.rs:91-105), output_features rows of input_features/32 blocks,
 * repacked block-major at prepare time.  bias and gamma ([N]) may be NULL.
 * Each run quantises the f32 input rows on the device (quantize_row_q8_0,
 * src/q8_0_dot.rs:27-46), forms the exact block-dot sums, and applies the
 * f32 epilogue as the engine's separate passes would (src/scalar.rs:65-81
 * add_bias_rows, src/scalar.rs:139-155 layerscale, src/dispatch.rs:56-83 gelu
 * and add), each op rounded as there.  Bit-exact with that composition. */
vh_status vh_prepare_linear_q8_0(const vh_runtime *rt, size_t input_features,
                                 size_t output_features, const void *weight_blocks,
                                 const float *bias, const float *gamma, vh_linear_q8 **out);
void vh_linear_q8_0_free(vh_linear_q8 *linear);
size_t vh_linear_q8_0_input_features(const vh_linear_q8 *linear);
size_t vh_linear_q8_0_output_features(const vh_linear_q8 *linear);
/* out = (gemm_q8_0(quantize(input), W) + bias) * gamma */
vh_status vh_linear_q8_0_run(const vh_linear_q8 *linear, const vh_tensor *input, size_t rows,
                             vh_tensor **out);
/* out = gelu(gemm_q8_0(quantize(input), W) + bias); gamma must be NULL. */
vh_status vh_linear_q8_0_run_gelu(const vh_linear_q8 *linear, const vh_tensor *input,
                                  size_t rows, vh_tensor **out);
/* residual += (gemm_q8_0(quantize(input), W) + bias) * gamma */
vh_status vh_linear_q8_0_run_residual(const vh_linear_q8 *linear, const vh_tensor *input,
                                      size_t rows, vh_tensor *residual);

/* ---- DA3-BASE encoder block ------------------------------------------------ */
/* Host pointers to one block's parameters, row-major [in, out] weights. */
typedef struct vh_block_params {
    const float *ln1_gamma, *ln1_beta; /* [768] */
    const float *w_qkv, *b_qkv;        /* [768*2304], [2304] */
    const float *w_proj, *b_proj;      /* [768*768], [768] */
    const float *ls1;                  /* [768] LayerScale */
    const float *ln2_gamma, *ln2_beta; /* [768] */
    const float *w_fc1, *b_fc1;        /* [768*3072], [3072] */
    const float *w_fc2, *b_fc2;        /* [3072*768], [768] */
    const float *ls2;                  /* [768] */
    /* DA3 late blocks: LayerNorm of each 64-wide Q and K head row before the
     * RoPE (qk_norm_rope_f32_da3_base, src/specialized.rs:278-316).  All four
     * NULL for a plain block, all four [64] otherwise. */
    const float *q_norm_gamma, *q_norm_beta, *k_norm_gamma, *k_norm_beta;
} vh_block_params;

/* Uploads and repacks one block's weights (model-load time). */
vh_status vh_block_prepare(const vh_runtime *rt, const vh_block_params *params, vh_block **out);
/* The same block with its four projections in Q8_0: each f32 weight W [in, out]
 * is quantised on the device as the rows of W^T (quantize_row_q8_0,
 * src/q8_0_dot.rs:27-46), and every projection quantises its input rows and
 * runs the block-dot GEMM of vh_linear_q8_0_run.  The crate has no Q8_0
 * block; this one follows the same engine composition with
 * Kernels::gemm_q8_0 (src/dispatch.rs:91-105) in place of each f32 GEMM. */
vh_status vh_block_prepare_q8_0(const vh_runtime *rt, const vh_block_params *params,
                                vh_block **out);
int vh_block_is_q8_0(const vh_block *block);
void vh_block_free(vh_block *block);
/* One pre-LN DA3-BASE block in place on x [images*tokens*768]: LN, QKV (+bias,
 * + 2-D RoPE when pos_yx != NULL; a late block first normalises each Q and K
 * head row, with all tokens at (0, 0) when pos_yx is NULL), attention,
 * out-proj (+bias, *ls1) +
 * residual, LN, fc1 (+bias, GELU), fc2 (+bias, *ls2) + residual.  The CPU
 * composition it replaces chains src/scalar.rs:83, src/specialized.rs:996,
 * src/rope.rs:30, src/attention.rs:66, src/specialized.rs:811,
 * src/dispatch.rs:77, src/specialized.rs:770, src/scalar.rs:65 and
 * src/dispatch.rs:56. */
vh_status vh_vit_block_run(const vh_runtime *rt, const vh_block *block, vh_tensor *x,
                           size_t images, size_t tokens, const int64_t *pos_yx,
                           float rope_frequency, float epsilon);
/* `layers` blocks in sequence (the 12-layer encoder). */
vh_status vh_encoder_run(const vh_runtime *rt, const vh_block *const *blocks, size_t layers,
                         vh_tensor *x, size_t images, size_t tokens, const int64_t *pos_yx,
                         float rope_frequency, float epsilon);

/* ---- DPT head: convolution, transposed convolution, resize ----------------- */
/* Batch-1 CHW tensors as in src/conv.rs and src/resample.rs.  Convolutions run
 * as fp32-MFMA GEMMs (direct convolution: the crate's 3x3 stride-1 pad-1
 * Winograd F(2x2,3x3) path is tested against the same direct definition,
 * src/conv.rs:1438-1477); results agree with conv2d_naive (src/conv.rs:950-
 * 998) within f32 accumulation error.  The resizes are bit-exact. */

/* conv2d (src/conv.rs:877-945) with the weight prepared once, as
 * prepare_winograd_f2_filter (src/conv.rs:174-177) prepares it for the CPU:
 * weight OIHW [out_c*in_c*kh*kw], bias [out_c] or NULL. */
vh_status vh_prepare_conv2d_f32(const vh_runtime *rt, size_t in_c, size_t out_c, size_t kh,
                                size_t kw, size_t stride, size_t pad, const float *weight,
                                const float *bias, vh_conv2d **out);
void vh_conv2d_free(vh_conv2d *conv);
/* oh = (ih + 2*pad - kh)/stride + 1 (0 when the kernel exceeds the padded input). */
size_t vh_conv2d_output_height(const vh_conv2d *conv, size_t ih);
size_t vh_conv2d_output_width(const vh_conv2d *conv, size_t iw);
/* input [in_c*ih*iw] -> new [out_c*oh*ow] (conv3x3_winograd_f2_prepared,
 * src/conv.rs:282-293, for any kernel, stride and padding). */
vh_status vh_conv2d_run(const vh_conv2d *conv, const vh_tensor *input, size_t ih, size_t iw,
                        vh_tensor **out);
/* The same on max(input, 0) (conv3x3_winograd_f2_prepared_relu_input,
 * src/conv.rs:651-679): the ReLU is applied while the patches are gathered. */
vh_status vh_conv2d_run_relu_input(const vh_conv2d *conv, const vh_tensor *input, size_t ih,
                                   size_t iw, vh_tensor **out);
/* conv3x3_winograd_f2_prepared_resize_align_corners (src/conv.rs:304-320):
 * align-corners resize of input [in_c*ih*iw] to oh x ow, plus add
 * [in_c*oh*ow] when non-NULL, then the convolution. */
vh_status vh_conv2d_run_resize_align_corners(const vh_conv2d *conv, const vh_tensor *input,
                                             size_t ih, size_t iw, size_t oh, size_t ow,
                                             const vh_tensor *add, vh_tensor **out);
/* conv2d (src/conv.rs:877-945) in one call: host weight OIHW, bias or NULL. */
vh_status vh_conv2d_f32(const vh_runtime *rt, const vh_tensor *input, size_t in_c, size_t ih,
                        size_t iw, const float *weight, size_t out_c, size_t kh, size_t kw,
                        size_t stride, size_t pad, const float *bias, vh_tensor **out);

/* Transposed convolution (src/conv.rs:1009-1098), weight IOHW
 * [in_c*out_c*kh*kw], bias [out_c] or NULL, oh = (ih-1)*stride + kh.  With
 * kernel == stride (the DPT resize layers) the filter is packed as
 * prepare_nonoverlap_transpose_filter does (src/conv.rs:83-93,
 * src/specialized.rs:148-174) and the op is one GEMM plus a patch scatter;
 * any other geometry gathers per output element in the order of the
 * crate's conv_transpose2d_naive (src/conv.rs:1646-1704), bit-exact with it. */
vh_status vh_prepare_conv_transpose2d_f32(const vh_runtime *rt, size_t in_c, size_t out_c,
                                          size_t kh, size_t kw, size_t stride,
                                          const float *weight, const float *bias,
                                          vh_conv_transpose2d **out);
void vh_conv_transpose2d_free(vh_conv_transpose2d *conv);
/* conv_transpose2d_prepared (src/conv.rs:95-105): input [in_c*ih*iw], ih, iw >= 1. */
vh_status vh_conv_transpose2d_run(const vh_conv_transpose2d *conv, const vh_tensor *input,
                                  size_t ih, size_t iw, vh_tensor **out);
/* conv_transpose2d (src/conv.rs:1009-1098) in one call. */
vh_status vh_conv_transpose2d_f32(const vh_runtime *rt, const vh_tensor *input, size_t in_c,
                                  size_t ih, size_t iw, const float *weight, size_t out_c,
                                  size_t kh, size_t kw, size_t stride, const float *bias,
                                  vh_tensor **out);

/* bilinear_resize (src/resample.rs:10-77): half-pixel centres, clamp to edge;
 * [c*ih*iw] -> new [c*oh*ow].  An empty input gives zeros. */
vh_status vh_bilinear_resize_f32(const vh_runtime *rt, const vh_tensor *input, size_t c,
                                 size_t ih, size_t iw, size_t oh, size_t ow, vh_tensor **out);
/* bilinear_resize_align_corners (src/resample.rs:184-245), then + add
 * [c*oh*ow] when add is non-NULL (the DPT UV-embedding add). */
vh_status vh_bilinear_resize_align_corners_f32(const vh_runtime *rt, const vh_tensor *input,
                                               size_t c, size_t ih, size_t iw, size_t oh,
                                               size_t ow, const vh_tensor *add, vh_tensor **out);

/* ---- profiling (device twin of DA3_FLASH_PROFILE, src/specialized.rs:1324) - */
/* When enabled, every kernel launch is bracketed by HIP events on the
 * runtime's stream and its duration accumulated under the kernel's name. */
vh_status vh_profile_enable(vh_runtime *rt, int enabled);
vh_status vh_profile_reset(vh_runtime *rt);
/* Synchronises, then writes "name count total_ms\n" lines (NUL-terminated,
 * truncated to buflen). */
vh_status vh_profile_report(vh_runtime *rt, char *buf, size_t buflen);
/* Stream-ordered wall clock: start records an event, stop records another,
 * synchronises and returns the elapsed milliseconds. */
vh_status vh_timer_start(vh_runtime *rt);
vh_status vh_timer_stop(vh_runtime *rt, float *elapsed_ms);

#ifdef __cplusplus
}
#endif
#endif
