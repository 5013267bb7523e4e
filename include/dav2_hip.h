/*
 * Thin C-ABI HIP launcher layer: one extern "C" entry per gfx950 kernel.
 *
 * Every entry takes raw device pointers, plain sizes and a hipStream_t passed
 * as void* (NULL = the null stream), enqueues asynchronously and returns the
 * hipError_t value as int (0 = hipSuccess; hipErrorInvalidValue = 1 for
 * rejected arguments). No entry allocates memory. The C++ operator surface
 * (dav2::HipOperators, mirroring the reference's src/operators.h) calls only
 * these; tests and FFI callers may call them directly.
 *
 * int8 matrices are row-major [rows][ld] bytes, ld a multiple of 64 and bytes
 * [K, ld) zero: the first K bytes of a row are the byte view of the
 * reference's packed 4x int8 words (quantize_rows_int8_fused.glsl:51).
 */
#ifndef DAV2_HIP_H
#define DAV2_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifndef DAV2_API
#define DAV2_API __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces quantize_rows_int8_fused.glsl:20-55 as dispatched by
 * VulkanOperators::linear_int8 (src/operators.cpp:810-818) and
 * project_tokens_int8 (:1514-1522). Row r reads input[input_offset + r*columns + c].
 * columns % 4 == 0, input_offset % 4 == 0. */
DAV2_API int dav2_hip_quantize_rows_i8(const float* input, uint64_t input_offset,
                                       uint32_t rows, uint32_t columns, int8_t* q,
                                       uint32_t ldq, float* scales, void* stream);

/* gelu.glsl:16-49 followed by quantize_rows_int8_fused.glsl:20-55 in one pass:
 * the row quantized is gelu(input row), bit for bit what the reference's
 * GELU pass after fc1 (linear_int8 with gelu, src/operators.cpp:837-843,
 * called from src/encoder.cpp:525-528) and fc2's input quantization
 * (src/operators.cpp:810-818) produce. Arguments as dav2_hip_quantize_rows_i8;
 * columns <= 4096. */
DAV2_API int dav2_hip_gelu_quantize_rows_i8(const float* input, uint64_t input_offset,
                                            uint32_t rows, uint32_t columns, int8_t* q,
                                            uint32_t ldq, float* scales, void* stream);

/* int8 weight rows of `columns` bytes -- the reference GpuModel layout,
 * [rows][columns/4] little-endian words (src/gpu_model.cpp:241-284) -- to the
 * GEMM layout [rows][ld] (ld % 16 == 0, ld >= columns), bytes [columns, ld)
 * zero. rows <= 65535. No reference counterpart (a layout conversion). */
DAV2_API int dav2_hip_pad_rows_i8(const int8_t* src, uint32_t rows, uint32_t columns, int8_t* dst, uint32_t ld,
                                  void* stream);
/* The reference's transposed int8 weight layout (src/gpu_model.cpp:241-258,
 * int8_transposed_buffer: [K][N] bytes, byte k*N + n = weight of output n,
 * input k), consumed by linear_int8(..., weight_transposed=true)
 * (src/operators.cpp:819-832), to the GEMM layout: N rows of ld bytes
 * (ld % 64 == 0, ld >= K), zero beyond K. */
DAV2_API int dav2_hip_transpose_rows_i8(const int8_t* src, uint32_t k_rows, uint32_t n_columns, int8_t* dst,
                                        uint32_t ld, void* stream);

/* Replaces im2col_quantize_int8.glsl:26-83 (src/operators.cpp:1284-1298,
 * :1787-1801, :1946-1960). CHW input; rows = output_width*output_height.
 * scratch (optional, dav2_hip_im2col_scratch_floats() floats) enables the
 * tiled 3x3-stride-1 and 1x1 kernels and, for other geometries, row scales
 * from per-pixel channel-group maxima; without it the generic gather runs.
 * All produce the same bytes. */
DAV2_API uint64_t dav2_hip_im2col_scratch_floats(uint32_t input_width, uint32_t input_height,
                                                 uint32_t input_channels);
DAV2_API int dav2_hip_im2col_quantize_i8(const float* input, uint32_t input_width,
                                         uint32_t input_height, uint32_t input_channels,
                                         uint32_t output_width, uint32_t output_height,
                                         uint32_t kernel, uint32_t stride, int32_t padding,
                                         int8_t* q, uint32_t ldq, float* scales,
                                         float* scratch, uint64_t scratch_floats, void* stream);
/* The same for max(input, 0) (relu.glsl ahead of the convolution, as the DPT
 * residual units apply it), without materialising the ReLU: any geometry on
 * maps of up to 8192 output pixels (rows of up to 9216 columns), else kernel
 * 3 / stride 1 / padding 1 (channels % 16 == 0) or kernel 1 / stride 1 /
 * padding 0 with scratch only; other calls return hipErrorInvalidValue. No
 * reference counterpart (a fusion of two reference passes). */
DAV2_API int dav2_hip_im2col_quantize_relu_i8(const float* input, uint32_t input_width,
                                              uint32_t input_height, uint32_t input_channels,
                                              uint32_t output_width, uint32_t output_height,
                                              uint32_t kernel, uint32_t stride, int32_t padding,
                                              int8_t* q, uint32_t ldq, float* scales,
                                              float* scratch, uint64_t scratch_floats, void* stream);

/* Replaces layer_norm.glsl:27-68 (src/operators.cpp:1016-1042). */
DAV2_API int dav2_hip_layer_norm(float* out, const float* input, const float* weight,
                                 const float* bias, uint32_t rows, uint32_t columns,
                                 float epsilon, void* stream);

/* layer_norm.glsl followed by quantize_rows_int8_fused.glsl in one pass (the
 * reference runs them back to back at src/encoder.cpp:443-452, :500-528);
 * out may be NULL when the fp32 row is not needed. columns <= 4096. */
DAV2_API int dav2_hip_layer_norm_quantize_i8(int8_t* q, uint32_t ldq, float* scales,
                                             float* out, const float* input,
                                             const float* weight, const float* bias,
                                             uint32_t rows, uint32_t columns,
                                             float epsilon, void* stream);

/* GEMM epilogues. Reference: linear_int8_tiled.glsl:99-116,
 * gelu.glsl:16-49, add_scaled.glsl:23-32, conv_transpose_int8.glsl:31-58. */
enum {
    DAV2_GEMM_EPI_RAW_I32 = 0,        /* out_i32[m*n + n'] = int32 accumulator        */
    DAV2_GEMM_EPI_ROW = 1,            /* out[(m+off)*n + n'] = acc*sa*sb + bias        */
    DAV2_GEMM_EPI_ROW_GELU = 2,       /* ... then exact-erf GELU                        */
    DAV2_GEMM_EPI_ROW_LAYERSCALE = 3, /* out = residual + (acc*sa*sb + bias)*gamma[n'] */
    DAV2_GEMM_EPI_TRANSPOSED = 4,     /* out[n'*stride + m + off] (channel-major), plus
                                         residual at the same index when given, then
                                         max(., 0) when relu_output                     */
    DAV2_GEMM_EPI_CONVT = 5,          /* stride==kernel ConvTranspose scatter           */
    DAV2_GEMM_EPI_ROW_COLMAX = 6      /* ROW, and per tile of rows the max |out| of each
                                         column n' >= col_absmax_begin                  */
};

typedef struct dav2_gemm_i8_args {
    const int8_t* a;        /* activations [m][lda], 16-byte aligned          */
    uint64_t lda;
    const int8_t* b;        /* weights [n][ldb], 16-byte aligned              */
    uint64_t ldb;
    uint32_t m, n, k;       /* k: multiple of 64, padding bytes zero          */
    uint32_t epilogue;      /* DAV2_GEMM_EPI_*                                */
    const float* a_scales;  /* [m] per-row activation scales                  */
    const float* b_scales;  /* [n] per-row weight scales                      */
    const float* bias;      /* [n] (CONVT: [convt_channels]) or NULL = 0      */
    int32_t* out_i32;
    float* out;
    uint64_t out_row_offset;
    uint64_t out_row_stride;
    const float* residual;  /* LAYERSCALE (may alias out) or TRANSPOSED        */
    const float* gamma;
    uint32_t convt_kernel, convt_width, convt_height, convt_channels;
    /* ROW_COLMAX: col_absmax[t][n' - col_absmax_begin] = max |out[m][n']| over
     * the rows m of row tile t (dav2_hip_gemm_i8_row_tiles() tiles); the
     * begin is a multiple of 64, n % 4 == 0 and out 16-byte aligned. */
    float* col_absmax;
    uint32_t col_absmax_begin;
    uint32_t relu_output;   /* TRANSPOSED only: max(out, 0) after the residual */
    /* TRANSPOSED only: split_k > 1 runs K in that many slices on more
     * workgroups (for GEMMs with few output tiles), their int32 sums in
     * split_scratch (dav2_hip_gemm_i8_split_scratch_bytes), then one pass
     * adds them (exact) and applies the epilogue. Same output bits. */
    uint32_t split_k;
    int32_t* split_scratch;
} dav2_gemm_i8_args;

/* Replaces linear_int8_tiled.glsl:40-117 (src/operators.cpp:847-880) and
 * conv_transpose_int8.glsl:31-58 (:1969-1975). */
DAV2_API int dav2_hip_gemm_i8(const dav2_gemm_i8_args* args, void* stream);
/* Timing hook, no reference counterpart: hipEvent_t start / stop for the
 * calling thread's next dav2_hip_gemm_i8, recorded by its kernel dispatches
 * (the GEMM's start, the last kernel's end); NULL, NULL clears. */
DAV2_API void dav2_hip_gemm_i8_events(void* start, void* stop);
/* Timing hook, no reference counterpart: hipEvent_t start / stop for the
 * calling thread's kernel dispatches: the next kernel launched records start
 * when it begins, every launch until the hook is cleared (NULL, NULL) records
 * stop when it ends, so the pair spans all kernels of an operation. Returns 1
 * when a kernel launched under the pair being replaced, 0 when none did (its
 * events then hold no record of that operation). */
DAV2_API int dav2_hip_launch_events(void* start, void* stop);

/* fp32 GEMM of the fp32 precision mode: out = a . b^T + bias with the
 * epilogues ROW, ROW_GELU, ROW_LAYERSCALE, TRANSPOSED (residual, relu_output)
 * and CONVT of the int8 GEMM. a [m][lda], b [n][ldb] float32, 16-byte
 * aligned, k, lda, ldb multiples of 4 (pad columns with zeros).
 * Replaces linear_tiled.glsl / linear_vec*.glsl (src/operators.cpp:882-955),
 * the GEMM of conv2d (:1528-1676), conv_transpose_nonoverlap (:1807-1861) and
 * project_tokens (:1408-1452). */
typedef struct dav2_gemm_f32_args {
    const float* a;
    uint64_t lda;
    const float* b;
    uint64_t ldb;
    uint32_t m, n, k;
    uint32_t epilogue;      /* DAV2_GEMM_EPI_* (not RAW_I32 / ROW_COLMAX)      */
    const float* bias;      /* [n] (CONVT: [convt_channels]) or NULL = 0      */
    float* out;
    uint64_t out_row_offset;
    uint64_t out_row_stride;
    const float* residual;  /* LAYERSCALE (may alias out) or TRANSPOSED        */
    const float* gamma;
    uint32_t convt_kernel, convt_width, convt_height, convt_channels;
    uint32_t relu_output;   /* TRANSPOSED only                                 */
    /* 1: both operands rounded to binary16 before the (exact) products, fp32
     * accumulation: the fp16 mode's cooperative-matrix linears
     * (linear_coop_fp16.glsl, src/operators.cpp:540-768). 0: fp32. */
    uint32_t half_operands;
} dav2_gemm_f32_args;
DAV2_API int dav2_hip_gemm_f32(const dav2_gemm_f32_args* args, void* stream);
/* Native binary16 products: out = sum over k ascending of
 * float(fp16(h(a) * h(b))) in fp32 (h = round to binary16), then the ROW,
 * TRANSPOSED or CONVT epilogue (+ bias; no residual / ReLU). Replaces the
 * dot products of prepare_tokens_fp16.glsl:37-52, project_tokens_fp16.glsl
 * and conv_transpose_nonoverlap_fp16.glsl (src/operators.cpp:1211-1406,
 * :1453-1481, :1862-1906); the same bits as the CPU oracle. */
DAV2_API int dav2_hip_gemm_h16_products(const dav2_gemm_f32_args* args, void* stream);

/* fp32 im2col of conv2d (src/operators.cpp:1528-1676): out[p][c], p = oy*OW
 * + ox, c = ic*k*k + ky*k + kx, zero padding, columns C*k*k .. ld-1 zero;
 * relu != 0 takes max(input, 0) (the DPT residual units' ReLU). */
DAV2_API int dav2_hip_im2col_f32(const float* input, uint32_t input_width, uint32_t input_height,
                                 uint32_t input_channels, uint32_t output_width, uint32_t output_height,
                                 uint32_t kernel, uint32_t stride, int32_t padding, uint32_t relu, float* out,
                                 uint32_t ld, void* stream);
/* Row tiles (rows of col_absmax) of a dav2_hip_gemm_i8 call with m rows and
 * n output columns. No reference counterpart: the attention's digit packing
 * reads these maxima instead of a pass over k and v. */
DAV2_API uint32_t dav2_hip_gemm_i8_row_tiles(uint32_t m, uint32_t n, uint32_t epilogue);
/* Scratch bytes of a split-K dav2_hip_gemm_i8 call. No reference counterpart. */
DAV2_API uint64_t dav2_hip_gemm_i8_split_scratch_bytes(uint32_t m, uint32_t n, uint32_t split_k);

/* Implicit-GEMM int8 convolution: replaces the im2col_quantize_int8.glsl +
 * linear_int8_tiled.glsl pair of VulkanOperators::conv2d_int8
 * (src/operators.cpp:1735-1805) for kernel 3 / stride 1 / padding 1 and
 * kernel 1 / stride 1 / padding 0, channels % 64 == 0, out_channels % 32 == 0
 * (dav2_hip_conv2d_i8_supported). Same output bits as
 * dav2_hip_im2col_quantize_i8 followed by dav2_hip_gemm_i8 with
 * DAV2_GEMM_EPI_TRANSPOSED; the im2col matrix is never stored. The weights are
 * the GpuModel int8 rows packed by dav2_hip_conv_weights_pack: K walked
 * tap-major (k = (ky*k + kx)*channels + c holds src[n][c*k*k + ky*k + kx])
 * and cut into 16-row x 64-byte MFMA operand fragments, fragment (rows
 * 16 nb.., K step ks) at byte (nb * K/64 + ks) * 1024, lane l's 16 bytes at
 * + 16 l (row 16 nb + l % 16, K bytes 64 ks + 16 (l / 16) ..). Needs
 * out_channels % 16 == 0 and kernel*kernel*channels % 64 == 0. */
enum {
    DAV2_CONV_RELU_INPUT = 1,   /* convolve max(input, 0) (relu.glsl before the conv)  */
    DAV2_CONV_RELU_OUTPUT = 2,  /* out = max(out, 0) after the residual (relu.glsl)     */
    /* Also write the next convolution's per-pixel channel-group maxima of the
     * output into partial_out ([out_channels/32][height*width], the layout of
     * the scratch): |out| (EMIT_ABSMAX) or max(out, 0) (EMIT_RELU_MAX, for a
     * consumer that applies DAV2_CONV_RELU_INPUT). Needs out_channels / 32
     * groups that each lie in one wave's channels (dav2_hip_conv2d_i8_emits). */
    DAV2_CONV_EMIT_ABSMAX = 4,
    DAV2_CONV_EMIT_RELU_MAX = 8
};

typedef struct dav2_conv_i8_args {
    const float* input;          /* CHW [channels][height][width]                  */
    uint32_t width, height, channels;
    uint32_t kernel;             /* 1 or 3                                         */
    const int8_t* weight;        /* packed (dav2_hip_conv_weights_pack)            */
    const float* weight_scales;  /* [out_channels]                                 */
    const float* bias;           /* [out_channels] or NULL = 0                     */
    uint32_t out_channels;
    float* out;                  /* CHW [out_channels][height][width]              */
    float* scratch;              /* dav2_hip_im2col_scratch_floats() floats        */
    uint64_t scratch_floats;
    uint32_t flags;              /* DAV2_CONV_*                                    */
    const float* residual;       /* NULL, or CHW like out: out = conv + residual   */
    /* The input's channel-group maxima (|x|, or max(x, 0) with RELU_INPUT)
     * when a producer has already written them (an EMIT flag or
     * dav2_hip_bilinear_align_true_maxima); NULL: computed into scratch. */
    const float* partial_in;
    float* partial_out;          /* with an EMIT flag                              */
} dav2_conv_i8_args;

DAV2_API int dav2_hip_conv2d_i8_supported(uint32_t width, uint32_t height, uint32_t channels,
                                          uint32_t out_channels, uint32_t kernel, uint32_t stride,
                                          uint32_t padding);
/* Nonzero if a supported convolution to out_channels can also emit its
 * output's channel-group maxima (DAV2_CONV_EMIT_*). No reference
 * counterpart (a fusion of channel_group maxima into the producer). */
DAV2_API int dav2_hip_conv2d_i8_emits(uint32_t out_channels, uint32_t kernel);
DAV2_API int dav2_hip_conv_weights_pack(int8_t* dst, const int8_t* src, uint32_t out_channels,
                                            uint32_t channels, uint32_t kernel, uint64_t ldb,
                                            void* stream);
DAV2_API int dav2_hip_conv2d_i8(const dav2_conv_i8_args* args, void* stream);

/* 1x1 convolution to a few output channels (out_channels <= 4, channels <=
 * 64), the DPT head's last layer (dpt.cpp:838-855 routed through the int8
 * convolution): same bits as dav2_hip_im2col_quantize_i8 + dav2_hip_gemm_i8
 * (DAV2_GEMM_EPI_TRANSPOSED), one thread per pixel. weight is the GpuModel
 * int8 layout [out_channels][ldw]. flags as above (no residual); pre_relu
 * (optional) receives the output before DAV2_CONV_RELU_OUTPUT. */
DAV2_API int dav2_hip_conv1x1_narrow_i8(const float* input, uint32_t width, uint32_t height,
                                        uint32_t channels, const int8_t* weight, uint32_t ldw,
                                        const float* weight_scales, const float* bias,
                                        uint32_t out_channels, float* out, float* pre_relu,
                                        uint32_t flags, void* stream);

/* Elementwise kernels. Reference: gelu.glsl, add_scaled.glsl, add.glsl, relu.glsl. */
DAV2_API int dav2_hip_gelu(float* out, const float* input, uint64_t count, void* stream);
DAV2_API int dav2_hip_add_scaled(float* out, const float* residual, const float* addend,
                                 const float* scale, uint64_t count, uint32_t columns,
                                 void* stream);
DAV2_API int dav2_hip_add(float* out, const float* left, const float* right, uint64_t count,
                          void* stream);
DAV2_API int dav2_hip_relu(float* out, const float* input, uint64_t count, void* stream);
/* Each float replaced by the nearest binary16 value (round to nearest even),
 * kept as a float: the fp16 mode's half weights, the reference's float_to_half
 * (src/gpu_model.cpp:51-98) applied on the device. */
DAV2_API int dav2_hip_round_half(float* data, uint64_t count, void* stream);

/* fp32 attention, head_dim 64, on the matrix cores (the fp32 precision
 * mode's path; src/operators.cpp:1169-1208 with bmm.glsl and
 * softmax_lastdim.glsl, sums in the MFMA's order: within tolerance of the
 * reference, not bit for bit). qkv is [batch*T][3*H*64] token-major (q | k |
 * v, head h at h*64); scores [batch][H][T][T] fp32, softmax in place,
 * dav2_hip_attention_scratch_bytes() bytes. fp16 must be 0 (binary16 is
 * dav2_hip_attention_ref_*). */
DAV2_API uint64_t dav2_hip_attention_scratch_bytes(uint32_t tokens, uint32_t heads, uint32_t batch,
                                                   int fp16);
DAV2_API int dav2_hip_attention_scores(void* scores, const float* qkv, uint32_t tokens,
                                       uint32_t heads, uint32_t batch, int fp16,
                                       void* stream);
DAV2_API int dav2_hip_softmax_rows(void* scores, uint64_t rows, uint32_t columns,
                                   uint32_t row_stride, int fp16, void* stream);
DAV2_API int dav2_hip_attention_values(float* out, const void* probabilities,
                                       const float* qkv, uint32_t tokens, uint32_t heads,
                                       uint32_t batch, int fp16, void* stream);

/* Attention in the reference shaders' own arithmetic order (VALU): fp16 = 0
 * follows bmm.glsl + softmax_lastdim.glsl (fp32 scores [batch][H][T][T]),
 * fp16 = 1 follows bmm_score_fp16.glsl + softmax_lastdim_half.glsl +
 * bmm_value_fp16.glsl (binary16 scores packed as half2 words
 * [batch][H][T][ceil(T/2)], every product rounded to binary16). Scores and
 * values sum in feature / source-token order, the softmax over 128 lanes and
 * the halving tree, exp is exp_cw, the division IEEE: the CPU oracle's
 * orc_attention_head64 modes 0 and 1 give the same bits. Reference:
 * src/operators.cpp:1098-1209. Scratch: dav2_hip_attention_ref_scratch_bytes()
 * (the reference's score buffer size). The softmax works in place on rows of
 * `columns` scores. */
DAV2_API uint64_t dav2_hip_attention_ref_scratch_bytes(uint32_t tokens, uint32_t heads, uint32_t batch, int fp16);
DAV2_API int dav2_hip_attention_ref_scores(void* scores, const float* qkv, uint32_t tokens, uint32_t heads,
                                           uint32_t batch, int fp16, void* stream);
DAV2_API int dav2_hip_attention_ref_softmax(void* scores, uint64_t rows, uint32_t columns, int fp16, void* stream);
DAV2_API int dav2_hip_attention_ref_values(float* out, const void* probabilities, const float* qkv,
                                           uint32_t tokens, uint32_t heads, uint32_t batch, int fp16,
                                           void* stream);

/* The binary16 pipeline above (bmm_score_fp16.glsl, softmax_lastdim_half.glsl,
 * bmm_value_fp16.glsl) fused per block of query rows, the same bits as the
 * three kernels: keys and values are rounded to binary16 once into the
 * scratch (dav2_hip_attention_ref16_fused_scratch_bytes() bytes; 0 above
 * 2240 tokens, where the three kernels are faster: use them), then each
 * workgroup keeps its 16 rows' binary16 scores in LDS through the softmax
 * and the value sums. No reference counterpart as one
 * kernel; reference: src/operators.cpp:1132-1167. */
DAV2_API uint64_t dav2_hip_attention_ref16_fused_scratch_bytes(uint32_t tokens, uint32_t heads, uint32_t batch);
DAV2_API int dav2_hip_attention_ref16_fused(float* out, const float* qkv, uint32_t tokens, uint32_t heads,
                                            uint32_t batch, void* scratch, uint64_t scratch_bytes, void* stream);

/* The reference's int8-mode scores on devices with cooperative_matrix_fp16
 * (src/operators.cpp:1137-1148 selects bmm_score_coop_fp16.glsl:12-33):
 * binary16(q * 0.125) and binary16(k) operands, every product exact, the fp32
 * sums in the matrix unit's order (v_mfma_f32_16x16x32_f16, two K steps of
 * 32 features), each score stored as binary16 in the packed
 * [batch][H][T][ceil(T/2)] layout of dav2_hip_attention_ref_scores (fp16 = 1);
 * the softmax and values then run as above. The shader leaves the sum order
 * to the device, so these scores are held to the oracle's mode 3 (exact
 * products summed in double, rounded to fp32 and then binary16) within one
 * binary16 rounding, not bit for bit. */
DAV2_API int dav2_hip_attention_ref_scores_coop(void* scores, const float* qkv, uint32_t tokens, uint32_t heads,
                                                uint32_t batch, void* stream);
/* dav2_hip_attention_ref16_fused with the cooperative-matrix scores above
 * (same scratch); the same bits as dav2_hip_attention_ref_scores_coop +
 * _ref_softmax + _ref_values with fp16 = 1. */
DAV2_API int dav2_hip_attention_ref16_fused_coop(float* out, const float* qkv, uint32_t tokens, uint32_t heads,
                                                 uint32_t batch, void* scratch, uint64_t scratch_bytes,
                                                 void* stream);

/* Fused attention (int8-mode default): replaces the materialised binary16
 * path of src/operators.cpp:1132-1167 (bmm_score_fp16.glsl,
 * softmax_lastdim_half.glsl, bmm_value_fp16.glsl) with an integer-exact
 * kernel: q*0.125, k and v in 15-bit block floating point split into int8
 * digit planes, every dot product an exact int32 MFMA sum, 21-bit softmax
 * numerators, one rounding of the exact quotient per output. The result does
 * not depend on summation order. qkv and out as above; scratch holds the
 * digit planes, exponents and block maxima,
 * dav2_hip_attention_fused_scratch_bytes() bytes, 16-byte aligned. */
DAV2_API uint64_t dav2_hip_attention_fused_scratch_bytes(uint32_t tokens, uint32_t heads, uint32_t batch);
DAV2_API int dav2_hip_attention_fused(float* out, const float* qkv, uint32_t tokens, uint32_t heads,
                                      uint32_t batch, void* scratch, uint64_t scratch_bytes, void* stream);
/* The same attention for one image (batch 1) when the qkv GEMM ran with
 * DAV2_GEMM_EPI_ROW_COLMAX from column heads*64 on: col_absmax holds
 * [partial_rows][2*heads*64] maxima of |k| and |v| per column and row tile,
 * so the digit packing reads qkv once. Same output bits as
 * dav2_hip_attention_fused. No reference counterpart (a fusion). */
DAV2_API int dav2_hip_attention_fused_colmax(float* out, const float* qkv, uint32_t tokens, uint32_t heads,
                                             const float* col_absmax, uint32_t partial_rows, void* scratch,
                                             uint64_t scratch_bytes, void* stream);

/* bilinear_align_true.glsl:27-63, CHW. */
DAV2_API int dav2_hip_bilinear_align_true(float* out, const float* input,
                                          uint32_t input_width, uint32_t input_height,
                                          uint32_t output_width, uint32_t output_height,
                                          uint32_t channels, void* stream);
/* The same output bits, plus the per-pixel maxima of |out| over each group of
 * 32 channels into partial ([channels/32][output plane], channels % 32 == 0):
 * the input maxima of a following dav2_hip_conv2d_i8 (partial_in). No
 * reference counterpart (a fusion). */
DAV2_API int dav2_hip_bilinear_align_true_maxima(float* out, float* partial, const float* input,
                                                 uint32_t input_width, uint32_t input_height,
                                                 uint32_t output_width, uint32_t output_height,
                                                 uint32_t channels, void* stream);

/* reduce_minmax.glsl as a two-stage grid reduction; partials must hold
 * 2*dav2_hip_minmax_partials(count) floats. range[0] = min, range[1] = max. */
DAV2_API uint32_t dav2_hip_minmax_partials(uint64_t count);
DAV2_API int dav2_hip_reduce_minmax(const float* input, uint64_t count, float* range,
                                    float* partials, void* stream);
/* normalize_relative.glsl:8-16 */
DAV2_API int dav2_hip_normalize_relative(float* depth, const float* range, uint64_t count,
                                         void* stream);

/* Host-image paths (the reference runs them on the CPU around the tensor
 * inference; here they run on the device buffers of the image).
 * preprocess_bgr8: src/image.cpp:163-270 (dav2::preprocess_bgr8) -- bgr is
 *   height rows of `stride` bytes, 3 bytes (B, G, R) per pixel; out is the
 *   normalised RGB CHW float32 [3][dst_height][dst_width] of the cubic resize.
 * preprocess_bgra8_nearest: src/image.cpp:289-339
 *   (dav2::preprocess_inferbridge_bgra8) -- 4 bytes per pixel, stride and base
 *   4-byte aligned; model channel c is byte c of the pixel.
 * normalize_span: src/dav2.cpp:787-800 -- out = (depth - range[0]) /
 *   (range[1] - range[0]), or 0 everywhere when that span is not positive;
 *   range from dav2_hip_reduce_minmax. */
DAV2_API int dav2_hip_preprocess_bgr8(const uint8_t* bgr, uint32_t width, uint32_t height, uint64_t stride,
                                      uint32_t dst_width, uint32_t dst_height, float* out, void* stream);
DAV2_API int dav2_hip_preprocess_bgra8_nearest(const uint8_t* bgra, uint32_t width, uint32_t height,
                                               uint64_t stride, uint32_t dst_width, uint32_t dst_height,
                                               float* out, void* stream);
DAV2_API int dav2_hip_normalize_span(const float* depth, const float* range, uint64_t count, float* out,
                                     void* stream);
/* preprocess_rgba.glsl (src/gpu_preprocess.cpp:41-104, the resize of the
 * GPU submit path): 32-bit pixels, rgba_order 1 = R in byte 0 (RGBA8), 0 =
 * R in byte 2 (BGRA8); stride a multiple of 4 bytes; float32 cubic resize to
 * the normalised RGB CHW [3][dst_height][dst_width]. */
DAV2_API int dav2_hip_preprocess_rgba8(const uint32_t* pixels, uint32_t width, uint32_t height,
                                       uint64_t stride_bytes, uint32_t dst_width, uint32_t dst_height,
                                       uint32_t rgba_order, float* out, void* stream);

/* position_bicubic.glsl:76-105 with the set-up of src/operators.cpp:1323-1376:
 * position is the [1370][D] pos_embed, out is CHW [D][ph][pw]. */
DAV2_API int dav2_hip_position_bicubic(float* out, const float* position,
                                       uint32_t patch_width, uint32_t patch_height,
                                       uint32_t embedding, void* stream);
/* copy_class_token.glsl + add_position.glsl (src/operators.cpp:1299-1304,
 * :1389-1405) for batch images of T = pw*ph+1 tokens each: token 0 becomes
 * class_token + position[0..D), token t > 0 gets interpolated[f*pw*ph + t-1]
 * added. */
DAV2_API int dav2_hip_finish_tokens(float* tokens, const float* interpolated,
                                    const float* position, const float* class_token,
                                    uint32_t patch_width, uint32_t patch_height,
                                    uint32_t embedding, uint32_t batch, void* stream);

DAV2_API const char* dav2_hip_error_string(int error);

#ifdef __cplusplus
}
#endif

#endif /* DAV2_HIP_H */
