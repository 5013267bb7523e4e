/*
 * CPU oracle for the Depth-Anything-V2 int8 operator hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library restates, on the CPU, what the
 * reference runtime's Vulkan compute shaders and host quantizer compute, so
 * that the HIP implementation can be checked against it on identical inputs.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it; the product library never links, loads or calls it.
 *
 * Each function names the reference file:line it follows. Layout conventions:
 *  - int8 matrices are row-major [rows][K] bytes, K unpadded (the byte view of
 *    the reference's little-endian 4x8 packing, quantize_rows_int8_fused.glsl:51);
 *  - feature maps are CHW float32; token matrices are row-major [T][D].
 *
 * Pinning (see tests/test_oracle_*.py): quantizers by hand-derived vectors and
 * invariants, the int32 GEMM by exact integer brute force, conv/conv-transpose
 * by the reference's own int8-vs-fp32 tolerance tests, LN/softmax/attention/
 * bilinear/bicubic by the reference KATs and by torch's CPU routines, the
 * graph by the reference's int8 acceptance gate against an fp32 forward.
 */
#ifndef DAV2_ORACLE_H
#define DAV2_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int orc_set_threads(int threads);
int orc_get_threads(void);

/* quantize_rows_int8_fused.glsl:20-55 */
void orc_quantize_rows(const float* input, uint32_t rows, uint32_t columns,
                       uint32_t input_offset, int8_t* q, float* scales);
/* im2col_quantize_int8.glsl:26-83 (rows = OW*OH, K = C*k*k) */
void orc_im2col_quantize(const float* input, uint32_t input_width,
                         uint32_t input_height, uint32_t input_channels,
                         uint32_t output_width, uint32_t output_height,
                         uint32_t kernel, uint32_t stride, int32_t padding,
                         int8_t* q, float* scales);
/* weight quantizer, gpu_model.cpp:241-264, per output row */
void orc_quantize_weight_rows(const float* weight, uint64_t rows,
                              uint64_t columns, int8_t* q, float* scales);
/* weight layout, gpu_model.cpp:210-240, ConvTranspose [IC][OC][k][k] -> rows (ky*k+kx)*OC+oc */
void orc_quantize_convT_weight(const float* weight, uint32_t in_channels,
                               uint32_t out_channels, uint32_t kernel,
                               int8_t* q, float* scales);
/* exact int32 accumulators, acc[m][n] = sum_k a[m][k]*b[n][k] */
void orc_gemm_i8(const int8_t* a, const int8_t* b, uint32_t m, uint32_t n,
                 uint32_t k, int32_t* acc);
/* linear_int8_tiled.glsl:99-116 epilogue */
void orc_linear_epilogue(const int32_t* acc, const float* input_scales,
                         const float* weight_scales, const float* bias,
                         uint32_t rows, uint32_t columns,
                         uint32_t output_row_offset, uint32_t output_row_stride,
                         int transposed, float* out);

/* Operator surface (operators.h), fp32 in / fp32 out. */
void orc_linear_int8(const float* input, const int8_t* w8, const float* w_scales,
                     const float* bias, uint32_t rows, uint32_t in_columns,
                     uint32_t out_columns, int gelu, float* out);
/* gelu.glsl:16-49 (Numerical Recipes erfc fit, shader operation order). */
void orc_gelu(const float* input, uint64_t count, float* out);
/* e^x as the kernels evaluate it (Cody-Waite reduction, degree-7 Taylor). */
void orc_exp(const float* input, uint64_t count, float* out);
void orc_layer_norm(const float* input, const float* weight, const float* bias,
                    uint32_t rows, uint32_t columns, float epsilon, float* out);
void orc_add_scaled(const float* residual, const float* addend,
                    const float* scale, uint64_t count, uint32_t columns,
                    float* out);
void orc_add(const float* left, const float* right, uint64_t count, float* out);
void orc_relu(const float* input, uint64_t count, float* out);
void orc_softmax_rows(const float* input, uint64_t rows, uint32_t columns,
                      float* out);
/* mode 0: fp32 bmm/softmax (bmm.glsl, softmax_lastdim.glsl).
 * mode 1: materialised binary16 scores and probabilities, the arithmetic of
 *         bmm_score_fp16.glsl, softmax_lastdim_half.glsl, bmm_value_fp16.glsl:
 *         every product rounded to binary16, fp32 sums in the shaders' order.
 * mode 2: integer-exact (the int8-mode kernel): 15-bit block floating point
 *         q*0.125 (per token), k (per head) and v (per feature), exact
 *         integer dot products, 21-bit softmax numerators.
 * mode 3: mode 1 with the scores of bmm_score_coop_fp16.glsl (devices with
 *         cooperative_matrix_fp16): binary16 operands, exact products summed
 *         in double (feature order) and rounded to fp32, then to binary16.
 *         The shader leaves the order of the fp32 sums to the matrix unit,
 *         so a GPU result is held to this within a tolerance.
 * probabilities (optional) receives [H][T][T]. */
void orc_attention_head64(const float* qkv, uint32_t tokens, uint32_t heads,
                          int mode, float* out, float* probabilities);
/* The binary16 scores of mode 1 before the softmax (bmm_score_fp16.glsl):
 * scores [H][T][T] binary16 bit patterns. */
void orc_attention_scores_binary16(const float* qkv, uint32_t tokens, uint32_t heads, uint16_t* scores);
/* The binary16 scores of mode 3 (bmm_score_coop_fp16.glsl, sums as above). */
void orc_attention_scores_coop(const float* qkv, uint32_t tokens, uint32_t heads, uint16_t* scores);
/* out[i] = fp16(a[i] * b[i]) for binary16 values a, b (the vector path the
 * mode-1 attention uses; the tail uses the scalar conversion). */
void orc_round_half_product(const float* a, const float* b, uint64_t count, float* out);
/* The 21-bit softmax numerator of mode 2 for each x (as a float integer). */
void orc_numerator21(const float* x, uint64_t count, float* out);
// the same function eight values at a time (the form the attention uses)
void orc_numerator21_x8(const float* x, uint64_t count, float* out);
void orc_bilinear_align_true(const float* input, uint32_t input_width,
                             uint32_t input_height, uint32_t output_width,
                             uint32_t output_height, uint32_t channels,
                             float* out);
void orc_reduce_minmax(const float* input, uint64_t count, float* range);
void orc_normalize_relative(float* depth, const float* range, uint64_t count);
/* position_bicubic.glsl:76-105 with the block set up at operators.cpp:1346-1364;
 * output CHW [D][ph][pw] */
void orc_position_bicubic(const float* position, uint32_t patch_width,
                          uint32_t patch_height, uint32_t embedding,
                          float* out);
void orc_prepare_tokens_int8(const float* image, const int8_t* w8,
                             const float* w_scales, const float* bias,
                             const float* class_token, const float* position,
                             uint32_t width, uint32_t height,
                             uint32_t embedding, float* tokens);
void orc_project_tokens_int8(const float* tokens, const int8_t* w8,
                             const float* w_scales, const float* bias,
                             uint32_t width, uint32_t height,
                             uint32_t embedding, uint32_t out_channels,
                             float* out);
void orc_conv2d_int8(const float* input, const int8_t* w8, const float* w_scales,
                     const float* bias, uint32_t width, uint32_t height,
                     uint32_t in_channels, uint32_t out_channels,
                     uint32_t kernel, uint32_t stride, uint32_t padding,
                     int has_bias, float* out);
void orc_conv_transpose_int8(const float* input, const int8_t* w8,
                             const float* w_scales, const float* bias,
                             uint32_t width, uint32_t height,
                             uint32_t in_channels, uint32_t out_channels,
                             uint32_t kernel, float* out);

/* Whole int8 graph: encoder.cpp:322-597 + dpt.cpp:628-863 (all DPT convs int8). */
typedef struct orc_model orc_model;
orc_model* orc_model_load(const char* path, int encoder, char* error,
                          size_t error_bytes);
void orc_model_free(orc_model* model);
/* attention_mode selects orc_attention_head64's mode for every block: 2 (the
 * integer-exact attention, this build's int8-mode default), 1 (the
 * reference's binary16 pipeline, DAV2_CREATE_REFERENCE_FP16_ATTENTION), 3
 * (the same with cooperative-matrix scores,
 * DAV2_CREATE_REFERENCE_FP16_COOP_ATTENTION) or 0 (fp32 scores,
 * FORCE_FP32_ATTENTION).
 * depth: W*H raw ReLU depth. pre_relu (nullable): W*H before the final ReLU.
 * features (nullable): 4*T*D captured encoder features.
 * Returns 0 on success. */
int orc_model_infer(orc_model* model, const float* chw, uint32_t width,
                    uint32_t height, int attention_mode, float* depth,
                    float* pre_relu, float* features);
/* The same graph in the fp32 precision mode (DAV2_CREATE_FORCE_FP32): fp32
 * weights and activations, fp32 attention. */
int orc_model_infer_fp32(orc_model* model, const float* chw, uint32_t width,
                         uint32_t height, float* depth, float* pre_relu,
                         float* features);
/* fp32 operators (operators.cpp:882-955, :1211-1452, :1528-1676,
 * :1807-1861): float32 sums in k order. Weights in the model file layout. */
void orc_linear_f32(const float* input, const float* weight, const float* bias,
                    uint32_t rows, uint32_t in_cols, uint32_t out_cols, int gelu,
                    float* out);
void orc_conv2d_f32(const float* input, const float* weight, const float* bias,
                    uint32_t width, uint32_t height, uint32_t in_channels,
                    uint32_t out_channels, uint32_t kernel, uint32_t stride,
                    uint32_t padding, int has_bias, float* out);
void orc_conv_transpose_f32(const float* input, const float* weight,
                            const float* bias, uint32_t width, uint32_t height,
                            uint32_t in_channels, uint32_t out_channels,
                            uint32_t kernel, float* out);
void orc_project_tokens_f32(const float* tokens, const float* weight,
                            const float* bias, uint32_t width, uint32_t height,
                            uint32_t D, uint32_t C, float* out);
void orc_prepare_tokens_f32(const float* image, const float* weight,
                            const float* bias, const float* class_token,
                            const float* position, uint32_t width,
                            uint32_t height, uint32_t D, float* tokens);
/* The graph in the fp16 precision mode (DAV2_CREATE_FORCE_FP16): half
 * weights; cooperative-matrix linears (binary16 operands, exact products,
 * fp32 sums) with layer_norm_fp16 / pack_fp16 inputs and fc1's half output;
 * native binary16 patch embedding, projections and transposed convolutions;
 * DPT convolutions through conv2d with half weights (fp32 arithmetic);
 * attention_mode 1 (binary16, the default) or 0 (FORCE_FP32_ATTENTION). */
int orc_model_infer_fp16(orc_model* model, const float* chw, uint32_t width,
                         uint32_t height, int attention_mode, float* depth,
                         float* pre_relu, float* features);
/* fp16 operators. orc_gemm_h16_products: out[m][n] = sum over k ascending of
 * float(fp16(h(a) * h(b))) in fp32, h = round to binary16 (the native
 * binary16 shaders' dot products). orc_linear_f16: linear_coop_fp16.glsl
 * (operators.cpp:540-768), optional GELU and half output. The others:
 * prepare_tokens_fp16.glsl, project_tokens_fp16.glsl,
 * conv_transpose_nonoverlap_fp16.glsl. Weights in the model file layout
 * (fp32, rounded to binary16 inside). */
void orc_gemm_h16_products(const float* a, uint64_t lda, const float* b, uint64_t ldb,
                           uint32_t m, uint32_t n, uint32_t k, float* out);
void orc_linear_f16(const float* input, const float* weight, const float* bias,
                    uint32_t rows, uint32_t in_cols, uint32_t out_cols, int gelu,
                    int half_output, float* out);
void orc_project_tokens_f16(const float* tokens, const float* weight,
                            const float* bias, uint32_t width, uint32_t height,
                            uint32_t D, uint32_t C, float* out);
void orc_conv_transpose_f16(const float* input, const float* weight,
                            const float* bias, uint32_t width, uint32_t height,
                            uint32_t in_channels, uint32_t out_channels,
                            uint32_t kernel, float* out);
void orc_prepare_tokens_f16(const float* image, const float* weight,
                            const float* bias, const float* class_token,
                            const float* position, uint32_t width,
                            uint32_t height, uint32_t D, float* tokens);
/* Encoder blocks [first, last) only, on tokens [T][D] in place (timing sample). */
int orc_model_encoder_blocks(orc_model* model, float* tokens, uint32_t tokens_count,
                             uint32_t first, uint32_t last, int attention_mode);

/* Host image paths (src/image.cpp, src/dav2.cpp:630-665, :754-802).
 * network_shape: image.cpp:138-161; returns 0, or 1 for a non-positive size.
 * preprocess_bgr8: image.cpp:163-270 -- interleaved BGR bytes (row stride in
 *   bytes) -> normalised RGB CHW float32 [3][dh][dw], separable cubic resize
 *   with float32 coefficients and float64 intermediates.
 * preprocess_bgra8_nearest: image.cpp:289-339 -- BGRA bytes kept in BGR
 *   channel order, floor-nearest resize, float32 normalisation.
 * normalize_span: dav2.cpp:787-800 -- (x - min) / (max - min), all zero when
 *   the span is not positive. */
int orc_network_shape(int width, int height, int input_size, int* out_width,
                      int* out_height);
void orc_preprocess_bgr8(const uint8_t* bgr, int width, int height,
                         int64_t stride, int dst_width, int dst_height,
                         float* out);
void orc_preprocess_bgra8_nearest(const uint8_t* bgra, int width, int height,
                                  int64_t stride, int dst_width,
                                  int dst_height, float* out);
void orc_normalize_span(const float* depth, uint64_t count, float* out);
/* preprocess_rgba.glsl (src/gpu_preprocess.cpp:41-104): float32 cubic
 * resize of 32-bit pixels (rgba_order 1: R in byte 0; 0: BGRA, R in byte 2). */
void orc_preprocess_rgba8(const uint32_t* pixels, int width, int height,
                          int64_t stride_pixels, int dst_width, int dst_height,
                          int rgba_order, float* out);

/* IEEE binary16 round-to-nearest-even helpers used by the fp16 attention path. */
uint16_t orc_float_to_half(float value);
float orc_half_to_float(uint16_t value);
uint32_t orc_crc32(const void* data, size_t bytes);

#ifdef __cplusplus
}
#endif

#endif
