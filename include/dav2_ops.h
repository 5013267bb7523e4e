/*
 * C ABI over the operator surface (dav2::HipOperators), which mirrors the
 * reference's internal operator class VulkanOperators (src/operators.h:11-383).
 * Each entry replaces the same-named VulkanOperators method: same argument
 * meaning and order, same size validation (a buffer that is too small, zero
 * or inconsistent dimensions -> DAV2_STATUS_INVALID_ARGUMENT, the reference's
 * std::invalid_argument). Buffers are device memory described by
 * {pointer, bytes}; work is enqueued on the instance's stream.
 *
 * int8 weights use the reference GpuModel's layout (src/gpu_model.cpp:241-284):
 * [rows][columns] bytes -- [rows][columns/4] little-endian words of four int8,
 * as quantize_rows_int8_fused.glsl packs them -- with columns % 4 == 0 (row r,
 * column c = int8 weight of output r, input c; convolution columns
 * ic*k*k + ky*k + kx; ConvTranspose rows (ky*k+kx)*OC + oc, columns IC).
 * Rows whose length is not a multiple of 64 (patch embedding 588, 3x3 over
 * 48 channels 432, ...) are copied into a padded buffer of the instance on
 * its stream before use.
 */
#ifndef DAV2_OPS_H
#define DAV2_OPS_H

#include "depth_anything_v2.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct dav2_ops dav2_ops;

typedef struct dav2_device_buffer {
    void* data;
    uint64_t bytes;
} dav2_device_buffer;

/* Precision values of attention_head64 / prepare_tokens (InferBridge Precision). */
enum { DAV2_PRECISION_FP32 = 0, DAV2_PRECISION_FP16 = 1, DAV2_PRECISION_INT8 = 2 };

/* Creates an operator instance on HIP device `device_index` with its own
 * stream. Returns NULL on failure (reason in dav2_last_error()). */
DAV2_API dav2_ops* DAV2_CALL dav2_ops_create(int32_t device_index);
DAV2_API void DAV2_CALL dav2_ops_destroy(dav2_ops* ops);
/* Message of the last failed dav2_ops_* call on this thread. */
DAV2_API const char* DAV2_CALL dav2_ops_last_error(void);
DAV2_API void* DAV2_CALL dav2_ops_stream(dav2_ops* ops);
DAV2_API dav2_status DAV2_CALL dav2_ops_synchronize(dav2_ops* ops);

/* src/operators.h:82-92 (VulkanOperators::linear_int8, same argument order).
 * weight_transposed == 0: int8_weight is the GpuModel's int8_buffer,
 * [output_columns][input_columns] bytes. weight_transposed != 0: it is the
 * int8_transposed_buffer (src/gpu_model.cpp:241-258), [input_columns]
 * [output_columns] bytes, byte k*N + n = weight of output n, input k; it is
 * turned into rows on the instance's stream before the GEMM, and the output
 * is bit-identical to the untransposed call's. */
DAV2_API dav2_status DAV2_CALL dav2_ops_linear_int8(dav2_ops* ops, dav2_device_buffer output,
                                                    dav2_device_buffer input, dav2_device_buffer int8_weight,
                                                    dav2_device_buffer weight_scales, dav2_device_buffer bias,
                                                    uint32_t rows, uint32_t input_columns,
                                                    uint32_t output_columns, int32_t gelu,
                                                    int32_t weight_transposed);
/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Same arguments, checks and output bits as
 * dav2_ops_linear_int8, but the quantized input rows (rows x roundup(K, 64)
 * bytes), their scales and, when K % 64 != 0 or the weight is transposed, the
 * weight rows (N x roundup(K, 64) bytes) go into a fixed 32 MiB device array
 * per GPU instead of the instance's growing workspace; the call allocates
 * nothing. Sizes beyond the array -> DAV2_STATUS_INVALID_ARGUMENT. Calls on
 * one GPU from several instances (several streams) are ordered through a
 * per-device event, each waiting for the previous call; calls enqueued under
 * HIP graph capture are not, so a captured graph replayed while another call
 * runs on the same GPU races on the array: serialise those. */
DAV2_API dav2_status DAV2_CALL dav2_ops_linear_int8_noalloc(dav2_ops* ops, dav2_device_buffer output,
                                                            dav2_device_buffer input, dav2_device_buffer int8_weight,
                                                            dav2_device_buffer weight_scales,
                                                            dav2_device_buffer bias, uint32_t rows,
                                                            uint32_t input_columns, uint32_t output_columns,
                                                            int32_t gelu, int32_t weight_transposed);
/* src/operators.h:94-101 */
DAV2_API dav2_status DAV2_CALL dav2_ops_layer_norm(dav2_ops* ops, dav2_device_buffer output,
                                                   dav2_device_buffer input, dav2_device_buffer weight,
                                                   dav2_device_buffer bias, uint32_t rows, uint32_t columns,
                                                   float epsilon);
/* src/operators.h:111-117 */
DAV2_API dav2_status DAV2_CALL dav2_ops_add_scaled(dav2_ops* ops, dav2_device_buffer output,
                                                   dav2_device_buffer residual, dav2_device_buffer addend,
                                                   dav2_device_buffer scale, uint32_t count, uint32_t columns);
/* src/operators.h:119-126. score_scratch.data may be NULL (allocated internally).
 * Scratch sizes are the reference's (src/operators.cpp:1112-1119): fp32 H*T*T
 * floats, fp16 H*T*ceil(T/2) packed half2 words. Both precisions compute in
 * the reference shaders' arithmetic order (bmm.glsl / softmax_lastdim.glsl,
 * and the binary16 shaders with every product rounded to binary16). */
DAV2_API dav2_status DAV2_CALL dav2_ops_attention_head64(dav2_ops* ops, dav2_device_buffer output,
                                                         dav2_device_buffer qkv, uint32_t tokens, uint32_t heads,
                                                         dav2_device_buffer score_scratch, int32_t precision);
/* src/operators.h:128-141, INT8 precision only (fp32/fp16 weights ignored). */
DAV2_API dav2_status DAV2_CALL dav2_ops_prepare_tokens(dav2_ops* ops, dav2_device_buffer output,
                                                       dav2_device_buffer image, dav2_device_buffer patch_int8_weight,
                                                       dav2_device_buffer patch_int8_scales,
                                                       dav2_device_buffer patch_bias, dav2_device_buffer class_token,
                                                       dav2_device_buffer position, uint32_t input_width,
                                                       uint32_t input_height, uint32_t embedding);
/* src/operators.h:162-171 */
DAV2_API dav2_status DAV2_CALL dav2_ops_project_tokens_int8(dav2_ops* ops, dav2_device_buffer output,
                                                            dav2_device_buffer tokens, dav2_device_buffer int8_weight,
                                                            dav2_device_buffer weight_scales, dav2_device_buffer bias,
                                                            uint32_t width, uint32_t height, uint32_t embedding,
                                                            uint32_t output_channels);
/* src/operators.h:203-216 */
DAV2_API dav2_status DAV2_CALL dav2_ops_conv2d_int8(dav2_ops* ops, dav2_device_buffer output,
                                                    dav2_device_buffer input, dav2_device_buffer int8_weight,
                                                    dav2_device_buffer weight_scales, dav2_device_buffer bias,
                                                    uint32_t input_width, uint32_t input_height,
                                                    uint32_t input_channels, uint32_t output_channels,
                                                    uint32_t kernel, uint32_t stride, uint32_t padding,
                                                    int32_t has_bias);
/* src/operators.h:239-249 */
DAV2_API dav2_status DAV2_CALL dav2_ops_conv_transpose_nonoverlap_int8(
    dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer input, dav2_device_buffer int8_weight,
    dav2_device_buffer weight_scales, dav2_device_buffer bias, uint32_t input_width, uint32_t input_height,
    uint32_t input_channels, uint32_t output_channels, uint32_t kernel);
/* fp32 precision mode (src/operators.h: linear :62-80, project_tokens
 * :143-152, conv2d :173-187, conv_transpose_nonoverlap :218-227). fp32
 * weights: linear/projection [N][K], conv [OC][C*k*k], transposed conv rows
 * (ky*k + kx)*OC + oc of IC columns; K, C*k*k and IC multiples of 4.
 * prepare_tokens_f32: the fp32 patch embedding, weight [D][3*14*14]. */
DAV2_API dav2_status DAV2_CALL dav2_ops_linear(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer input,
                                               dav2_device_buffer weight, dav2_device_buffer bias, uint32_t rows,
                                               uint32_t input_columns, uint32_t output_columns, int32_t gelu);
DAV2_API dav2_status DAV2_CALL dav2_ops_project_tokens(dav2_ops* ops, dav2_device_buffer output,
                                                       dav2_device_buffer tokens, dav2_device_buffer weight,
                                                       dav2_device_buffer bias, uint32_t width, uint32_t height,
                                                       uint32_t embedding, uint32_t output_channels);
DAV2_API dav2_status DAV2_CALL dav2_ops_conv2d(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer input,
                                               dav2_device_buffer weight, dav2_device_buffer bias,
                                               uint32_t input_width, uint32_t input_height, uint32_t input_channels,
                                               uint32_t output_channels, uint32_t kernel, uint32_t stride,
                                               uint32_t padding, int32_t has_bias);
DAV2_API dav2_status DAV2_CALL dav2_ops_conv_transpose_nonoverlap(
    dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer input, dav2_device_buffer weight,
    dav2_device_buffer bias, uint32_t input_width, uint32_t input_height, uint32_t input_channels,
    uint32_t output_channels, uint32_t kernel);
DAV2_API dav2_status DAV2_CALL dav2_ops_prepare_tokens_f32(dav2_ops* ops, dav2_device_buffer output,
                                                           dav2_device_buffer image, dav2_device_buffer patch_weight,
                                                           dav2_device_buffer patch_bias,
                                                           dav2_device_buffer class_token,
                                                           dav2_device_buffer position, uint32_t input_width,
                                                           uint32_t input_height, uint32_t embedding);
/* src/operators.h:251-258 */
DAV2_API dav2_status DAV2_CALL dav2_ops_bilinear_align_true(dav2_ops* ops, dav2_device_buffer output,
                                                            dav2_device_buffer input, uint32_t input_width,
                                                            uint32_t input_height, uint32_t output_width,
                                                            uint32_t output_height, uint32_t channels);
/* src/operators.h:267-272 */
DAV2_API dav2_status DAV2_CALL dav2_ops_reduce_minmax(dav2_ops* ops, dav2_device_buffer input,
                                                      dav2_device_buffer range, uint32_t count);
DAV2_API dav2_status DAV2_CALL dav2_ops_normalize_relative(dav2_ops* ops, dav2_device_buffer depth,
                                                           dav2_device_buffer range, uint32_t count);
/* src/operators.h:277, :282-286; gelu is the reference's separate GELU pass (gelu.glsl). */
DAV2_API dav2_status DAV2_CALL dav2_ops_relu(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer input,
                                             uint32_t count);
DAV2_API dav2_status DAV2_CALL dav2_ops_add(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer left,
                                            dav2_device_buffer right, uint32_t count);
DAV2_API dav2_status DAV2_CALL dav2_ops_gelu(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer input,
                                             uint32_t count);

/* Whole-graph variant of dav2_infer_tensor_f32_device that also returns the
 * depth logits before the final ReLU (batch 1); for parity checks where
 * random weights drive most of the ReLU output to zero. No reference
 * counterpart. */
DAV2_API dav2_status DAV2_CALL dav2_infer_tensor_f32_device_logits(dav2_context* context,
                                                                   const float* device_input, int32_t network_width,
                                                                   int32_t network_height, float* device_depth,
                                                                   float* device_logits, void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* DAV2_OPS_H */
