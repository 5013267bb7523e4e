// Operator surface of the int8 hot path on HIP.
//
// Same method names, argument order and validation behaviour as the int8 and
// shared operators of the reference's VulkanOperators (src/operators.h:11-383):
// sizes are checked against the buffers (too small -> std::invalid_argument,
// src/operators.cpp:93-102) and work is enqueued asynchronously on the
// context's active stream. DeviceBuffer replaces VulkanBuffer; the int8 weight
// buffers are the GpuModel layout ([rows][ld] bytes, ld = K rounded up to 64).
// The fp32 variants (linear, project_tokens, conv2d, conv_transpose_nonoverlap,
// prepare_tokens with Precision::fp32) serve the fp32 precision mode; the fp16
// mode uses them with binary16-rounded weights, plus project_tokens_fp16,
// conv_transpose_nonoverlap_fp16, prepare_tokens with Precision::fp16 (native
// binary16 products) and linear_f32 with half operands.
//
// Fused variants (no reference counterpart) serve the encoder/DPT drivers:
// they compute the same arithmetic as the reference's separate passes.
#pragma once

#include "runtime.h"

#include <cstdint>

namespace dav2 {

// Mirrors the InferBridge native Precision enum used by the reference.
enum class Precision { fp32, fp16, int8 };

// Work folded into a convolution: a ReLU on its input, a residual added to its
// output, then a ReLU on the result (relu.glsl / add.glsl semantics, the
// order the DPT residual units apply them in).
struct ConvFusion {
    bool relu_input = false;
    bool relu_output = false;
    const DeviceBuffer* residual = nullptr;
    // Per-pixel maxima over 32-channel groups of the input, already written
    // by its producer (|x|, or max(x, 0) when relu_input): the implicit-GEMM
    // path then skips computing them.
    const DeviceBuffer* input_maxima = nullptr;
    // Ask the implicit-GEMM path to write the output's group maxima (of
    // max(out, 0) with emit_relu, for a consumer with relu_input) here;
    // conv2d_int8 returns whether it did.
    DeviceBuffer* emit_maxima = nullptr;
    bool emit_relu = false;
};

// Reusable int8 activation workspace (role of the reference's
// Int8ActivationWorkspace): packed rows + per-row scales, grown on demand.
class Int8Workspace {
public:
    DeviceBuffer& packed(std::uint64_t bytes);
    DeviceBuffer& scales(std::uint64_t bytes);
    // weights handed over in the reference's transposed [K][N] layout,
    // turned into the GEMM's [N][ld] rows
    DeviceBuffer& weight(std::uint64_t bytes);

private:
    DeviceBuffer packed_;
    DeviceBuffer scales_;
    DeviceBuffer weight_;
};

class HipOperators {
public:
    explicit HipOperators(HipContext& context);

    // Stream the operators enqueue on: the context's active stream, unless a
    // fixed one is set (a second operator set working beside the first on its
    // own stream, with its own workspaces).
    void set_stream(hipStream_t stream) { stream_ = stream; }
    hipStream_t stream() const { return stream_ ? stream_ : context_.active_stream(); }

    void linear_int8(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& int8_weight,
                     const DeviceBuffer& weight_scales, const DeviceBuffer& bias, std::uint32_t rows,
                     std::uint32_t input_columns, std::uint32_t output_columns, bool gelu,
                     bool weight_transposed = false);
    // linear_int8 with the quantized rows in caller memory: packed holds
    // rows x roundup(input_columns, 64) bytes, scales rows floats. The same
    // kernels and bits as linear_int8; allocates nothing (no workspace
    // growth, no profiling events).
    void linear_int8_in(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& int8_weight,
                        const DeviceBuffer& weight_scales, const DeviceBuffer& bias, std::uint32_t rows,
                        std::uint32_t input_columns, std::uint32_t output_columns, bool gelu,
                        const DeviceBuffer& packed, const DeviceBuffer& scales);

    void layer_norm(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& weight,
                    const DeviceBuffer& bias, std::uint32_t rows, std::uint32_t columns, float epsilon);

    void add_scaled(DeviceBuffer& output, const DeviceBuffer& residual, const DeviceBuffer& addend,
                    const DeviceBuffer& scale, std::uint32_t count, std::uint32_t columns);

    void attention_head64(DeviceBuffer& output, const DeviceBuffer& qkv, std::uint32_t tokens,
                          std::uint32_t heads, DeviceBuffer* score_scratch = nullptr,
                          Precision precision = Precision::fp32);

    void prepare_tokens(DeviceBuffer& output, const DeviceBuffer& image, const DeviceBuffer& patch_weight,
                        const DeviceBuffer& patch_half_weight, const DeviceBuffer& patch_int8_weight,
                        const DeviceBuffer& patch_int8_scales, const DeviceBuffer& patch_bias,
                        const DeviceBuffer& class_token, const DeviceBuffer& position, std::uint32_t input_width,
                        std::uint32_t input_height, std::uint32_t embedding, Precision precision,
                        bool position_is_constant = false);

    void project_tokens_int8(DeviceBuffer& output, const DeviceBuffer& tokens, const DeviceBuffer& int8_weight,
                             const DeviceBuffer& weight_scales, const DeviceBuffer& bias, std::uint32_t width,
                             std::uint32_t height, std::uint32_t embedding, std::uint32_t output_channels);

    // Returns true when fusion.emit_maxima was written.
    bool conv2d_int8(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& int8_weight,
                     const DeviceBuffer& weight_scales, const DeviceBuffer& bias, std::uint32_t input_width,
                     std::uint32_t input_height, std::uint32_t input_channels, std::uint32_t output_channels,
                     std::uint32_t kernel, std::uint32_t stride, std::uint32_t padding, bool has_bias,
                     const DeviceBuffer* packed_weight = nullptr, const ConvFusion& fusion = ConvFusion{});

    // 1x1 convolution to at most 4 output channels from at most 64 (the DPT
    // head's last layer); pre_relu, when given, receives the output before
    // fusion.relu_output. No residual.
    void conv1x1_narrow_int8(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& int8_weight,
                             std::uint32_t weight_ld, const DeviceBuffer& weight_scales, const DeviceBuffer& bias,
                             std::uint32_t width, std::uint32_t height, std::uint32_t channels,
                             std::uint32_t output_channels, bool has_bias, const ConvFusion& fusion,
                             DeviceBuffer* pre_relu);

    void conv_transpose_nonoverlap_int8(DeviceBuffer& output, const DeviceBuffer& input,
                                        const DeviceBuffer& int8_weight, const DeviceBuffer& weight_scales,
                                        const DeviceBuffer& bias, std::uint32_t input_width,
                                        std::uint32_t input_height, std::uint32_t input_channels,
                                        std::uint32_t output_channels, std::uint32_t kernel);

    // ---- fp32 precision mode ---------------------------------------------
    // fp32 weights: linear/projection [N][K], conv [OC][C*k*k] (the model
    // layout), conv-transpose rows (ky*k + kx)*OC + oc of IC columns (the
    // GpuModel reorder); K, C*k*k and IC multiples of 4.
    void linear(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& weight, const DeviceBuffer& bias,
                std::uint32_t rows, std::uint32_t input_columns, std::uint32_t output_columns, bool gelu);
    void project_tokens(DeviceBuffer& output, const DeviceBuffer& tokens, const DeviceBuffer& weight,
                        const DeviceBuffer& bias, std::uint32_t width, std::uint32_t height, std::uint32_t embedding,
                        std::uint32_t output_channels);
    void conv2d(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& weight, const DeviceBuffer& bias,
                std::uint32_t input_width, std::uint32_t input_height, std::uint32_t input_channels,
                std::uint32_t output_channels, std::uint32_t kernel, std::uint32_t stride, std::uint32_t padding,
                bool has_bias, const ConvFusion& fusion = ConvFusion{});
    void conv_transpose_nonoverlap(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& weight,
                                   const DeviceBuffer& bias, std::uint32_t input_width, std::uint32_t input_height,
                                   std::uint32_t input_channels, std::uint32_t output_channels, std::uint32_t kernel);

    // ---- fp16 precision mode (native binary16 products, k-order fp32 sums) --
    // (the float variants behind project_tokens / conv_transpose_nonoverlap
    // and their fp16 forms)
    void project_tokens_float(DeviceBuffer& output, const DeviceBuffer& tokens, const DeviceBuffer& weight,
                              const DeviceBuffer& bias, std::uint32_t width, std::uint32_t height,
                              std::uint32_t embedding, std::uint32_t output_channels, bool half_products);
    void conv_transpose_float(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& weight,
                              const DeviceBuffer& bias, std::uint32_t input_width, std::uint32_t input_height,
                              std::uint32_t input_channels, std::uint32_t output_channels, std::uint32_t kernel,
                              bool half_products);
    // Weights as the fp32 variants take them (binary16 values or not: they
    // are rounded to binary16 when staged).
    void project_tokens_fp16(DeviceBuffer& output, const DeviceBuffer& tokens, const DeviceBuffer& weight,
                             const DeviceBuffer& bias, std::uint32_t width, std::uint32_t height,
                             std::uint32_t embedding, std::uint32_t output_channels);
    void conv_transpose_nonoverlap_fp16(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& weight,
                                        const DeviceBuffer& bias, std::uint32_t input_width,
                                        std::uint32_t input_height, std::uint32_t input_channels,
                                        std::uint32_t output_channels, std::uint32_t kernel);

    void bilinear_align_true(DeviceBuffer& output, const DeviceBuffer& input, std::uint32_t input_width,
                             std::uint32_t input_height, std::uint32_t output_width, std::uint32_t output_height,
                             std::uint32_t channels);
    // The same, also writing the output's 32-channel group maxima (|out|)
    // into maxima (channels % 32 == 0).
    void bilinear_align_true_maxima(DeviceBuffer& output, DeviceBuffer& maxima, const DeviceBuffer& input,
                                    std::uint32_t input_width, std::uint32_t input_height,
                                    std::uint32_t output_width, std::uint32_t output_height, std::uint32_t channels);
    // Whether conv2d_int8 takes the implicit-GEMM path for this geometry (the
    // path that reads input_maxima), and whether that path can emit maxima.
    static bool implicit_conv(std::uint32_t width, std::uint32_t height, std::uint32_t channels,
                              std::uint32_t output_channels, std::uint32_t kernel, std::uint32_t stride,
                              std::uint32_t padding);
    static bool implicit_conv_emits(std::uint32_t width, std::uint32_t height, std::uint32_t channels,
                                    std::uint32_t output_channels, std::uint32_t kernel, std::uint32_t stride,
                                    std::uint32_t padding);

    void reduce_minmax(const DeviceBuffer& input, DeviceBuffer& range, std::uint32_t count);
    void normalize_relative(DeviceBuffer& depth, const DeviceBuffer& range, std::uint32_t count);

    void relu(DeviceBuffer& output, const DeviceBuffer& input, std::uint32_t count);
    void add(DeviceBuffer& output, const DeviceBuffer& left, const DeviceBuffer& right, std::uint32_t count);
    void gelu(DeviceBuffer& output, const DeviceBuffer& input, std::uint32_t count);

    // ---- fused variants used by the graph drivers ------------------------
    // LayerNorm whose output row is quantized straight into the workspace
    // (layer_norm + quantize_rows of linear_int8); fp32 row optional.
    void layer_norm_quantize(const DeviceBuffer& input, const DeviceBuffer& weight, const DeviceBuffer& bias,
                             std::uint32_t rows, std::uint32_t columns, float epsilon, DeviceBuffer* fp32_out);
    // quantize_rows of linear_int8 into the workspace; gelu: of gelu(input)
    // (the GELU pass of a linear_int8 with gelu, then the next linear's
    // quantization), columns <= 4096.
    void quantize_rows(const DeviceBuffer& input, std::uint64_t input_offset, std::uint32_t rows,
                       std::uint32_t columns, bool gelu = false);
    // GEMM on the rows currently held by the workspace.
    // row_colmax: row, and per GEMM row tile the maxima of |out| of the
    // columns from col_absmax_begin on into col_absmax
    // (gemm_row_tiles() x (output_columns - col_absmax_begin) floats).
    enum class Epilogue { row, row_gelu, row_layerscale, row_colmax };
    void linear_int8_prequantized(DeviceBuffer& output, const DeviceBuffer& int8_weight,
                                  const DeviceBuffer& weight_scales, const DeviceBuffer* bias, std::uint32_t rows,
                                  std::uint32_t input_columns, std::uint32_t output_columns, Epilogue epilogue,
                                  const DeviceBuffer* gamma = nullptr, std::uint64_t output_row_offset = 0,
                                  DeviceBuffer* col_absmax = nullptr, std::uint32_t col_absmax_begin = 0);
    static std::uint32_t gemm_row_tiles(std::uint32_t rows, std::uint32_t output_columns);
    // fp32 GEMM with the row epilogues (row_colmax excluded), for the fp32
    // precision mode's encoder; half_operands: both operands rounded to
    // binary16 first (the fp16 mode's cooperative-matrix linears).
    void linear_f32(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& weight,
                    const DeviceBuffer* bias, std::uint32_t rows, std::uint32_t input_columns,
                    std::uint32_t output_columns, Epilogue epilogue, const DeviceBuffer* gamma = nullptr,
                    std::uint64_t output_row_offset = 0, bool half_operands = false);
    // Batched attention over `batch` token matrices of `tokens` rows each, in
    // the reference shaders' arithmetic order (fp32: bmm.glsl /
    // softmax_lastdim.glsl; fp16: the binary16 shaders), VALU kernels.
    // cooperative (fp16 only): the scores of bmm_score_coop_fp16.glsl on the
    // matrix cores instead of bmm_score_fp16.glsl.
    void attention_batched(DeviceBuffer& output, const DeviceBuffer& qkv, std::uint32_t tokens,
                           std::uint32_t heads, std::uint32_t batch, DeviceBuffer& score_scratch,
                           Precision precision, bool cooperative = false);
    static std::uint64_t attention_score_bytes(std::uint32_t tokens, std::uint32_t heads, std::uint32_t batch,
                                               Precision precision);
    // fp32 attention on the matrix cores (fp32 precision mode): the same
    // scratch as attention_batched(fp32), sums in the MFMA's own order.
    void attention_mfma_f32(DeviceBuffer& output, const DeviceBuffer& qkv, std::uint32_t tokens,
                            std::uint32_t heads, std::uint32_t batch, DeviceBuffer& scores);
    // Fused integer-exact attention (int8 digit planes, exact int32 MFMA
    // sums): the int8-mode default in place of the materialised binary16
    // scores.
    // With col_absmax (batch 1): the |k| and |v| column maxima of a
    // row_colmax qkv GEMM from column heads*64 on, partial_rows row tiles;
    // the digit packing then reads qkv once.
    void attention_fused(DeviceBuffer& output, const DeviceBuffer& qkv, std::uint32_t tokens, std::uint32_t heads,
                         std::uint32_t batch, DeviceBuffer& scratch, const DeviceBuffer* col_absmax = nullptr,
                         std::uint32_t partial_rows = 0);
    static std::uint64_t attention_fused_scratch_bytes(std::uint32_t tokens, std::uint32_t heads,
                                                       std::uint32_t batch);

    Int8Workspace& workspace() { return workspace_; }
    HipContext& context() { return context_; }

private:
    void linear_int8_packed(DeviceBuffer& output, const DeviceBuffer& packed_input, std::uint32_t packed_ld,
                            const DeviceBuffer& int8_weight, const DeviceBuffer& input_scales,
                            const DeviceBuffer& weight_scales, const DeviceBuffer& bias, std::uint32_t rows,
                            std::uint32_t input_columns, std::uint32_t output_columns,
                            std::uint32_t output_row_offset, std::uint32_t output_row_stride, bool output_transposed,
                            bool has_bias, const DeviceBuffer* residual = nullptr, bool relu_output = false);

    HipContext& context_;
    hipStream_t stream_ = nullptr;
    Int8Workspace workspace_;
    DeviceBuffer minmax_partials_;
    DeviceBuffer interpolated_;
    // Inputs of the position interpolation held in interpolated_. It depends
    // only on pos_embed and the patch grid; callers whose pos_embed never
    // changes (the model graph) pass position_is_constant and a fixed
    // resolution computes it once.
    const void* interpolated_position_ = nullptr;
    std::uint32_t interpolated_pw_ = 0, interpolated_ph_ = 0, interpolated_dim_ = 0;
    DeviceBuffer im2col_scratch_;  // per-channel-group maxima for the tiled im2col kernels
    DeviceBuffer conv_weights_;    // packed weights of a conv2d_int8 call that brought none
    DeviceBuffer conv_act_;        // ReLU of a conv2d_int8 input on the im2col path
    DeviceBuffer gemm_split_;      // int32 slices of split-K channel-major GEMMs
    DeviceBuffer f32_cols_;        // fp32 im2col rows of the fp32 convolutions
    std::uint32_t workspace_ld_ = 0;  // row stride of the int8 rows currently in the workspace
};

}  // namespace dav2
