#include "operators.h"

#include <algorithm>

#include "dav2_hip.h"

#include <limits>
#include <stdexcept>
#include <string>

namespace dav2 {
namespace {

// src/operators.cpp:93-102
void require_bytes(const DeviceBuffer& buffer, std::uint64_t elements, const char* name) {
    if (elements > std::numeric_limits<std::uint64_t>::max() / sizeof(float) ||
        buffer.size() < elements * sizeof(float))
        throw std::invalid_argument(std::string(name) + " device buffer is too small");
}

void require_int8_weight(const DeviceBuffer& weight, std::uint64_t rows, std::uint64_t columns, const char* what) {
    const std::uint64_t ld = (columns + 63) & ~63ull;
    if (weight.size() < rows * ld) throw std::invalid_argument(std::string(what) + " is too small");
}

std::uint32_t ld64(std::uint64_t columns) { return static_cast<std::uint32_t>((columns + 63) & ~63ull); }

// 32-channel groups of the per-pixel maxima the convolutions' scales use.
std::uint32_t channel_group_count(std::uint32_t channels) { return (channels + 31u) / 32u; }

DeviceBuffer& grow(DeviceBuffer& buffer, std::uint64_t bytes) {
    if (buffer.size() < bytes) {
        // Work already queued may still read the old allocation.
        hip_check(hipDeviceSynchronize(), "workspace grow");
        buffer.reset();
        buffer = DeviceBuffer(bytes);
    }
    return buffer;
}

}  // namespace

DeviceBuffer& Int8Workspace::packed(std::uint64_t bytes) { return grow(packed_, bytes); }
DeviceBuffer& Int8Workspace::scales(std::uint64_t bytes) { return grow(scales_, bytes); }
DeviceBuffer& Int8Workspace::weight(std::uint64_t bytes) { return grow(weight_, bytes); }

HipOperators::HipOperators(HipContext& context) : context_(context) {}

// ---------------------------------------------------------------------------
// src/operators.cpp:770-845. weight_transposed: int8_weight is the
// reference's [K][N] byte layout (int8_transposed_buffer, gpu_model.cpp:
// 241-258), turned into the GEMM's rows on this stream first; the result is
// the same as for the [N][K] weight.
void HipOperators::linear_int8(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& int8_weight,
                               const DeviceBuffer& weight_scales, const DeviceBuffer& bias, std::uint32_t rows,
                               std::uint32_t input_columns, std::uint32_t output_columns, bool gelu,
                               bool weight_transposed) {
    if (rows == 0 || input_columns == 0 || output_columns == 0 || input_columns % 4 != 0)
        throw std::invalid_argument("invalid INT8 linear dimensions");
    require_bytes(input, std::uint64_t(rows) * input_columns, "input");
    const DeviceBuffer* weight = &int8_weight;
    if (weight_transposed) {
        if (int8_weight.size() < std::uint64_t(output_columns) * input_columns)
            throw std::invalid_argument("transposed INT8 weight buffer is too small");
    } else {
        require_int8_weight(int8_weight, output_columns, input_columns, "packed INT8 weight buffer");
    }
    require_bytes(weight_scales, output_columns, "weight scale");
    require_bytes(bias, output_columns, "bias");
    require_bytes(output, std::uint64_t(rows) * output_columns, "output");
    if (weight_transposed) {
        const std::uint32_t ld = ld64(input_columns);
        DeviceBuffer& rows_layout = workspace_.weight(std::uint64_t(output_columns) * ld);
        hip_check(dav2_hip_transpose_rows_i8(int8_weight.as<int8_t>(), input_columns, output_columns,
                                             rows_layout.as<int8_t>(), ld, stream()),
                  "transpose int8 weight");
        weight = &rows_layout;
    }
    quantize_rows(input, 0, rows, input_columns);
    linear_int8_prequantized(output, *weight, weight_scales, &bias, rows, input_columns, output_columns,
                             gelu ? Epilogue::row_gelu : Epilogue::row);
}

void HipOperators::linear_int8_in(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& int8_weight,
                                  const DeviceBuffer& weight_scales, const DeviceBuffer& bias, std::uint32_t rows,
                                  std::uint32_t input_columns, std::uint32_t output_columns, bool gelu,
                                  const DeviceBuffer& packed, const DeviceBuffer& scales) {
    if (rows == 0 || input_columns == 0 || output_columns == 0 || input_columns % 4 != 0)
        throw std::invalid_argument("invalid INT8 linear dimensions");
    require_bytes(input, std::uint64_t(rows) * input_columns, "input");
    require_int8_weight(int8_weight, output_columns, input_columns, "packed INT8 weight buffer");
    require_bytes(weight_scales, output_columns, "weight scale");
    require_bytes(bias, output_columns, "bias");
    require_bytes(output, std::uint64_t(rows) * output_columns, "output");
    const std::uint32_t ld = ld64(input_columns);
    if (packed.size() < std::uint64_t(rows) * ld || scales.size() < std::uint64_t(rows) * sizeof(float))
        throw std::invalid_argument("INT8 linear workspace is too small");
    hip_check(dav2_hip_quantize_rows_i8(input.as<float>(), 0, rows, input_columns, packed.as<int8_t>(), ld,
                                        scales.as<float>(), stream()),
              "quantize_rows_int8");
    dav2_gemm_i8_args a{};
    a.a = packed.as<int8_t>();
    a.lda = ld;
    a.b = int8_weight.as<int8_t>();
    a.ldb = ld;
    a.m = rows;
    a.n = output_columns;
    a.k = ld;
    a.epilogue = gelu ? DAV2_GEMM_EPI_ROW_GELU : DAV2_GEMM_EPI_ROW;
    a.a_scales = scales.as<float>();
    a.b_scales = weight_scales.as<float>();
    a.bias = bias.as<float>();
    a.out = output.as<float>();
    hip_check(dav2_hip_gemm_i8(&a, stream()), "int8 GEMM");
}

void HipOperators::quantize_rows(const DeviceBuffer& input, std::uint64_t input_offset, std::uint32_t rows,
                                 std::uint32_t columns, bool gelu) {
    const std::uint32_t ld = ld64(columns);
    DeviceBuffer& packed = workspace_.packed(std::uint64_t(rows) * ld);
    DeviceBuffer& scales = workspace_.scales(std::uint64_t(rows) * sizeof(float));
    ProfileScope prof(context_.profiler(), gelu ? "gelu_quantize_rows_i8" : "quantize_rows_i8",
                      5.0 * rows * columns + 4.0 * rows, "B", stream());
    const auto quantize = gelu ? dav2_hip_gelu_quantize_rows_i8 : dav2_hip_quantize_rows_i8;
    hip_check(quantize(input.as<float>(), input_offset, rows, columns, packed.as<int8_t>(), ld, scales.as<float>(),
                       stream()),
              "quantize_rows_int8");
    workspace_ld_ = ld;
}

void HipOperators::layer_norm_quantize(const DeviceBuffer& input, const DeviceBuffer& weight,
                                       const DeviceBuffer& bias, std::uint32_t rows, std::uint32_t columns,
                                       float epsilon, DeviceBuffer* fp32_out) {
    if (rows == 0 || columns == 0 || columns % 4 != 0 || epsilon <= 0.0f)
        throw std::invalid_argument("invalid layer norm parameters");
    require_bytes(input, std::uint64_t(rows) * columns, "input");
    require_bytes(weight, columns, "weight");
    require_bytes(bias, columns, "bias");
    if (fp32_out) require_bytes(*fp32_out, std::uint64_t(rows) * columns, "output");
    const std::uint32_t ld = ld64(columns);
    DeviceBuffer& packed = workspace_.packed(std::uint64_t(rows) * ld);
    DeviceBuffer& scales = workspace_.scales(std::uint64_t(rows) * sizeof(float));
    ProfileScope prof(context_.profiler(), "layer_norm_quantize_i8",
                      5.0 * rows * columns + 8.0 * columns + 4.0 * rows + (fp32_out ? 4.0 * rows * columns : 0.0),
                      "B", stream());
    hip_check(dav2_hip_layer_norm_quantize_i8(packed.as<int8_t>(), ld, scales.as<float>(),
                                              fp32_out ? fp32_out->as<float>() : nullptr, input.as<float>(),
                                              weight.as<float>(), bias.as<float>(), rows, columns, epsilon,
                                              stream()),
              "layer_norm_quantize");
    workspace_ld_ = ld;
}

void HipOperators::linear_int8_prequantized(DeviceBuffer& output, const DeviceBuffer& int8_weight,
                                            const DeviceBuffer& weight_scales, const DeviceBuffer* bias,
                                            std::uint32_t rows, std::uint32_t input_columns,
                                            std::uint32_t output_columns, Epilogue epilogue,
                                            const DeviceBuffer* gamma, std::uint64_t output_row_offset,
                                            DeviceBuffer* col_absmax, std::uint32_t col_absmax_begin) {
    if (workspace_ld_ != ld64(input_columns)) throw std::logic_error("int8 workspace holds rows of another width");
    require_bytes(output, (std::uint64_t(rows) + output_row_offset) * output_columns, "output");
    if (epilogue == Epilogue::row_layerscale && (!gamma || gamma->size() < output_columns * sizeof(float)))
        throw std::invalid_argument("layer scale buffer is too small");
    if (epilogue == Epilogue::row_colmax) {
        if (!col_absmax || col_absmax_begin % 64 || col_absmax_begin >= output_columns || output_row_offset != 0)
            throw std::invalid_argument("invalid column maxima request");
        require_bytes(*col_absmax,
                      std::uint64_t(gemm_row_tiles(rows, output_columns)) * (output_columns - col_absmax_begin),
                      "column maxima");
    }
    dav2_gemm_i8_args a{};
    a.a = workspace_.packed(0).as<int8_t>();
    a.lda = workspace_ld_;
    a.b = int8_weight.as<int8_t>();
    a.ldb = ld64(input_columns);
    a.m = rows;
    a.n = output_columns;
    a.k = ld64(input_columns);
    a.epilogue = epilogue == Epilogue::row ? DAV2_GEMM_EPI_ROW
                 : epilogue == Epilogue::row_gelu ? DAV2_GEMM_EPI_ROW_GELU
                 : epilogue == Epilogue::row_colmax ? DAV2_GEMM_EPI_ROW_COLMAX
                                                    : DAV2_GEMM_EPI_ROW_LAYERSCALE;
    if (epilogue == Epilogue::row_colmax) {
        a.col_absmax = col_absmax->as<float>();
        a.col_absmax_begin = col_absmax_begin;
    }
    a.a_scales = workspace_.scales(0).as<float>();
    a.b_scales = weight_scales.as<float>();
    a.bias = bias ? bias->as<float>() : nullptr;
    a.out = output.as<float>();
    a.out_row_offset = output_row_offset;
    a.residual = output.as<float>();
    a.gamma = gamma ? gamma->as<float>() : nullptr;
    ProfileScope prof(context_.profiler(), "gemm_i8", 2.0 * rows * output_columns * input_columns, "OP",
                      stream());
    prof.shape(rows, output_columns, input_columns,
               epilogue == Epilogue::row        ? "row"
               : epilogue == Epilogue::row_gelu ? "row_gelu"
               : epilogue == Epilogue::row_colmax ? "row_colmax"
                                                  : "row_layerscale");
    hip_check(dav2_hip_gemm_i8(&a, stream()), "int8 GEMM");
}

// src/operators.cpp:847-880
void HipOperators::linear_int8_packed(DeviceBuffer& output, const DeviceBuffer& packed_input,
                                      std::uint32_t packed_ld, const DeviceBuffer& int8_weight,
                                      const DeviceBuffer& input_scales, const DeviceBuffer& weight_scales,
                                      const DeviceBuffer& bias, std::uint32_t rows, std::uint32_t input_columns,
                                      std::uint32_t output_columns, std::uint32_t output_row_offset,
                                      std::uint32_t output_row_stride, bool output_transposed, bool has_bias,
                                      const DeviceBuffer* residual, bool relu_output) {
    dav2_gemm_i8_args a{};
    a.a = packed_input.as<int8_t>();
    a.lda = packed_ld;
    a.b = int8_weight.as<int8_t>();
    a.ldb = ld64(input_columns);
    a.m = rows;
    a.n = output_columns;
    a.k = ld64(input_columns);
    a.epilogue = output_transposed ? DAV2_GEMM_EPI_TRANSPOSED : DAV2_GEMM_EPI_ROW;
    a.a_scales = input_scales.as<float>();
    a.b_scales = weight_scales.as<float>();
    a.bias = has_bias ? bias.as<float>() : nullptr;
    a.out = output.as<float>();
    a.out_row_offset = output_row_offset;
    a.out_row_stride = output_row_stride;
    a.residual = residual ? residual->as<float>() : nullptr;  // TRANSPOSED only
    a.relu_output = relu_output ? 1u : 0u;
    if (output_transposed) {
        // Few output tiles (the DPT's 37x37 / 19x19 maps): split K so that
        // about 384 workgroups run, each slice at least six 128-byte stages.
        // Measured per shape (M x N x K, us: unsplit / about 256 workgroups
        // with two-stage slices / this rule): 1369x512x1024 7.8 / 11.5 / 7.8,
        // 1369x256x9216 32.7 / 18.0 / 15.7, 361x1024x9216 33.8 / 18.9 / 17.3,
        // 361x256x2304 11.3 / 8.8 / 8.4; the int32 partial sums make every
        // split bit-identical.
        const std::uint32_t tiles = ((output_columns + 63) / 64) * ((rows + 63) / 64);
        const std::uint32_t ksteps = (a.k + 127) / 128;
        const std::uint32_t split = std::min({8u, (384u + tiles - 1) / tiles, ksteps / 6});
        if (split > 1) {
            grow(gemm_split_, dav2_hip_gemm_i8_split_scratch_bytes(rows, output_columns, split));
            a.split_k = split;
            a.split_scratch = gemm_split_.as<std::int32_t>();
        }
    }
    ProfileScope prof(context_.profiler(), "gemm_i8", 2.0 * rows * output_columns * input_columns, "OP",
                      stream());
    prof.shape(rows, output_columns, input_columns, output_transposed ? (residual ? "transposed_residual"
                                                                                  : "transposed")
                                                                      : "row");
    hip_check(dav2_hip_gemm_i8(&a, stream()), "int8 GEMM");
}

// src/operators.cpp:1016-1042
void HipOperators::layer_norm(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& weight,
                              const DeviceBuffer& bias, std::uint32_t rows, std::uint32_t columns, float epsilon) {
    if (rows == 0 || columns == 0 || epsilon <= 0.0f) throw std::invalid_argument("invalid layer norm parameters");
    require_bytes(input, std::uint64_t(rows) * columns, "input");
    require_bytes(output, std::uint64_t(rows) * columns, "output");
    require_bytes(weight, columns, "weight");
    require_bytes(bias, columns, "bias");
    ProfileScope prof(context_.profiler(), "layer_norm", 8.0 * rows * columns + 8.0 * columns, "B",
                      stream());
    hip_check(dav2_hip_layer_norm(output.as<float>(), input.as<float>(), weight.as<float>(), bias.as<float>(), rows,
                                  columns, epsilon, stream()),
              "layer_norm");
}

// src/operators.cpp:1072-1096
void HipOperators::add_scaled(DeviceBuffer& output, const DeviceBuffer& residual, const DeviceBuffer& addend,
                              const DeviceBuffer& scale, std::uint32_t count, std::uint32_t columns) {
    if (count == 0 || columns == 0 || count % columns != 0) throw std::invalid_argument("invalid add-scaled dimensions");
    require_bytes(output, count, "output");
    require_bytes(residual, count, "residual");
    require_bytes(addend, count, "addend");
    require_bytes(scale, columns, "scale");
    ProfileScope prof(context_.profiler(), "add_scaled", 12.0 * count, "B", stream());
    hip_check(dav2_hip_add_scaled(output.as<float>(), residual.as<float>(), addend.as<float>(), scale.as<float>(),
                                  count, columns, stream()),
              "add_scaled");
}

std::uint64_t HipOperators::attention_score_bytes(std::uint32_t tokens, std::uint32_t heads, std::uint32_t batch,
                                                  Precision precision) {
    // fp32: H*T*T floats; fp16: H*T*ceil(T/2) packed half2 words (the
    // reference's sizes, operators.cpp:1112-1119)
    return dav2_hip_attention_ref_scratch_bytes(tokens, heads, batch, precision == Precision::fp16 ? 1 : 0);
}

// src/operators.cpp:1098-1209
void HipOperators::attention_head64(DeviceBuffer& output, const DeviceBuffer& qkv, std::uint32_t tokens,
                                    std::uint32_t heads, DeviceBuffer* score_scratch, Precision precision) {
    if (tokens == 0 || heads == 0) throw std::invalid_argument("invalid attention dimensions");
    const std::uint64_t elements = std::uint64_t(tokens) * heads * 64;
    require_bytes(output, elements, "attention output");
    require_bytes(qkv, elements * 3, "QKV");
    const std::uint64_t score_bytes = attention_score_bytes(tokens, heads, 1, precision);
    DeviceBuffer owned;
    if (score_scratch == nullptr) {
        owned = context_.create_device_buffer(score_bytes);
        score_scratch = &owned;
    } else if (score_scratch->size() < score_bytes) {
        throw std::invalid_argument("attention score scratch device buffer is too small");
    }
    attention_batched(output, qkv, tokens, heads, 1, *score_scratch, precision);
    if (owned) context_.synchronize();  // the local scratch must outlive the kernels
}

void HipOperators::attention_batched(DeviceBuffer& output, const DeviceBuffer& qkv, std::uint32_t tokens,
                                     std::uint32_t heads, std::uint32_t batch, DeviceBuffer& scores,
                                     Precision precision, bool cooperative) {
    if (tokens == 0 || heads == 0 || batch == 0) throw std::invalid_argument("invalid attention dimensions");
    const int fp16 = precision == Precision::fp16 ? 1 : 0;
    if (cooperative && !fp16) throw std::invalid_argument("cooperative-matrix scores are binary16");
    if (scores.size() < attention_score_bytes(tokens, heads, batch, precision))
        throw std::invalid_argument("attention score scratch device buffer is too small");
    const hipStream_t s = stream();
    const double flops = 2.0 * batch * heads * double(tokens) * tokens * 64.0;
    const double score_bytes = double(dav2_hip_attention_ref_scratch_bytes(tokens, heads, batch, fp16));
    Profiler& prof = context_.profiler();
    if (fp16) {
        // the same bits in one pass per query block, when the scratch holds
        // its binary16 keys and values (all but the shortest sequences)
        const std::uint64_t fused = dav2_hip_attention_ref16_fused_scratch_bytes(tokens, heads, batch);
        if (fused != 0 && scores.size() >= fused) {
            ProfileScope p(prof, cooperative ? "attention_ref16_coop_fused" : "attention_ref16_fused", 2.0 * flops,
                           "FLOP", s);
            const auto run = cooperative ? dav2_hip_attention_ref16_fused_coop : dav2_hip_attention_ref16_fused;
            hip_check(run(output.as<float>(), qkv.as<float>(), tokens, heads, batch, scores.data(), scores.size(), s),
                      "fused binary16 attention");
            return;
        }
    }
    if (cooperative) {
        ProfileScope p(prof, "attention_scores_coop_f16", flops, "FLOP", s);
        hip_check(dav2_hip_attention_ref_scores_coop(scores.data(), qkv.as<float>(), tokens, heads, batch, s),
                  "cooperative-matrix attention scores");
    } else {
        ProfileScope p(prof, fp16 ? "attention_scores_ref_f16" : "attention_scores_ref_f32", flops, "FLOP", s);
        hip_check(dav2_hip_attention_ref_scores(scores.data(), qkv.as<float>(), tokens, heads, batch, fp16, s),
                  "attention scores");
    }
    {
        // bytes: the row read once and written once
        ProfileScope p(prof, fp16 ? "softmax_f16" : "softmax_f32", 2.0 * score_bytes, "B", s);
        hip_check(dav2_hip_attention_ref_softmax(scores.data(), std::uint64_t(batch) * heads * tokens, tokens, fp16, s),
                  "attention softmax");
    }
    {
        ProfileScope p(prof, fp16 ? "attention_values_ref_f16" : "attention_values_ref_f32", flops, "FLOP", s);
        hip_check(dav2_hip_attention_ref_values(output.as<float>(), scores.data(), qkv.as<float>(), tokens, heads,
                                                batch, fp16, s),
                  "attention values");
    }
}

void HipOperators::attention_mfma_f32(DeviceBuffer& output, const DeviceBuffer& qkv, std::uint32_t tokens,
                                      std::uint32_t heads, std::uint32_t batch, DeviceBuffer& scores) {
    if (scores.size() < dav2_hip_attention_scratch_bytes(tokens, heads, batch, 0))
        throw std::invalid_argument("attention score scratch device buffer is too small");
    const hipStream_t s = stream();
    const double flops = 2.0 * batch * heads * double(tokens) * tokens * 64.0;
    const double score_bytes = double(batch) * heads * tokens * tokens * 4.0;
    Profiler& prof = context_.profiler();
    {
        ProfileScope p(prof, "attention_scores", flops, "FLOP", s);
        hip_check(dav2_hip_attention_scores(scores.data(), qkv.as<float>(), tokens, heads, batch, 0, s),
                  "attention scores");
    }
    {
        ProfileScope p(prof, "softmax_f32_mfma_path", 2.0 * score_bytes, "B", s);
        hip_check(dav2_hip_softmax_rows(scores.data(), std::uint64_t(batch) * heads * tokens, tokens, tokens, 0, s),
                  "attention softmax");
    }
    {
        ProfileScope p(prof, "attention_values", flops, "FLOP", s);
        hip_check(dav2_hip_attention_values(output.as<float>(), scores.data(), qkv.as<float>(), tokens, heads, batch,
                                            0, s),
                  "attention values");
    }
}

std::uint64_t HipOperators::attention_fused_scratch_bytes(std::uint32_t tokens, std::uint32_t heads,
                                                          std::uint32_t batch) {
    return dav2_hip_attention_fused_scratch_bytes(tokens, heads, batch);
}

std::uint32_t HipOperators::gemm_row_tiles(std::uint32_t rows, std::uint32_t output_columns) {
    return dav2_hip_gemm_i8_row_tiles(rows, output_columns, DAV2_GEMM_EPI_ROW_COLMAX);
}

void HipOperators::attention_fused(DeviceBuffer& output, const DeviceBuffer& qkv, std::uint32_t tokens,
                                   std::uint32_t heads, std::uint32_t batch, DeviceBuffer& scratch,
                                   const DeviceBuffer* col_absmax, std::uint32_t partial_rows) {
    if (tokens == 0 || heads == 0 || batch == 0) throw std::invalid_argument("invalid attention dimensions");
    const std::uint64_t elements = std::uint64_t(batch) * tokens * heads * 64;
    require_bytes(output, elements, "attention output");
    require_bytes(qkv, elements * 3, "QKV");
    const std::uint64_t need = attention_fused_scratch_bytes(tokens, heads, batch);
    if (scratch.size() < need) throw std::invalid_argument("attention scratch device buffer is too small");
    const hipStream_t s = stream();
    // QK^T and PV: 4*T*T*64 flops per head.
    const double flops = 4.0 * batch * heads * double(tokens) * tokens * 64.0;
    ProfileScope p(context_.profiler(), "attention_fused", flops, "FLOP", s);
    if (col_absmax) {
        if (batch != 1 || partial_rows == 0) throw std::invalid_argument("column maxima serve one image");
        require_bytes(*col_absmax, std::uint64_t(partial_rows) * 2 * heads * 64, "column maxima");
        hip_check(dav2_hip_attention_fused_colmax(output.as<float>(), qkv.as<float>(), tokens, heads,
                                                  col_absmax->as<float>(), partial_rows, scratch.data(),
                                                  scratch.size(), s),
                  "fused attention");
        return;
    }
    hip_check(dav2_hip_attention_fused(output.as<float>(), qkv.as<float>(), tokens, heads, batch, scratch.data(),
                                       scratch.size(), s),
              "fused attention");
}

// src/operators.cpp:1211-1406 (int8 branch)
void HipOperators::prepare_tokens(DeviceBuffer& output, const DeviceBuffer& image, const DeviceBuffer& patch_weight,
                                  const DeviceBuffer&, const DeviceBuffer& patch_int8_weight,
                                  const DeviceBuffer& patch_int8_scales, const DeviceBuffer& patch_bias,
                                  const DeviceBuffer& class_token, const DeviceBuffer& position,
                                  std::uint32_t input_width, std::uint32_t input_height, std::uint32_t embedding,
                                  Precision precision, bool position_is_constant) {
    if (input_width == 0 || input_height == 0 || input_width % 14 != 0 || input_height % 14 != 0 || embedding == 0)
        throw std::invalid_argument("invalid patch embedding dimensions");
    const std::uint32_t pw = input_width / 14, ph = input_height / 14, spatial = pw * ph;
    const std::uint64_t tokens = std::uint64_t(spatial) + 1;
    constexpr std::uint32_t patch_columns = 3u * 14u * 14u;
    require_bytes(image, std::uint64_t(input_width) * input_height * 3, "image");
    if (precision == Precision::int8) {
        require_int8_weight(patch_int8_weight, embedding, patch_columns, "INT8 patch weight buffer");
        require_bytes(patch_int8_scales, embedding, "patch weight scale");
    } else {
        require_bytes(patch_weight, std::uint64_t(embedding) * patch_columns, "patch weight");
    }
    require_bytes(patch_bias, embedding, "patch bias");
    require_bytes(class_token, embedding, "class token");
    require_bytes(position, std::uint64_t(1370) * embedding, "position");
    require_bytes(output, tokens * embedding, "token output");
    const hipStream_t s = stream();
    if (precision == Precision::int8) {
        const std::uint32_t ld = ld64(patch_columns);
        DeviceBuffer& packed = workspace_.packed(std::uint64_t(spatial) * ld);
        DeviceBuffer& scales = workspace_.scales(std::uint64_t(spatial) * sizeof(float));
        {  // the scope ends before the GEMM launch: it times the im2col kernel alone
            ProfileScope prof_patch(context_.profiler(), "im2col_quantize_i8",
                                    12.0 * input_width * input_height + 1.0 * spatial * patch_columns + 4.0 * spatial,
                                    "B", s);
            hip_check(dav2_hip_im2col_quantize_i8(image.as<float>(), input_width, input_height, 3, pw, ph, 14, 14, 0,
                                                  packed.as<int8_t>(), ld, scales.as<float>(), nullptr, 0, s),
                      "patch im2col");
        }
        linear_int8_packed(output, packed, ld, patch_int8_weight, scales, patch_int8_scales, patch_bias, spatial,
                           patch_columns, embedding, 1u, static_cast<std::uint32_t>(tokens), false, true);
        workspace_ld_ = ld;
    } else {
        // fp32 / fp16: im2col rows of the 14x14 patches, GEMM into token rows
        // 1.. (fp16: prepare_tokens_fp16.glsl's binary16 products)
        DeviceBuffer& cols = grow(f32_cols_, std::uint64_t(spatial) * patch_columns * sizeof(float));
        hip_check(dav2_hip_im2col_f32(image.as<float>(), input_width, input_height, 3, pw, ph, 14, 14, 0, 0,
                                      cols.as<float>(), patch_columns, s),
                  "patch im2col");
        if (precision == Precision::fp16) {
            dav2_gemm_f32_args a{};
            a.a = cols.as<float>();
            a.lda = patch_columns;
            a.b = patch_weight.as<float>();
            a.ldb = patch_columns;
            a.m = spatial;
            a.n = embedding;
            a.k = patch_columns;
            a.epilogue = DAV2_GEMM_EPI_ROW;
            a.bias = patch_bias.as<float>();
            a.out = output.as<float>();
            a.out_row_offset = 1;
            ProfileScope prof(context_.profiler(), "gemm_h16_products", 2.0 * spatial * embedding * patch_columns,
                              "OP", s);
            hip_check(dav2_hip_gemm_h16_products(&a, s), "fp16 patch embedding");
        } else {
            linear_f32(output, cols, patch_weight, &patch_bias, spatial, patch_columns, embedding, Epilogue::row,
                       nullptr, 1);
        }
    }
    const void* before = interpolated_.data();
    grow(interpolated_, std::uint64_t(spatial) * embedding * sizeof(float));
    if (!position_is_constant || interpolated_.data() != before || interpolated_position_ != position.data() ||
        interpolated_pw_ != pw || interpolated_ph_ != ph || interpolated_dim_ != embedding) {
        hip_check(dav2_hip_position_bicubic(interpolated_.as<float>(), position.as<float>(), pw, ph, embedding, s),
                  "position bicubic");
        interpolated_position_ = position.data();
        interpolated_pw_ = pw;
        interpolated_ph_ = ph;
        interpolated_dim_ = embedding;
        if (!position_is_constant) interpolated_position_ = nullptr;
    }
    hip_check(dav2_hip_finish_tokens(output.as<float>(), interpolated_.as<float>(), position.as<float>(),
                                     class_token.as<float>(), pw, ph, embedding, 1, s),
              "class/position tokens");
}

// ---- fp32 precision mode ------------------------------------------------------
void HipOperators::linear_f32(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& weight,
                              const DeviceBuffer* bias, std::uint32_t rows, std::uint32_t input_columns,
                              std::uint32_t output_columns, Epilogue epilogue, const DeviceBuffer* gamma,
                              std::uint64_t output_row_offset, bool half_operands) {
    if (rows == 0 || input_columns == 0 || output_columns == 0)
        throw std::invalid_argument("linear dimensions cannot be zero");
    if (input_columns % 4u) throw std::invalid_argument("fp32 linear input columns must be a multiple of four");
    if (epilogue == Epilogue::row_colmax) throw std::invalid_argument("no column maxima on the fp32 GEMM");
    require_bytes(input, std::uint64_t(rows) * input_columns, "input");
    require_bytes(weight, std::uint64_t(output_columns) * input_columns, "weight");
    if (bias) require_bytes(*bias, output_columns, "bias");
    require_bytes(output, (std::uint64_t(rows) + output_row_offset) * output_columns, "output");
    dav2_gemm_f32_args a{};
    a.a = input.as<float>();
    a.lda = input_columns;
    a.b = weight.as<float>();
    a.ldb = input_columns;
    a.m = rows;
    a.n = output_columns;
    a.k = input_columns;
    a.bias = bias ? bias->as<float>() : nullptr;
    a.out = output.as<float>();
    a.out_row_offset = output_row_offset;
    a.half_operands = half_operands ? 1u : 0u;
    switch (epilogue) {
        case Epilogue::row_gelu: a.epilogue = DAV2_GEMM_EPI_ROW_GELU; break;
        case Epilogue::row_layerscale:
            if (!gamma) throw std::invalid_argument("LayerScale epilogue needs gamma");
            require_bytes(*gamma, output_columns, "LayerScale gamma");
            a.epilogue = DAV2_GEMM_EPI_ROW_LAYERSCALE;
            a.residual = output.as<float>();
            a.gamma = gamma->as<float>();
            break;
        default: a.epilogue = DAV2_GEMM_EPI_ROW; break;
    }
    ProfileScope prof(context_.profiler(), "gemm_f32", 2.0 * rows * output_columns * input_columns, "OP", stream());
    hip_check(dav2_hip_gemm_f32(&a, stream()), "fp32 linear");
}

// src/operators.cpp:882-955
void HipOperators::linear(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& weight,
                          const DeviceBuffer& bias, std::uint32_t rows, std::uint32_t input_columns,
                          std::uint32_t output_columns, bool gelu) {
    linear_f32(output, input, weight, &bias, rows, input_columns, output_columns,
               gelu ? Epilogue::row_gelu : Epilogue::row);
}

// src/operators.cpp:1408-1452: CLS skipped, channel-major output
void HipOperators::project_tokens(DeviceBuffer& output, const DeviceBuffer& tokens, const DeviceBuffer& weight,
                                  const DeviceBuffer& bias, std::uint32_t width, std::uint32_t height,
                                  std::uint32_t embedding, std::uint32_t output_channels) {
    project_tokens_float(output, tokens, weight, bias, width, height, embedding, output_channels, false);
}

// src/operators.cpp:1453-1481 (project_tokens_fp16.glsl)
void HipOperators::project_tokens_fp16(DeviceBuffer& output, const DeviceBuffer& tokens, const DeviceBuffer& weight,
                                       const DeviceBuffer& bias, std::uint32_t width, std::uint32_t height,
                                       std::uint32_t embedding, std::uint32_t output_channels) {
    project_tokens_float(output, tokens, weight, bias, width, height, embedding, output_channels, true);
}

void HipOperators::project_tokens_float(DeviceBuffer& output, const DeviceBuffer& tokens, const DeviceBuffer& weight,
                                        const DeviceBuffer& bias, std::uint32_t width, std::uint32_t height,
                                        std::uint32_t embedding, std::uint32_t output_channels, bool half_products) {
    const std::uint32_t spatial = width * height;
    if (width == 0 || height == 0 || embedding == 0 || output_channels == 0)
        throw std::invalid_argument("invalid token projection dimensions");
    if (embedding % 4u) throw std::invalid_argument("fp32 token embedding must be a multiple of four");
    require_bytes(tokens, std::uint64_t(spatial + 1u) * embedding, "tokens");
    require_bytes(weight, std::uint64_t(output_channels) * embedding, "weight");
    require_bytes(bias, output_channels, "bias");
    require_bytes(output, std::uint64_t(spatial) * output_channels, "output");
    dav2_gemm_f32_args a{};
    a.a = tokens.as<float>() + embedding;
    a.lda = embedding;
    a.b = weight.as<float>();
    a.ldb = embedding;
    a.m = spatial;
    a.n = output_channels;
    a.k = embedding;
    a.epilogue = DAV2_GEMM_EPI_TRANSPOSED;
    a.bias = bias.as<float>();
    a.out = output.as<float>();
    a.out_row_stride = spatial;
    ProfileScope prof(context_.profiler(), half_products ? "gemm_h16_products" : "gemm_f32",
                      2.0 * spatial * output_channels * embedding, "OP", stream());
    hip_check(half_products ? dav2_hip_gemm_h16_products(&a, stream()) : dav2_hip_gemm_f32(&a, stream()),
              "token projection");
}

// src/operators.cpp:1528-1676: im2col + GEMM, CHW output; fusion as conv2d_int8
void HipOperators::conv2d(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& weight,
                          const DeviceBuffer& bias, std::uint32_t input_width, std::uint32_t input_height,
                          std::uint32_t input_channels, std::uint32_t output_channels, std::uint32_t kernel,
                          std::uint32_t stride, std::uint32_t padding, bool has_bias, const ConvFusion& fusion) {
    if (input_width == 0 || input_height == 0 || input_channels == 0 || output_channels == 0 || kernel == 0 ||
        stride == 0 || input_width + 2u * padding < kernel || input_height + 2u * padding < kernel)
        throw std::invalid_argument("invalid convolution dimensions");
    const std::uint32_t inner = input_channels * kernel * kernel;
    if (inner % 4u) throw std::invalid_argument("fp32 convolution inner size must be a multiple of four");
    const std::uint32_t ow = (input_width + 2u * padding - kernel) / stride + 1u;
    const std::uint32_t oh = (input_height + 2u * padding - kernel) / stride + 1u;
    const std::uint64_t pixels = std::uint64_t(ow) * oh;
    if (pixels > 0xffffffffull) throw std::invalid_argument("convolution output too large");
    require_bytes(input, std::uint64_t(input_width) * input_height * input_channels, "convolution input");
    require_bytes(weight, std::uint64_t(output_channels) * inner, "convolution weight");
    if (has_bias) require_bytes(bias, output_channels, "convolution bias");
    require_bytes(output, pixels * output_channels, "convolution output");
    if (fusion.residual) require_bytes(*fusion.residual, pixels * output_channels, "convolution residual");
    const hipStream_t s = stream();
    DeviceBuffer& cols = grow(f32_cols_, pixels * inner * sizeof(float));
    ProfileScope prof_cols(context_.profiler(), "im2col_f32", 4.0 * pixels * inner, "B", s);
    hip_check(dav2_hip_im2col_f32(input.as<float>(), input_width, input_height, input_channels, ow, oh, kernel, stride,
                                  static_cast<std::int32_t>(padding), fusion.relu_input ? 1u : 0u, cols.as<float>(),
                                  inner, s),
              "fp32 im2col");
    dav2_gemm_f32_args a{};
    a.a = cols.as<float>();
    a.lda = inner;
    a.b = weight.as<float>();
    a.ldb = inner;
    a.m = static_cast<std::uint32_t>(pixels);
    a.n = output_channels;
    a.k = inner;
    a.epilogue = DAV2_GEMM_EPI_TRANSPOSED;
    a.bias = has_bias ? bias.as<float>() : nullptr;
    a.out = output.as<float>();
    a.out_row_stride = pixels;
    a.residual = fusion.residual ? fusion.residual->as<float>() : nullptr;
    a.relu_output = fusion.relu_output ? 1u : 0u;
    ProfileScope prof(context_.profiler(), "gemm_f32", 2.0 * pixels * output_channels * inner, "OP", s);
    hip_check(dav2_hip_gemm_f32(&a, s), "fp32 convolution");
}

// src/operators.cpp:1807-1861, stride == kernel
void HipOperators::conv_transpose_nonoverlap(DeviceBuffer& output, const DeviceBuffer& input,
                                             const DeviceBuffer& weight, const DeviceBuffer& bias,
                                             std::uint32_t input_width, std::uint32_t input_height,
                                             std::uint32_t input_channels, std::uint32_t output_channels,
                                             std::uint32_t kernel) {
    conv_transpose_float(output, input, weight, bias, input_width, input_height, input_channels, output_channels,
                         kernel, false);
}

// src/operators.cpp:1862-1906 (conv_transpose_nonoverlap_fp16.glsl)
void HipOperators::conv_transpose_nonoverlap_fp16(DeviceBuffer& output, const DeviceBuffer& input,
                                                  const DeviceBuffer& weight, const DeviceBuffer& bias,
                                                  std::uint32_t input_width, std::uint32_t input_height,
                                                  std::uint32_t input_channels, std::uint32_t output_channels,
                                                  std::uint32_t kernel) {
    conv_transpose_float(output, input, weight, bias, input_width, input_height, input_channels, output_channels,
                         kernel, true);
}

void HipOperators::conv_transpose_float(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& weight,
                                        const DeviceBuffer& bias, std::uint32_t input_width,
                                        std::uint32_t input_height, std::uint32_t input_channels,
                                        std::uint32_t output_channels, std::uint32_t kernel, bool half_products) {
    if (input_width == 0 || input_height == 0 || input_channels == 0 || output_channels == 0 || kernel == 0)
        throw std::invalid_argument("invalid transposed convolution dimensions");
    if (input_channels % 4u) throw std::invalid_argument("fp32 transposed convolution channels must be a multiple of four");
    const std::uint64_t pixels = std::uint64_t(input_width) * input_height;
    const std::uint32_t wrows = kernel * kernel * output_channels;
    require_bytes(input, pixels * input_channels, "transposed convolution input");
    require_bytes(weight, std::uint64_t(wrows) * input_channels, "transposed convolution weight");
    require_bytes(bias, output_channels, "transposed convolution bias");
    require_bytes(output, pixels * kernel * kernel * output_channels, "transposed convolution output");
    const hipStream_t s = stream();
    DeviceBuffer& cols = grow(f32_cols_, pixels * input_channels * sizeof(float));
    hip_check(dav2_hip_im2col_f32(input.as<float>(), input_width, input_height, input_channels, input_width,
                                  input_height, 1, 1, 0, 0, cols.as<float>(), input_channels, s),
              "fp32 pixel rows");
    dav2_gemm_f32_args a{};
    a.a = cols.as<float>();
    a.lda = input_channels;
    a.b = weight.as<float>();
    a.ldb = input_channels;
    a.m = static_cast<std::uint32_t>(pixels);
    a.n = wrows;
    a.k = input_channels;
    a.epilogue = DAV2_GEMM_EPI_CONVT;
    a.bias = bias.as<float>();
    a.out = output.as<float>();
    a.convt_kernel = kernel;
    a.convt_width = input_width;
    a.convt_height = input_height;
    a.convt_channels = output_channels;
    ProfileScope prof(context_.profiler(), half_products ? "gemm_h16_products" : "gemm_f32",
                      2.0 * pixels * wrows * input_channels, "OP", s);
    hip_check(half_products ? dav2_hip_gemm_h16_products(&a, s) : dav2_hip_gemm_f32(&a, s),
              "transposed convolution");
}

// src/operators.cpp:1483-1526
void HipOperators::project_tokens_int8(DeviceBuffer& output, const DeviceBuffer& tokens,
                                       const DeviceBuffer& int8_weight, const DeviceBuffer& weight_scales,
                                       const DeviceBuffer& bias, std::uint32_t width, std::uint32_t height,
                                       std::uint32_t embedding, std::uint32_t output_channels) {
    const std::uint32_t spatial = width * height;
    if (embedding % 4u != 0u || embedding == 0 || spatial == 0 || output_channels == 0)
        throw std::invalid_argument("INT8 token embedding must be divisible by four");
    require_bytes(tokens, std::uint64_t(spatial + 1u) * embedding, "tokens");
    require_int8_weight(int8_weight, output_channels, embedding, "INT8 projection weight");
    require_bytes(weight_scales, output_channels, "weight scale");
    require_bytes(bias, output_channels, "bias");
    require_bytes(output, std::uint64_t(spatial) * output_channels, "output");
    quantize_rows(tokens, embedding, spatial, embedding);
    linear_int8_packed(output, workspace_.packed(0), workspace_ld_, int8_weight, workspace_.scales(0),
                       weight_scales, bias, spatial, embedding, output_channels, 0u, spatial, true, true);
}

// src/operators.cpp:1735-1805
bool HipOperators::implicit_conv(std::uint32_t width, std::uint32_t height, std::uint32_t channels,
                                 std::uint32_t output_channels, std::uint32_t kernel, std::uint32_t stride,
                                 std::uint32_t padding) {
    // 3x3 convolutions of maps narrower than the implicit GEMM's 64-pixel row
    // tiles (37x37, 19x19 in the DPT head) run as fast or faster as im2col +
    // GEMM with split K (ViT-L's 19x19 layer4_rn: 33 against 74 us); a 1x1
    // convolution of such a map is faster implicit (37x37, 256 channels: 8.6
    // against 23 us for channel maxima + im2col + GEMM).
    return (width >= 64 || kernel == 1) &&
           dav2_hip_conv2d_i8_supported(width, height, channels, output_channels, kernel, stride, padding) != 0;
}

bool HipOperators::implicit_conv_emits(std::uint32_t width, std::uint32_t height, std::uint32_t channels,
                                       std::uint32_t output_channels, std::uint32_t kernel, std::uint32_t stride,
                                       std::uint32_t padding) {
    return implicit_conv(width, height, channels, output_channels, kernel, stride, padding) &&
           dav2_hip_conv2d_i8_emits(output_channels, kernel) != 0;
}

bool HipOperators::conv2d_int8(DeviceBuffer& output, const DeviceBuffer& input, const DeviceBuffer& int8_weight,
                               const DeviceBuffer& weight_scales, const DeviceBuffer& bias,
                               std::uint32_t input_width, std::uint32_t input_height, std::uint32_t input_channels,
                               std::uint32_t output_channels, std::uint32_t kernel, std::uint32_t stride,
                               std::uint32_t padding, bool has_bias, const DeviceBuffer* packed_weight,
                               const ConvFusion& fusion) {
    if (input_width == 0 || input_height == 0 || input_channels == 0 || output_channels == 0 || kernel == 0 ||
        stride == 0 || input_width + 2u * padding < kernel || input_height + 2u * padding < kernel)
        throw std::invalid_argument("invalid INT8 convolution dimensions");
    const std::uint32_t inner = input_channels * kernel * kernel;
    if (inner % 4u != 0u) throw std::invalid_argument("INT8 convolution inner size is not packed");
    const std::uint32_t ow = (input_width + 2u * padding - kernel) / stride + 1u;
    const std::uint32_t oh = (input_height + 2u * padding - kernel) / stride + 1u;
    const std::uint32_t rows = ow * oh;
    require_bytes(input, std::uint64_t(input_width) * input_height * input_channels, "convolution input");
    require_int8_weight(int8_weight, output_channels, inner, "INT8 convolution weight");
    require_bytes(weight_scales, output_channels, "convolution weight scale");
    require_bytes(bias, has_bias ? output_channels : 1u, "convolution bias");
    require_bytes(output, std::uint64_t(rows) * output_channels, "output");
    if (fusion.residual) require_bytes(*fusion.residual, std::uint64_t(rows) * output_channels, "residual");
    const hipStream_t s = stream();
    const std::uint64_t scratch_floats = dav2_hip_im2col_scratch_floats(input_width, input_height, input_channels);
    // Implicit GEMM: same bits as im2col + GEMM, no im2col matrix.
    if (implicit_conv(input_width, input_height, input_channels, output_channels, kernel, stride, padding)) {
        const DeviceBuffer* packed = packed_weight;
        if (!packed || !*packed) {
            grow(conv_weights_, std::uint64_t(output_channels) * inner);
            hip_check(dav2_hip_conv_weights_pack(conv_weights_.as<int8_t>(), int8_weight.as<int8_t>(),
                                                 output_channels, input_channels, kernel, ld64(inner), s),
                      "packed conv weights");
            packed = &conv_weights_;
        } else {
            if (packed->size() < std::uint64_t(output_channels) * inner)
                throw std::invalid_argument("packed convolution weight is too small");
        }
        grow(im2col_scratch_, scratch_floats * sizeof(float));
        ProfileScope prof(context_.profiler(), "conv2d_i8", 2.0 * rows * output_channels * inner, "OP", s);
        dav2_conv_i8_args a{};
        a.input = input.as<float>();
        a.width = input_width;
        a.height = input_height;
        a.channels = input_channels;
        a.kernel = kernel;
        a.weight = packed->as<int8_t>();
        a.weight_scales = weight_scales.as<float>();
        a.bias = has_bias ? bias.as<float>() : nullptr;
        a.out_channels = output_channels;
        a.out = output.as<float>();
        a.scratch = im2col_scratch_.as<float>();
        a.scratch_floats = scratch_floats;
        a.flags = (fusion.relu_input ? DAV2_CONV_RELU_INPUT : 0u) | (fusion.relu_output ? DAV2_CONV_RELU_OUTPUT : 0u);
        a.residual = fusion.residual ? fusion.residual->as<float>() : nullptr;
        const std::uint64_t group_floats = std::uint64_t(channel_group_count(input_channels)) * rows;
        if (fusion.input_maxima) {
            require_bytes(*fusion.input_maxima, group_floats, "convolution input maxima");
            a.partial_in = fusion.input_maxima->as<float>();
        }
        const bool emit = fusion.emit_maxima && dav2_hip_conv2d_i8_emits(output_channels, kernel);
        if (emit) {
            require_bytes(*fusion.emit_maxima, std::uint64_t(output_channels / 32u) * rows, "convolution output maxima");
            a.partial_out = fusion.emit_maxima->as<float>();
            a.flags |= fusion.emit_relu ? DAV2_CONV_EMIT_RELU_MAX : DAV2_CONV_EMIT_ABSMAX;
        }
        hip_check(dav2_hip_conv2d_i8(&a, s), "implicit-GEMM convolution");
        return emit;
    }
    // im2col + GEMM: the input ReLU is taken by the tiled im2col kernels
    // (other geometries get a separate pass), the residual and the output
    // ReLU by the GEMM's channel-major epilogue.
    const bool tiled = stride == 1 && ((kernel == 3 && padding == 1 && input_channels % 16 == 0) ||
                                       (kernel == 1 && padding == 0));
    const DeviceBuffer* src = &input;
    if (fusion.relu_input && !tiled) {
        const std::uint32_t count = input_width * input_height * input_channels;
        grow(conv_act_, std::uint64_t(count) * sizeof(float));
        relu(conv_act_, input, count);
        src = &conv_act_;
    }
    const std::uint32_t ld = ld64(inner);
    DeviceBuffer& packed = workspace_.packed(std::uint64_t(rows) * ld);
    DeviceBuffer& scales = workspace_.scales(std::uint64_t(rows) * sizeof(float));
    grow(im2col_scratch_, scratch_floats * sizeof(float));
    {  // the scope ends before the GEMM launch: it times the im2col kernels alone
        ProfileScope prof(context_.profiler(), "im2col_quantize_i8",
                          4.0 * input_width * input_height * input_channels + 1.0 * rows * inner + 4.0 * rows, "B", s);
        const auto im2col =
            fusion.relu_input && tiled ? dav2_hip_im2col_quantize_relu_i8 : dav2_hip_im2col_quantize_i8;
        hip_check(im2col(src->as<float>(), input_width, input_height, input_channels, ow, oh, kernel, stride,
                         static_cast<std::int32_t>(padding), packed.as<int8_t>(), ld, scales.as<float>(),
                         im2col_scratch_.as<float>(), scratch_floats, s),
                  "im2col quantize");
    }
    workspace_ld_ = ld;
    linear_int8_packed(output, packed, ld, int8_weight, scales, weight_scales, bias, rows, inner, output_channels, 0u,
                       rows, true, has_bias, fusion.residual, fusion.relu_output);
    return false;
}

void HipOperators::conv1x1_narrow_int8(DeviceBuffer& output, const DeviceBuffer& input,
                                       const DeviceBuffer& int8_weight, std::uint32_t weight_ld,
                                       const DeviceBuffer& weight_scales, const DeviceBuffer& bias,
                                       std::uint32_t width, std::uint32_t height, std::uint32_t channels,
                                       std::uint32_t output_channels, bool has_bias, const ConvFusion& fusion,
                                       DeviceBuffer* pre_relu) {
    if (width == 0 || height == 0 || channels == 0 || channels > 64 || output_channels == 0 || output_channels > 4 ||
        weight_ld < channels || fusion.residual)
        throw std::invalid_argument("invalid narrow 1x1 INT8 convolution");
    const std::uint64_t plane = std::uint64_t(width) * height;
    require_bytes(input, plane * channels, "convolution input");
    if (int8_weight.size() < std::uint64_t(output_channels) * weight_ld)
        throw std::invalid_argument("INT8 convolution weight is too small");
    require_bytes(weight_scales, output_channels, "convolution weight scale");
    if (has_bias) require_bytes(bias, output_channels, "convolution bias");
    require_bytes(output, plane * output_channels, "output");
    if (pre_relu) require_bytes(*pre_relu, plane * output_channels, "pre-ReLU output");
    const hipStream_t s = stream();
    ProfileScope prof(context_.profiler(), "conv1x1_narrow_i8", 4.0 * plane * (channels + output_channels), "B", s);
    const std::uint32_t flags =
        (fusion.relu_input ? DAV2_CONV_RELU_INPUT : 0u) | (fusion.relu_output ? DAV2_CONV_RELU_OUTPUT : 0u);
    hip_check(dav2_hip_conv1x1_narrow_i8(input.as<float>(), width, height, channels, int8_weight.as<int8_t>(), weight_ld,
                                         weight_scales.as<float>(), has_bias ? bias.as<float>() : nullptr,
                                         output_channels, output.as<float>(), pre_relu ? pre_relu->as<float>() : nullptr,
                                         flags, s),
              "narrow 1x1 convolution");
}

// src/operators.cpp:1908-1976
void HipOperators::conv_transpose_nonoverlap_int8(DeviceBuffer& output, const DeviceBuffer& input,
                                                  const DeviceBuffer& int8_weight,
                                                  const DeviceBuffer& weight_scales, const DeviceBuffer& bias,
                                                  std::uint32_t input_width, std::uint32_t input_height,
                                                  std::uint32_t input_channels, std::uint32_t output_channels,
                                                  std::uint32_t kernel) {
    if (input_width == 0 || input_height == 0 || input_channels == 0 || output_channels == 0 || kernel == 0 ||
        input_channels % 4u != 0u)
        throw std::invalid_argument("invalid INT8 transposed convolution");
    const std::uint32_t input_rows = input_width * input_height;
    const std::uint32_t weight_rows = kernel * kernel * output_channels;
    require_bytes(input, std::uint64_t(input_rows) * input_channels, "transposed convolution input");
    require_int8_weight(int8_weight, weight_rows, input_channels, "INT8 transposed weight");
    require_bytes(weight_scales, weight_rows, "transposed weight scale");
    require_bytes(bias, output_channels, "transposed bias");
    require_bytes(output, std::uint64_t(input_rows) * kernel * kernel * output_channels, "transposed output");
    const std::uint32_t ld = ld64(input_channels);
    DeviceBuffer& packed = workspace_.packed(std::uint64_t(input_rows) * ld);
    DeviceBuffer& scales = workspace_.scales(std::uint64_t(input_rows) * sizeof(float));
    const hipStream_t s = stream();
    const std::uint64_t scratch_floats = dav2_hip_im2col_scratch_floats(input_width, input_height, input_channels);
    grow(im2col_scratch_, scratch_floats * sizeof(float));
    {  // the scope ends before the GEMM launch: it times the im2col kernels alone
        ProfileScope prof_q(context_.profiler(), "im2col_quantize_i8",
                            4.0 * input_rows * input_channels + 1.0 * input_rows * input_channels + 4.0 * input_rows,
                            "B", s);
        hip_check(dav2_hip_im2col_quantize_i8(input.as<float>(), input_width, input_height, input_channels,
                                              input_width, input_height, 1, 1, 0, packed.as<int8_t>(), ld,
                                              scales.as<float>(), im2col_scratch_.as<float>(), scratch_floats, s),
                  "im2col quantize");
    }
    workspace_ld_ = ld;
    dav2_gemm_i8_args a{};
    a.a = packed.as<int8_t>();
    a.lda = ld;
    a.b = int8_weight.as<int8_t>();
    a.ldb = ld;
    a.m = input_rows;
    a.n = weight_rows;
    a.k = ld;
    a.epilogue = DAV2_GEMM_EPI_CONVT;
    a.a_scales = scales.as<float>();
    a.b_scales = weight_scales.as<float>();
    a.bias = bias.as<float>();
    a.out = output.as<float>();
    a.convt_kernel = kernel;
    a.convt_width = input_width;
    a.convt_height = input_height;
    a.convt_channels = output_channels;
    ProfileScope prof(context_.profiler(), "gemm_i8", 2.0 * input_rows * weight_rows * input_channels, "OP", s);
    prof.shape(input_rows, weight_rows, input_channels, "convt");
    hip_check(dav2_hip_gemm_i8(&a, s), "transposed convolution GEMM");
}

// src/operators.cpp:1978-2012
void HipOperators::bilinear_align_true(DeviceBuffer& output, const DeviceBuffer& input, std::uint32_t input_width,
                                       std::uint32_t input_height, std::uint32_t output_width,
                                       std::uint32_t output_height, std::uint32_t channels) {
    if (input_width == 0 || input_height == 0 || output_width == 0 || output_height == 0 || channels == 0)
        throw std::invalid_argument("invalid bilinear dimensions");
    require_bytes(input, std::uint64_t(input_width) * input_height * channels, "bilinear input");
    require_bytes(output, std::uint64_t(output_width) * output_height * channels, "bilinear output");
    ProfileScope prof(context_.profiler(), "bilinear",
                      4.0 * channels * (double(input_width) * input_height + double(output_width) * output_height), "B",
                      stream());
    hip_check(dav2_hip_bilinear_align_true(output.as<float>(), input.as<float>(), input_width, input_height,
                                           output_width, output_height, channels, stream()),
              "bilinear");
}

// src/operators.cpp:2050-2071
void HipOperators::bilinear_align_true_maxima(DeviceBuffer& output, DeviceBuffer& maxima, const DeviceBuffer& input,
                                              std::uint32_t input_width, std::uint32_t input_height,
                                              std::uint32_t output_width, std::uint32_t output_height,
                                              std::uint32_t channels) {
    if (input_width == 0 || input_height == 0 || output_width == 0 || output_height == 0 || channels == 0 ||
        channels % 32u)
        throw std::invalid_argument("invalid bilinear dimensions");
    require_bytes(input, std::uint64_t(input_width) * input_height * channels, "bilinear input");
    require_bytes(output, std::uint64_t(output_width) * output_height * channels, "bilinear output");
    require_bytes(maxima, std::uint64_t(output_width) * output_height * (channels / 32u), "bilinear maxima");
    ProfileScope prof(context_.profiler(), "bilinear",
                      4.0 * channels * (double(input_width) * input_height + double(output_width) * output_height), "B",
                      stream());
    hip_check(dav2_hip_bilinear_align_true_maxima(output.as<float>(), maxima.as<float>(), input.as<float>(),
                                                  input_width, input_height, output_width, output_height, channels,
                                                  stream()),
              "bilinear");
}

void HipOperators::reduce_minmax(const DeviceBuffer& input, DeviceBuffer& range, std::uint32_t count) {
    if (count == 0) throw std::invalid_argument("empty depth reduction");
    require_bytes(input, count, "depth reduction input");
    require_bytes(range, 2, "depth reduction range");
    grow(minmax_partials_, std::uint64_t(dav2_hip_minmax_partials(count)) * 2 * sizeof(float));
    ProfileScope prof(context_.profiler(), "reduce_minmax", 4.0 * count, "B", stream());
    hip_check(dav2_hip_reduce_minmax(input.as<float>(), count, range.as<float>(), minmax_partials_.as<float>(),
                                     stream()),
              "reduce_minmax");
}

void HipOperators::normalize_relative(DeviceBuffer& depth, const DeviceBuffer& range, std::uint32_t count) {
    if (count == 0) throw std::invalid_argument("empty relative depth");
    require_bytes(depth, count, "relative depth");
    require_bytes(range, 2, "relative depth range");
    ProfileScope prof(context_.profiler(), "normalize_relative", 8.0 * count, "B", stream());
    hip_check(dav2_hip_normalize_relative(depth.as<float>(), range.as<float>(), count, stream()),
              "normalize_relative");
}

// src/operators.cpp:2092-2130
void HipOperators::relu(DeviceBuffer& output, const DeviceBuffer& input, std::uint32_t count) {
    require_bytes(output, count, "ReLU output");
    require_bytes(input, count, "ReLU input");
    ProfileScope prof(context_.profiler(), "relu", 8.0 * count, "B", stream());
    hip_check(dav2_hip_relu(output.as<float>(), input.as<float>(), count, stream()), "relu");
}

void HipOperators::add(DeviceBuffer& output, const DeviceBuffer& left, const DeviceBuffer& right,
                       std::uint32_t count) {
    require_bytes(output, count, "add output");
    require_bytes(left, count, "add left");
    require_bytes(right, count, "add right");
    ProfileScope prof(context_.profiler(), "add", 12.0 * count, "B", stream());
    hip_check(dav2_hip_add(output.as<float>(), left.as<float>(), right.as<float>(), count, stream()),
              "add");
}

void HipOperators::gelu(DeviceBuffer& output, const DeviceBuffer& input, std::uint32_t count) {
    require_bytes(output, count, "GELU output");
    require_bytes(input, count, "GELU input");
    hip_check(dav2_hip_gelu(output.as<float>(), input.as<float>(), count, stream()), "gelu");
}

}  // namespace dav2
