#include "graph.h"

#include "dav2_hip.h"

#include <stdexcept>

namespace dav2 {

EncoderConfig encoder_config(dav2_encoder encoder) {
    switch (encoder) {
        case DAV2_ENCODER_VITS: return {384, 6, 12, {2, 5, 8, 11}};
        case DAV2_ENCODER_VITB: return {768, 12, 12, {2, 5, 8, 11}};
        case DAV2_ENCODER_VITL: return {1024, 16, 24, {4, 11, 17, 23}};
    }
    throw std::invalid_argument("unsupported DINOv2 encoder");
}

DptConfig dpt_config(dav2_encoder encoder) {
    switch (encoder) {
        case DAV2_ENCODER_VITS: return {384, 64, {48, 96, 192, 384}};
        case DAV2_ENCODER_VITB: return {768, 128, {96, 192, 384, 768}};
        case DAV2_ENCODER_VITL: return {1024, 256, {256, 512, 1024, 1024}};
    }
    throw std::invalid_argument("unsupported DPT encoder");
}

DeviceBuffer& Arena::get(const std::string& name, std::uint64_t bytes) {
    DeviceBuffer& b = buffers_[name];
    if (b.size() < bytes) {
        hip_check(hipDeviceSynchronize(), "arena grow");
        b.reset();
        b = DeviceBuffer(bytes);
    }
    return b;
}

std::uint64_t Arena::bytes() const {
    std::uint64_t total = 0;
    for (const auto& kv : buffers_) total += kv.second.size();
    return total;
}

namespace {
std::string block_name(std::uint32_t block, const char* suffix) {
    return "pretrained.blocks." + std::to_string(block) + suffix;
}
}  // namespace

// ---------------------------------------------------------------------------
DinoEncoder::DinoEncoder(dav2_encoder encoder, GpuModel& weights, HipOperators& operators,
                         AttentionMode attention, Precision precision)
    : config_(encoder_config(encoder)), weights_(weights), ops_(operators),
      attention_(attention), precision_(precision) {
    if (weights_.tensor("pretrained.cls_token").elements != config_.embedding ||
        weights_.tensor("pretrained.pos_embed").elements != std::uint64_t(1370) * config_.embedding)
        throw std::runtime_error("encoder tensor dimensions do not match");
}

const DeviceBuffer& DinoEncoder::fp32(const std::string& name) const { return weights_.tensor(name).buffer; }

void DinoEncoder::forward(const float* image, std::uint32_t width, std::uint32_t height, std::uint32_t batch,
                          Arena& arena, DeviceBuffer* features[4],
                          const std::function<void(std::uint32_t)>& on_capture) {
    if (width == 0 || height == 0 || width % 14 != 0 || height % 14 != 0 || batch == 0)
        throw std::invalid_argument("encoder dimensions must be positive multiples of 14");
    const std::uint32_t D = config_.embedding, H = config_.heads;
    const std::uint32_t pw = width / 14, ph = height / 14, T = pw * ph + 1;
    const std::uint64_t rows64 = std::uint64_t(T) * batch;
    if (rows64 > 0x7fffffffull) throw std::invalid_argument("token batch too large");
    const std::uint32_t rows = static_cast<std::uint32_t>(rows64);
    const std::uint64_t tok_bytes = rows64 * D * sizeof(float);
    DeviceBuffer& current = arena.get("enc.current", tok_bytes);
    DeviceBuffer& qkv = arena.get("enc.qkv", tok_bytes * 3);
    DeviceBuffer& attn = arena.get("enc.attention", tok_bytes);
    DeviceBuffer& hidden = arena.get("enc.hidden", tok_bytes * 4);
    const bool f32 = precision_ != Precision::int8;  // fp32 or fp16 mode: the float path
    const bool fused = !f32 && attention_ == AttentionMode::exact;
    const bool coop = attention_ == AttentionMode::binary16_coop;
    const Precision materialised =
        attention_ == AttentionMode::binary16 || coop ? Precision::fp16 : Precision::fp32;
    DeviceBuffer& scores =
        arena.get("enc.scores", fused ? HipOperators::attention_fused_scratch_bytes(T, H, batch)
                                      : HipOperators::attention_score_bytes(T, H, batch, materialised));
    for (int i = 0; i < 4; ++i) features[i] = &arena.get("enc.feature" + std::to_string(i), tok_bytes);
    // One image: the qkv GEMM also leaves the |k| and |v| column maxima per
    // row tile, so the attention's digit packing reads qkv once.
    const bool colmax = fused && batch == 1;
    const std::uint32_t qkv_tiles = colmax ? HipOperators::gemm_row_tiles(rows, 3 * D) : 0;
    DeviceBuffer* col_absmax =
        colmax ? &arena.get("enc.qkv_colmax", std::uint64_t(qkv_tiles) * 2 * D * sizeof(float)) : nullptr;

    // Patch embedding + class token + position (operators.cpp:1211-1406), one
    // image at a time into rows [b*T, (b+1)*T).
    const GpuTensor& patch = weights_.tensor("pretrained.patch_embed.proj.weight");
    const std::uint64_t image_elems = std::uint64_t(width) * height * 3;
    for (std::uint32_t b = 0; b < batch; ++b) {
        DeviceBuffer img = DeviceBuffer::view(const_cast<float*>(image) + b * image_elems, image_elems * sizeof(float));
        DeviceBuffer out = DeviceBuffer::view(current.as<float>() + std::uint64_t(b) * T * D,
                                              std::uint64_t(T) * D * sizeof(float));
        ops_.prepare_tokens(out, img, patch.buffer, DeviceBuffer(), patch.int8_buffer, patch.int8_scales,
                            fp32("pretrained.patch_embed.proj.bias"), fp32("pretrained.cls_token"),
                            fp32("pretrained.pos_embed"), width, height, D, precision_,
                            /*position_is_constant=*/true);
    }
    if (f32) {
        forward_fp32(rows, T, batch, arena, current, qkv, attn, hidden, scores, features, on_capture);
        return;
    }

    std::uint32_t capture = 0;
    for (std::uint32_t blk = 0; blk < config_.blocks; ++blk) {
        const auto W = [&](const char* s) -> const GpuTensor& { return weights_.tensor(block_name(blk, s)); };
        const auto F = [&](const char* s) -> const DeviceBuffer& { return fp32(block_name(blk, s)); };
        // norm1 -> qkv (encoder.cpp:443-452)
        ops_.layer_norm_quantize(current, F(".norm1.weight"), F(".norm1.bias"), rows, D, 1.0e-6f, nullptr);
        const GpuTensor& wqkv = W(".attn.qkv.weight");
        ops_.linear_int8_prequantized(qkv, wqkv.int8_buffer, wqkv.int8_scales, &F(".attn.qkv.bias"), rows, D, 3 * D,
                                      colmax ? HipOperators::Epilogue::row_colmax : HipOperators::Epilogue::row,
                                      nullptr, 0, col_absmax, D);
        // attention (encoder.cpp:454-460): the integer-exact fused kernel, or
        // the reference's materialised binary16 / fp32 pipeline in its own
        // arithmetic order
        if (fused)
            ops_.attention_fused(attn, qkv, T, H, batch, scores, col_absmax, qkv_tiles);
        else
            ops_.attention_batched(attn, qkv, T, H, batch, scores, materialised, coop);
        // proj + LayerScale residual (encoder.cpp:478-491), in place
        ops_.quantize_rows(attn, 0, rows, D);
        const GpuTensor& wproj = W(".attn.proj.weight");
        ops_.linear_int8_prequantized(current, wproj.int8_buffer, wproj.int8_scales, &F(".attn.proj.bias"), rows, D, D,
                                      HipOperators::Epilogue::row_layerscale, &F(".ls1.gamma"));
        // norm2 -> fc1 + GELU (encoder.cpp:500-529). From 4096 rows (batch 3
        // at 518) the GELU runs in fc2's row quantizer instead of fc1's
        // epilogue, bit-identical: at 10960 rows fc1 86 instead of 118 us,
        // the quantizer 58 instead of about 32 (VALU-bound, about 47 IEEE
        // operations per value), the pass 1.2% faster. At one image the
        // quantizer has too few waves and the epilogue's GELU overlaps other
        // tiles' main loops, so the epilogue keeps it.
        const bool gelu_in_quantizer = rows >= 4096;
        ops_.layer_norm_quantize(current, F(".norm2.weight"), F(".norm2.bias"), rows, D, 1.0e-6f, nullptr);
        const GpuTensor& wfc1 = W(".mlp.fc1.weight");
        ops_.linear_int8_prequantized(hidden, wfc1.int8_buffer, wfc1.int8_scales, &F(".mlp.fc1.bias"), rows, D, 4 * D,
                                      gelu_in_quantizer ? HipOperators::Epilogue::row
                                                        : HipOperators::Epilogue::row_gelu);
        // fc2 + LayerScale residual (encoder.cpp:560-574), in place
        ops_.quantize_rows(hidden, 0, rows, 4 * D, gelu_in_quantizer);
        const GpuTensor& wfc2 = W(".mlp.fc2.weight");
        ops_.linear_int8_prequantized(current, wfc2.int8_buffer, wfc2.int8_scales, &F(".mlp.fc2.bias"), rows, 4 * D, D,
                                      HipOperators::Epilogue::row_layerscale, &F(".ls2.gamma"));
        // captured features (encoder.cpp:576-589)
        if (capture < 4 && blk == config_.capture[capture]) {
            ops_.layer_norm(*features[capture], current, fp32("pretrained.norm.weight"), fp32("pretrained.norm.bias"),
                            rows, D, 1.0e-6f);
            if (on_capture) on_capture(capture);
            ++capture;
        }
    }
    if (capture != 4) throw std::runtime_error("encoder did not produce four features");
}

void DinoEncoder::forward_fp32(std::uint32_t rows, std::uint32_t T, std::uint32_t batch, Arena& arena,
                               DeviceBuffer& current, DeviceBuffer& qkv, DeviceBuffer& attn, DeviceBuffer& hidden,
                               DeviceBuffer& scores, DeviceBuffer* features[4],
                               const std::function<void(std::uint32_t)>& on_capture) {
    // encoder.cpp:407-597 in the fp32 precision mode: LayerNorm rows in fp32,
    // fp32 GEMMs (GELU and the LayerScale residual in their epilogues, the
    // arithmetic of the reference's separate gelu / add_scaled passes),
    // materialised fp32 attention. The fp16 mode (encoder.cpp:428-546): the
    // same with the GEMM operands rounded to binary16 (layer_norm_fp16 and
    // pack_fp16 produce binary16 inputs, fc1's output is stored as binary16
    // and fc2 reads it) and the reference's binary16 attention, or its fp32
    // attention under FORCE_FP32_ATTENTION, both in the shaders' order.
    const std::uint32_t D = config_.embedding, H = config_.heads;
    const bool half = precision_ == Precision::fp16;
    DeviceBuffer& normed = arena.get("enc.normed", std::uint64_t(rows) * D * sizeof(float));
    using E = HipOperators::Epilogue;
    std::uint32_t capture = 0;
    for (std::uint32_t blk = 0; blk < config_.blocks; ++blk) {
        const auto W = [&](const char* s) -> const DeviceBuffer& { return weights_.tensor(block_name(blk, s)).buffer; };
        ops_.layer_norm(normed, current, W(".norm1.weight"), W(".norm1.bias"), rows, D, 1.0e-6f);
        ops_.linear_f32(qkv, normed, W(".attn.qkv.weight"), &W(".attn.qkv.bias"), rows, D, 3 * D, E::row, nullptr, 0,
                        half);
        if (!half)
            ops_.attention_mfma_f32(attn, qkv, T, H, batch, scores);
        else
            ops_.attention_batched(attn, qkv, T, H, batch, scores,
                                   attention_ == AttentionMode::fp32 ? Precision::fp32 : Precision::fp16,
                                   attention_ == AttentionMode::binary16_coop);
        ops_.linear_f32(current, attn, W(".attn.proj.weight"), &W(".attn.proj.bias"), rows, D, D, E::row_layerscale,
                        &W(".ls1.gamma"), 0, half);
        ops_.layer_norm(normed, current, W(".norm2.weight"), W(".norm2.bias"), rows, D, 1.0e-6f);
        ops_.linear_f32(hidden, normed, W(".mlp.fc1.weight"), &W(".mlp.fc1.bias"), rows, D, 4 * D, E::row_gelu,
                        nullptr, 0, half);
        ops_.linear_f32(current, hidden, W(".mlp.fc2.weight"), &W(".mlp.fc2.bias"), rows, 4 * D, D, E::row_layerscale,
                        &W(".ls2.gamma"), 0, half);
        if (capture < 4 && blk == config_.capture[capture]) {
            ops_.layer_norm(*features[capture], current, fp32("pretrained.norm.weight"), fp32("pretrained.norm.bias"),
                            rows, D, 1.0e-6f);
            if (on_capture) on_capture(capture);
            ++capture;
        }
    }
    if (capture != 4) throw std::runtime_error("encoder did not produce four features");
}

// ---------------------------------------------------------------------------
DptHead::DptHead(dav2_encoder encoder, GpuModel& weights, HipOperators& operators, Precision precision)
    : config_(dpt_config(encoder)), weights_(weights), ops_(operators), zero_bias_(sizeof(float)),
      precision_(precision) {
    hip_check(hipMemsetAsync(zero_bias_.data(), 0, sizeof(float), ops_.context().active_stream()), "zero bias");
}

FeatureMap DptHead::conv(HipOperators& ops, const FeatureMap& in, const std::string& weight, const std::string& bias,
                         std::uint32_t oc, std::uint32_t k, std::uint32_t stride, std::uint32_t pad, bool has_bias,
                         Arena& arena, const std::string& slot, const ConvFusion& fusion, Emit emit) {
    // dpt.cpp:479-535, every convolution through conv2d_int8
    FeatureMap out;
    out.width = (in.width + 2 * pad - k) / stride + 1;
    out.height = (in.height + 2 * pad - k) / stride + 1;
    out.channels = oc;
    out.buffer = &arena.get(slot + suffix_, out.elements() * sizeof(float));
    const GpuTensor& w = weights_.tensor(weight);
    const DeviceBuffer& b = has_bias ? weights_.tensor(bias).buffer : zero_bias_;
    if (precision_ != Precision::int8) {
        // fp32, or fp16 through the reference's conv2d route with half
        // weights (dpt.cpp:507-517): fp32 arithmetic on binary16 weights
        ops.conv2d(*out.buffer, *in.buffer, w.buffer, b, in.width, in.height, in.channels, oc, k, stride, pad, has_bias,
                   fusion);
        return out;
    }
    if (!w.int8_buffer) throw std::runtime_error("convolution weight is not int8: " + weight);
    // Group maxima: the input's when its producer wrote them in the mode this
    // convolution reads (max(x, 0) under an input ReLU); the output's when
    // the consumer asked (same values as computing them afterwards: max is
    // exact and order-free).
    ConvFusion f = fusion;
    if (in.maxima && in.maxima_relu == f.relu_input) f.input_maxima = in.maxima;
    DeviceBuffer* maxima = nullptr;
    if (emit != Emit::none && oc % 32 == 0) {
        maxima = &arena.get(slot + suffix_ + ".max", std::uint64_t(oc / 32) * out.width * out.height * sizeof(float));
        f.emit_maxima = maxima;
        f.emit_relu = emit == Emit::relu;
    }
    if (ops.conv2d_int8(*out.buffer, *in.buffer, w.int8_buffer, w.int8_scales, b, in.width, in.height, in.channels, oc,
                        k, stride, pad, has_bias, &w.int8_packed, f)) {
        out.maxima = maxima;
        out.maxima_relu = emit == Emit::relu;
    }
    return out;
}

FeatureMap DptHead::resize(HipOperators& ops, const FeatureMap& in, std::uint32_t ow, std::uint32_t oh, Arena& arena,
                           const std::string& slot, std::uint32_t consumer_channels, std::uint32_t consumer_kernel) {
    FeatureMap out{&arena.get(slot + suffix_, std::uint64_t(ow) * oh * in.channels * sizeof(float)), ow, oh,
                   in.channels};
    const std::uint32_t pad = (consumer_kernel - 1) / 2;
    if (precision_ == Precision::int8 && in.channels % 32 == 0 &&
        HipOperators::implicit_conv(ow, oh, in.channels, consumer_channels, consumer_kernel, 1, pad)) {
        out.maxima = &arena.get(slot + suffix_ + ".max", std::uint64_t(in.channels / 32) * ow * oh * sizeof(float));
        ops.bilinear_align_true_maxima(*out.buffer, *out.maxima, *in.buffer, in.width, in.height, ow, oh, in.channels);
        return out;
    }
    ops.bilinear_align_true(*out.buffer, *in.buffer, in.width, in.height, ow, oh, in.channels);
    return out;
}

FeatureMap DptHead::residual_unit(HipOperators& ops, const FeatureMap& in, const std::string& prefix, Arena& arena,
                                  const std::string& temp_slot, const std::string& slot) {
    // dpt.cpp:537-572: relu -> conv3x3 -> relu -> conv3x3 -> + input, the
    // ReLUs and the residual add folded into the two convolutions.
    ConvFusion first_fusion;
    first_fusion.relu_input = true;
    first_fusion.relu_output = true;
    const bool second_implicit =
        HipOperators::implicit_conv(in.width, in.height, in.channels, in.channels, 3, 1, 1);
    FeatureMap first = conv(ops, in, prefix + ".conv1.weight", prefix + ".conv1.bias", in.channels, 3, 1, 1, true, arena,
                            temp_slot, first_fusion, second_implicit ? Emit::absolute : Emit::none);
    ConvFusion second_fusion;
    second_fusion.residual = in.buffer;
    return conv(ops, first, prefix + ".conv2.weight", prefix + ".conv2.bias", in.channels, 3, 1, 1, true, arena, slot,
                second_fusion);
}

FeatureMap DptHead::fusion(HipOperators& ops, const FeatureMap& path, const std::string& prefix, std::uint32_t ow,
                           std::uint32_t oh, const FeatureMap* next_skip, Arena& arena, const std::string& slot,
                           bool next_is_head) {
    // dpt.cpp:574-615 from resConfUnit2 on: the path arrives with this
    // refinenet's processed skip already added (by the previous out_conv).
    const std::uint32_t F = config_.features;
    FeatureMap unit = residual_unit(ops, path, prefix + ".resConfUnit2", arena, "dpt.ru.first", "dpt.fu.unit");
    FeatureMap resized = resize(ops, unit, ow, oh, arena, "dpt.fu.resized", F, 1);
    // path + processed skip of the next refinenet (add.glsl; a + b == b + a).
    // The output feeds the next refinenet's residual unit (input ReLU) or
    // the head's output_conv1.
    ConvFusion add_skip;
    add_skip.residual = next_skip ? next_skip->buffer : nullptr;
    const std::uint32_t next_oc = next_is_head ? F / 2 : F;
    const Emit emit = !HipOperators::implicit_conv(ow, oh, F, next_oc, 3, 1, 1) ? Emit::none
                      : next_is_head                                         ? Emit::absolute
                                                                             : Emit::relu;
    return conv(ops, resized, prefix + ".out_conv.weight", prefix + ".out_conv.bias", F, 1, 1, 0, true, arena, slot,
                add_skip, emit);
}

FeatureMap DptHead::prepare_level(std::uint32_t i, const DeviceBuffer& feature, std::uint32_t b, std::uint32_t pw,
                                  std::uint32_t ph, Arena& arena, HipOperators& ops) {
    const std::uint32_t D = config_.embedding, T = pw * ph + 1;
    // Projection and resize layer (dpt.cpp:635-736).
    const std::string prefix = "depth_head.projects." + std::to_string(i);
    const GpuTensor& w = weights_.tensor(prefix + ".weight");
    FeatureMap proj{&arena.get("dpt.proj" + std::to_string(i) + suffix_,
                               std::uint64_t(pw) * ph * config_.project[i] * sizeof(float)),
                    pw, ph, config_.project[i]};
    DeviceBuffer tokens = DeviceBuffer::view(feature.as<float>() + std::uint64_t(b) * T * D,
                                             std::uint64_t(T) * D * sizeof(float));
    if (precision_ == Precision::fp32)
        ops.project_tokens(*proj.buffer, tokens, w.buffer, weights_.tensor(prefix + ".bias").buffer, pw, ph, D,
                           config_.project[i]);
    else if (precision_ == Precision::fp16)
        ops.project_tokens_fp16(*proj.buffer, tokens, w.buffer, weights_.tensor(prefix + ".bias").buffer, pw, ph, D,
                                config_.project[i]);
    else
        ops.project_tokens_int8(*proj.buffer, tokens, w.int8_buffer, w.int8_scales,
                                weights_.tensor(prefix + ".bias").buffer, pw, ph, D, config_.project[i]);
    FeatureMap layer;
    if (i < 2) {
        const std::uint32_t k = i == 0 ? 4 : 2;
        const std::string r = "depth_head.resize_layers." + std::to_string(i);
        const GpuTensor& rw = weights_.tensor(r + ".weight");
        layer = FeatureMap{&arena.get("dpt.layer" + std::to_string(i) + suffix_,
                                      std::uint64_t(pw) * k * ph * k * proj.channels * sizeof(float)),
                           pw * k, ph * k, proj.channels};
        if (precision_ == Precision::fp32)
            ops.conv_transpose_nonoverlap(*layer.buffer, *proj.buffer, rw.buffer, weights_.tensor(r + ".bias").buffer,
                                          pw, ph, proj.channels, proj.channels, k);
        else if (precision_ == Precision::fp16)
            ops.conv_transpose_nonoverlap_fp16(*layer.buffer, *proj.buffer, rw.buffer,
                                               weights_.tensor(r + ".bias").buffer, pw, ph, proj.channels,
                                               proj.channels, k);
        else
            ops.conv_transpose_nonoverlap_int8(*layer.buffer, *proj.buffer, rw.int8_buffer, rw.int8_scales,
                                               weights_.tensor(r + ".bias").buffer, pw, ph, proj.channels,
                                               proj.channels, k);
    } else if (i == 2) {
        layer = proj;
    } else {
        layer = conv(ops, proj, "depth_head.resize_layers.3.weight", "depth_head.resize_layers.3.bias",
                     config_.project[3], 3, 2, 1, true, arena, "dpt.layer3");
    }
    // layer*_rn (dpt.cpp:743-756)
    const std::string level = std::to_string(i);
    // levels 0-2 feed the first residual unit of a refinenet (input ReLU)
    const bool unit_implicit = i < 3 && HipOperators::implicit_conv(layer.width, layer.height, config_.features,
                                                                    config_.features, 3, 1, 1);
    FeatureMap rn = conv(ops, layer, "depth_head.scratch.layer" + std::to_string(i + 1) + "_rn.weight", "",
                         config_.features, 3, 1, 1, false, arena, "dpt.rn" + level, ConvFusion{},
                         unit_implicit ? Emit::relu : Emit::none);
    if (i == 3) return rn;
    // refinenet(i+1).resConfUnit1 on this level (dpt.cpp:574-590): its own
    // arena slots, so it may run beside the other levels
    return residual_unit(ops, rn, "depth_head.scratch.refinenet" + std::to_string(i + 1) + ".resConfUnit1", arena,
                         "dpt.ru.first" + level, "dpt.skip" + level);
}

void DptHead::refine_and_head(const FeatureMap refined[4], std::uint32_t b, std::uint32_t pw, std::uint32_t ph,
                              Arena& arena, float* depth, float* pre_relu, HipOperators* ops_in) {
    HipOperators& ops = ops_in ? *ops_in : ops_;
    const std::uint32_t F = config_.features;
    // refinenets (dpt.cpp:759-790); refined[0..2] are the processed skip
    // inputs of refinenet1..3, refined[3] the deepest level. Outputs
    // alternate between two slots.
    FeatureMap path = fusion(ops, refined[3], "depth_head.scratch.refinenet4", refined[2].width, refined[2].height,
                             &refined[2], arena, "dpt.pathA");
    path = fusion(ops, path, "depth_head.scratch.refinenet3", refined[1].width, refined[1].height, &refined[1], arena,
                  "dpt.pathB");
    path = fusion(ops, path, "depth_head.scratch.refinenet2", refined[0].width, refined[0].height, &refined[0], arena,
                  "dpt.pathA");
    path = fusion(ops, path, "depth_head.scratch.refinenet1", refined[0].width * 2, refined[0].height * 2, nullptr, arena,
                  "dpt.pathB", /*next_is_head=*/true);
    // output head (dpt.cpp:792-855)
    path = conv(ops, path, "depth_head.scratch.output_conv1.weight", "depth_head.scratch.output_conv1.bias", F / 2, 3,
                1, 1, true, arena, "dpt.out1");
    FeatureMap full = resize(ops, path, pw * 14, ph * 14, arena, "dpt.full", 32, 3);
    ConvFusion relu_after;
    relu_after.relu_output = true;
    FeatureMap head = conv(ops, full, "depth_head.scratch.output_conv2.0.weight", "depth_head.scratch.output_conv2.0.bias",
                           32, 3, 1, 1, true, arena, "dpt.out2", relu_after);
    // output_conv2.2 (1x1, 32 -> 1) and the final ReLU in one pass; the
    // pre-ReLU logits go to pre_relu when asked.
    const std::uint64_t pixels = std::uint64_t(pw) * 14 * ph * 14;
    DeviceBuffer out = DeviceBuffer::view(depth + b * pixels, pixels * sizeof(float));
    DeviceBuffer logits;
    if (pre_relu) logits = DeviceBuffer::view(pre_relu, pixels * sizeof(float));
    const GpuTensor& w3 = weights_.tensor("depth_head.scratch.output_conv2.2.weight");
    if (precision_ != Precision::int8) {
        const DeviceBuffer& b3 = weights_.tensor("depth_head.scratch.output_conv2.2.bias").buffer;
        if (logits) {
            ops.conv2d(logits, *head.buffer, w3.buffer, b3, head.width, head.height, head.channels, 1, 1, 1, 0, true);
            ops.relu(out, logits, static_cast<std::uint32_t>(pixels));
        } else {
            ops.conv2d(out, *head.buffer, w3.buffer, b3, head.width, head.height, head.channels, 1, 1, 1, 0, true,
                        relu_after);
        }
        return;
    }
    if (!w3.int8_buffer) throw std::runtime_error("output_conv2.2 weight is not int8");
    ops.conv1x1_narrow_int8(out, *head.buffer, w3.int8_buffer, w3.int8_ld, w3.int8_scales,
                             weights_.tensor("depth_head.scratch.output_conv2.2.bias").buffer, head.width, head.height,
                             head.channels, 1, true, relu_after, logits ? &logits : nullptr);
}

void DptHead::forward(DeviceBuffer* features[4], std::uint32_t pw, std::uint32_t ph, std::uint32_t batch,
                      Arena& arena, float* depth, float* pre_relu) {
    for (std::uint32_t b = 0; b < batch; ++b) {
        FeatureMap refined[4];
        for (std::uint32_t i = 0; i < 4; ++i) refined[i] = prepare_level(i, *features[i], b, pw, ph, arena, ops_);
        refine_and_head(refined, b, pw, ph, arena, depth, b + 1 == batch ? pre_relu : nullptr);
    }
}

}  // namespace dav2
