// Graph drivers: the DINOv2 encoder (reference src/encoder.cpp:322-597) and
// the DPT head (src/dpt.cpp:479-863) over the HIP operator surface.
//
// Differences in structure, not arithmetic, from the reference drivers:
//  - the encoder runs `batch` images at once (rows = batch * tokens);
//  - LayerNorm writes its quantized rows directly (no fp32 round trip), GELU
//    is fused into the fc1 GEMM epilogue and the LayerScale residual into the
//    proj/fc2 epilogues;
//  - every DPT convolution, 3x3 and 1x1, runs as an int8 convolution (the
//    reference's int8 mode sends only resize_layers.* through conv2d_int8 and
//    the refinement convolutions through fp16); in the fp32 precision mode
//    everything runs in fp32, as in the reference's, and the fp16 mode
//    follows the reference's fp16 routing (half weights, cooperative-matrix
//    linears, native binary16 projections, conv2d with half weights);
//  - buffers come from a grow-only arena, so a fixed resolution allocates only
//    on its first run.
#pragma once

#include "gpu_model.h"
#include "operators.h"

#include <functional>
#include <map>
#include <string>

namespace dav2 {

struct EncoderConfig {
    std::uint32_t embedding, heads, blocks;
    std::uint32_t capture[4];
};
struct DptConfig {
    std::uint32_t embedding, features;
    std::uint32_t project[4];
};
EncoderConfig encoder_config(dav2_encoder encoder);  // src/encoder.cpp:40-70
DptConfig dpt_config(dav2_encoder encoder);          // src/dpt.cpp:51-78

class Arena {
public:
    DeviceBuffer& get(const std::string& name, std::uint64_t bytes);
    std::uint64_t bytes() const;

private:
    std::map<std::string, DeviceBuffer> buffers_;
};

// Attention of the int8 graph: the integer-exact fused kernel (default), the
// reference's binary16 pipeline, or fp32 scores (FORCE_FP32_ATTENTION; also
// the fp32 precision mode, which uses the matrix-core fp32 kernels).
enum class AttentionMode { exact, binary16, binary16_coop, fp32 };

class DinoEncoder {
public:
    // precision: int8 (the product path) or fp32 (the fp32 precision mode:
    // fp32 weights and GEMMs, no quantization).
    DinoEncoder(dav2_encoder encoder, GpuModel& weights, HipOperators& operators, AttentionMode attention,
                Precision precision = Precision::int8);
    // image: device [batch][3][height][width]. On return features[i] holds the
    // final-norm token matrix [batch*tokens][D] of capture layer i.
    // on_capture(i), when given, runs right after the work producing
    // features[i] has been enqueued.
    void forward(const float* image, std::uint32_t width, std::uint32_t height, std::uint32_t batch, Arena& arena,
                 DeviceBuffer* features[4], const std::function<void(std::uint32_t)>& on_capture = {});
    const EncoderConfig& config() const { return config_; }

private:
    const DeviceBuffer& fp32(const std::string& name) const;
    void forward_fp32(std::uint32_t rows, std::uint32_t tokens, std::uint32_t batch, Arena& arena,
                      DeviceBuffer& current, DeviceBuffer& qkv, DeviceBuffer& attn, DeviceBuffer& hidden,
                      DeviceBuffer& scores, DeviceBuffer* features[4],
                      const std::function<void(std::uint32_t)>& on_capture);
    EncoderConfig config_;
    GpuModel& weights_;
    HipOperators& ops_;
    AttentionMode attention_;
    Precision precision_;
};

struct FeatureMap {
    DeviceBuffer* buffer = nullptr;
    std::uint32_t width = 0, height = 0, channels = 0;
    // Per-pixel 32-channel group maxima written by the producer for the next
    // convolution (of max(x, 0) when maxima_relu), or null.
    DeviceBuffer* maxima = nullptr;
    bool maxima_relu = false;
    std::uint64_t elements() const { return std::uint64_t(width) * height * channels; }
};

// Group maxima a convolution writes for its consumer.
enum class Emit { none, absolute, relu };

class DptHead {
public:
    DptHead(dav2_encoder encoder, GpuModel& weights, HipOperators& operators, Precision precision = Precision::int8);
    // features[i]: [batch*tokens][D]; writes batch raw depth maps
    // [batch][ph*14][pw*14] to depth. pre_relu (optional) receives the last
    // image's depth before the final ReLU.
    void forward(DeviceBuffer* features[4], std::uint32_t patch_width, std::uint32_t patch_height,
                 std::uint32_t batch, Arena& arena, float* depth, float* pre_relu = nullptr);

    // The two phases of forward for image b. prepare_level runs projection,
    // resize layer and layer*_rn of level i (its own arena slots, so the four
    // levels may run on different operator sets / streams) and, for levels
    // 0-2, the first residual unit of the refinenet that takes the level as
    // its skip input (it does not depend on the deeper levels), returning
    // that unit's output; refine_and_head runs the rest of the refinenets and
    // the output head on the main operator set.
    FeatureMap prepare_level(std::uint32_t level, const DeviceBuffer& feature, std::uint32_t b,
                             std::uint32_t patch_width, std::uint32_t patch_height, Arena& arena, HipOperators& ops);
    void refine_and_head(const FeatureMap refined[4], std::uint32_t b, std::uint32_t patch_width,
                         std::uint32_t patch_height, Arena& arena, float* depth, float* pre_relu,
                         HipOperators* ops = nullptr);
    // Appended to every arena slot name of the calls that follow, so that
    // two images' heads can be in flight on two streams at once.
    void set_slot_suffix(const std::string& suffix) { suffix_ = suffix; }

private:
    FeatureMap conv(HipOperators& ops, const FeatureMap& input, const std::string& weight, const std::string& bias,
                    std::uint32_t output_channels, std::uint32_t kernel, std::uint32_t stride, std::uint32_t padding,
                    bool has_bias, Arena& arena, const std::string& slot, const ConvFusion& fusion = ConvFusion{},
                    Emit emit = Emit::none);
    // Bilinear resize; with maxima for a following implicit convolution of
    // `consumer_channels` outputs and kernel `consumer_kernel`.
    FeatureMap resize(HipOperators& ops, const FeatureMap& input, std::uint32_t width, std::uint32_t height,
                      Arena& arena, const std::string& slot, std::uint32_t consumer_channels,
                      std::uint32_t consumer_kernel);
    FeatureMap residual_unit(HipOperators& ops, const FeatureMap& input, const std::string& prefix, Arena& arena,
                             const std::string& temp_slot, const std::string& slot);
    // Second residual unit, resize and out_conv of a refinenet; out_conv adds
    // next_skip (the next refinenet's processed skip input, the add of
    // dpt.cpp:574-615) when given.
    // next_is_head: the output feeds the head's output_conv1 (no input ReLU)
    // rather than the next refinenet's residual unit.
    FeatureMap fusion(HipOperators& ops, const FeatureMap& path, const std::string& prefix,
                      std::uint32_t output_width, std::uint32_t output_height, const FeatureMap* next_skip,
                      Arena& arena, const std::string& slot, bool next_is_head = false);

    DptConfig config_;
    GpuModel& weights_;
    HipOperators& ops_;
    DeviceBuffer zero_bias_;
    Precision precision_;
    std::string suffix_;
};

}  // namespace dav2
