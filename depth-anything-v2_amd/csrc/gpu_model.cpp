#include "gpu_model.h"

#include "dav2_hip.h"

#include <memory>
#include <stdexcept>
#include <vector>

#include <zlib.h>

namespace dav2 {

namespace {

bool ends_with(std::string_view s, std::string_view suffix) {
    return s.size() >= suffix.size() && s.substr(s.size() - suffix.size()) == suffix;
}

bool quantizable_family(std::string_view name) {
    // src/gpu_model.cpp:16-33: patch embedding, every DPT weight, and the
    // attention/MLP weights of the transformer blocks.
    if (!ends_with(name, ".weight")) return false;
    if (name == "pretrained.patch_embed.proj.weight" || name.rfind("depth_head.", 0) == 0) return true;
    if (name.rfind("pretrained.blocks.", 0) != 0) return false;
    return name.find(".attn.") != std::string_view::npos || name.find(".mlp.") != std::string_view::npos;
}

std::uint32_t fast_crc32(const void* data, std::uint64_t bytes) {
    // zlib's CRC-32 is the IEEE 802.3 polynomial/reflection the .dav2 format stores
    // (IEEE 802.3), just faster; fed in <4 GiB pieces.
    uLong c = ::crc32(0L, Z_NULL, 0);
    const auto* p = static_cast<const Bytef*>(data);
    while (bytes > 0) {
        const uInt chunk = static_cast<uInt>(bytes > (1u << 30) ? (1u << 30) : bytes);
        c = ::crc32(c, p, chunk);
        p += chunk;
        bytes -= chunk;
    }
    return static_cast<std::uint32_t>(c);
}

}  // namespace

bool transposed_convolution_weight(std::string_view name) {
    return name == "depth_head.resize_layers.0.weight" || name == "depth_head.resize_layers.1.weight";
}

bool use_int8_weight(std::string_view name, const WeightRecord& t) {
    // src/gpu_model.cpp:35-44
    if (!quantizable_family(name) || t.shape[0] == 0) return false;
    if (t.rank == 2) return t.shape[1] % 4 == 0;
    if (t.rank != 4) return false;
    if (transposed_convolution_weight(name)) return t.shape[0] % 4 == 0;
    return (t.count / t.shape[0]) % 4 == 0;
}

GpuModel::GpuModel(const MappedModel& model, HipContext& context, Precision precision) {
    const bool fp32_weights = precision != Precision::int8;
    const bool half_weights = precision == Precision::fp16;
    tensors_.reserve(model.records().size());
    DeviceBuffer staging;
    std::vector<std::unique_ptr<std::vector<float>>> host_keepalive;
    const hipStream_t stream = context.active_stream();
    for (const WeightRecord& src : model.records()) {
        const std::string_view name = src.name;
        const std::uint64_t bytes = src.count * sizeof(float);
        if (fast_crc32(src.values, bytes) != src.checksum)
            throw std::runtime_error("model tensor checksum mismatch: " + std::string(name));
        GpuTensor dst;
        for (int d = 0; d < 4; ++d) dst.dimensions[d] = src.shape[d];
        dst.rank = src.rank;
        dst.elements = src.count;
        if (!use_int8_weight(name, src)) {
            dst.buffer = context.create_device_buffer(bytes);
            context.upload(dst.buffer, src.values, bytes);
            if (half_weights && quantizable_family(name))
                hip_check(dav2_hip_round_half(dst.buffer.as<float>(), src.count, stream), "half weights");
            device_bytes_ += bytes;
        } else {
            const bool convT = transposed_convolution_weight(name);
            const float* rows_source = src.values;
            std::uint64_t rows = 0, columns = 0;
            if (convT) {
                const std::uint64_t ic = src.shape[0], oc = src.shape[1], k = src.shape[2];
                if (src.rank != 4 || src.shape[3] != k) throw std::runtime_error("invalid ConvTranspose weight");
                rows = k * k * oc;
                columns = ic;
                auto reordered = std::make_unique<std::vector<float>>(rows * columns);
                for (std::uint64_t r = 0; r < rows; ++r) {
                    const std::uint64_t kidx = r / oc, o = r % oc, ky = kidx / k, kx = kidx % k;
                    for (std::uint64_t c = 0; c < ic; ++c)
                        (*reordered)[r * columns + c] = src.values[((c * oc + o) * k + ky) * k + kx];
                }
                rows_source = reordered->data();
                host_keepalive.push_back(std::move(reordered));
            } else {
                rows = src.shape[0];
                columns = src.count / rows;
            }
            if (rows > 0xffffffffull || columns > 0xffffffffull) throw std::runtime_error("weight too large");
            if (fp32_weights) {
                dst.f32_rows = static_cast<std::uint32_t>(rows);
                dst.f32_columns = static_cast<std::uint32_t>(columns);
                dst.buffer = context.create_device_buffer(bytes);
                context.upload(dst.buffer, rows_source, bytes);  // host copies live until the final sync
                if (half_weights)
                    hip_check(dav2_hip_round_half(dst.buffer.as<float>(), src.count, stream), "half weights");
                device_bytes_ += bytes;
                if (!tensors_.emplace(std::string(name), std::move(dst)).second)
                    throw std::runtime_error("duplicate GPU tensor name: " + std::string(name));
                continue;
            }
            dst.int8_rows = static_cast<std::uint32_t>(rows);
            dst.int8_columns = static_cast<std::uint32_t>(columns);
            dst.int8_ld = padded_k(columns);
            if (staging.size() < bytes) {
                context.synchronize();
                staging = context.create_device_buffer(bytes);
            }
            hip_check(hipMemcpyAsync(staging.data(), rows_source, bytes, hipMemcpyHostToDevice, stream),
                      "weight upload");
            dst.int8_buffer = context.create_device_buffer(static_cast<std::size_t>(rows) * dst.int8_ld);
            dst.int8_scales = context.create_device_buffer(rows * sizeof(float));
            // The per-row weight rule (gpu_model.cpp:241-264: max|w|/127 floored
            // at 1e-8, nearbyint(clamp(w/s))) is the activation row quantizer.
            hip_check(dav2_hip_quantize_rows_i8(staging.as<float>(), 0, dst.int8_rows, dst.int8_columns,
                                                dst.int8_buffer.as<int8_t>(), dst.int8_ld,
                                                dst.int8_scales.as<float>(), stream),
                      "weight quantization");
            device_bytes_ += rows * dst.int8_ld + rows * sizeof(float);
            const std::uint64_t k = src.shape[2];
            if (!convT && src.rank == 4 && src.shape[3] == k &&
                dav2_hip_conv2d_i8_supported(1, 1, static_cast<std::uint32_t>(src.shape[1]),
                                             dst.int8_rows, static_cast<std::uint32_t>(k), 1,
                                             static_cast<std::uint32_t>((k - 1) / 2))) {
                dst.int8_packed = context.create_device_buffer(rows * columns);
                hip_check(dav2_hip_conv_weights_pack(dst.int8_packed.as<int8_t>(), dst.int8_buffer.as<int8_t>(),
                                                     dst.int8_rows, static_cast<std::uint32_t>(src.shape[1]),
                                                     static_cast<std::uint32_t>(k), dst.int8_ld, stream),
                          "packed conv weights");
                device_bytes_ += rows * columns;
            }
        }
        if (!tensors_.emplace(std::string(name), std::move(dst)).second)
            throw std::runtime_error("duplicate GPU tensor name: " + std::string(name));
    }
    context.synchronize();
}

const GpuTensor& GpuModel::tensor(std::string_view name) const {
    const auto it = tensors_.find(std::string(name));
    if (it == tensors_.end()) throw std::runtime_error("GPU model is missing tensor: " + std::string(name));
    return it->second;
}

}  // namespace dav2
