// .dav2 model file: read-only mmap with bounded validation.
// Format and checks: reference src/model.{h,cpp} (header :27-69, checks
// :165-315) and tools/export_model.py:21-38.
#pragma once

#include "depth_anything_v2.h"

#include <array>
#include <cstddef>
#include <cstdint>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

namespace dav2 {

struct TensorView {
    const float* data = nullptr;
    std::array<std::uint64_t, 4> dimensions{};
    std::uint32_t rank = 0;
    std::uint64_t elements = 0;
    std::uint32_t crc32 = 0;
};

struct ModelDerivation {
    bool present = false;
    std::array<std::uint8_t, 32> canonical_sha256{};
    std::string converter;
    std::uint32_t format_version = 0;
    dav2_encoder encoder = DAV2_ENCODER_VITS;
    float metric_max_depth = 0.0f;
};

// Thrown for every malformed-file condition; the C ABI reports it as
// DAV2_STATUS_INTERNAL_ERROR like the reference (src/dav2.cpp:85-86).
class ModelFile {
public:
    ModelFile(const std::string& path_utf8, dav2_encoder expected_encoder);
    ~ModelFile();
    ModelFile(const ModelFile&) = delete;
    ModelFile& operator=(const ModelFile&) = delete;

    const TensorView& tensor(std::string_view name) const;
    bool contains(std::string_view name) const;
    std::size_t tensor_count() const { return tensors_.size(); }
    const std::vector<std::string_view>& tensor_names() const { return names_; }
    const ModelDerivation& derivation() const { return derivation_; }

private:
    void close() noexcept;

    int fd_ = -1;
    const std::byte* view_ = nullptr;
    std::uint64_t size_ = 0;
    std::unordered_map<std::string_view, TensorView> tensors_;
    std::vector<std::string_view> names_;
    ModelDerivation derivation_;
};

std::uint32_t crc32(const void* data, std::size_t bytes);

}  // namespace dav2
