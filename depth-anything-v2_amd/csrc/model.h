// .dav2 weight file, memory-mapped read-only and validated before use.
//
// The on-disk format (64-byte header, 192-byte tensor records, optional
// 128-byte provenance record, 64-byte aligned little-endian float32 payloads)
// and its acceptance rules are those of the reference loader,
// src/model.cpp:27-320, written by tools/export_model.py:21-38. The class
// below is this build's own: it keeps the mapping alive, exposes the tensors
// as a name-sorted table of WeightRecord entries for the GPU upload, and
// records the provenance fields the C ABI reports (dav2_get_model_info).
#pragma once

#include "depth_anything_v2.h"

#include <cstddef>
#include <cstdint>
#include <string>
#include <string_view>
#include <vector>

namespace dav2 {

// One float32 tensor inside the mapping.
struct WeightRecord {
    std::string_view name;     // points into the mapping (NUL-terminated there)
    const float* values = nullptr;
    std::uint32_t rank = 0;    // 1..4
    std::uint64_t shape[4] = {0, 0, 0, 0};  // unused dimensions are 0
    std::uint64_t count = 0;   // product of the used dimensions
    std::uint32_t checksum = 0;  // CRC-32 (IEEE 802.3) the file stores for the payload

    std::uint64_t dim(std::uint32_t i) const { return i < 4 ? shape[i] : 0; }
};

// The optional provenance record ("DAV2META").
struct ModelProvenance {
    bool recorded = false;
    bool metric = false;
    float metric_max_depth = 0.0f;  // 20 or 80 for metric heads, else 0
    std::string converter;
};

// Malformed files throw std::runtime_error with the reference's message; the
// C ABI reports them as DAV2_STATUS_INTERNAL_ERROR (src/dav2.cpp:85-86).
class MappedModel {
public:
    MappedModel(const std::string& path_utf8, dav2_encoder expected_encoder);
    ~MappedModel();
    MappedModel(const MappedModel&) = delete;
    MappedModel& operator=(const MappedModel&) = delete;

    // Tensors in file order.
    const std::vector<WeightRecord>& records() const { return records_; }
    // Lookup by name (binary search over a name-sorted index); find() returns
    // nullptr for a missing name, at() throws.
    const WeightRecord* find(std::string_view name) const;
    const WeightRecord& at(std::string_view name) const;
    const ModelProvenance& provenance() const { return provenance_; }

private:
    void unmap() noexcept;

    int fd_ = -1;
    const std::byte* base_ = nullptr;
    std::uint64_t bytes_ = 0;
    std::vector<WeightRecord> records_;
    std::vector<std::uint32_t> by_name_;  // indices into records_, sorted by name
    ModelProvenance provenance_;
};

}  // namespace dav2
