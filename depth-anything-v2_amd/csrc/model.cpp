// .dav2 loader: map the file, check it section by section (header,
// provenance, tensor table), then index the tensors by name.
//
// Acceptance rules and messages follow src/model.cpp:98-320 (they are
// observable through dav2_last_error and are compared with the reference's
// own loader in the format tests); the on-disk layouts below are fixed by the
// format (src/model.cpp:27-69, tools/export_model.py:25-38).

#include "model.h"

#include <algorithm>
#include <cstring>
#include <limits>
#include <stdexcept>
#include <unordered_set>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace dav2 {
namespace {

#pragma pack(push, 1)
struct OnDiskHeader {
    char magic[8];  // "DAV2MOD\0"
    std::uint32_t version;
    std::uint32_t endian;  // 0x01020304 written little-endian
    std::uint32_t encoder;
    std::uint32_t tensor_count;
    std::uint64_t directory_offset;
    std::uint64_t directory_bytes;
    std::uint64_t data_offset;
    std::uint64_t file_bytes;
    std::uint64_t metadata_offset;  // 0: no provenance record
};
struct OnDiskTensor {
    char name[112];
    std::uint32_t dtype;  // 1: float32
    std::uint32_t rank;
    std::uint64_t dimensions[4];
    std::uint64_t data_offset;
    std::uint64_t data_bytes;
    std::uint64_t element_count;
    std::uint32_t crc32;
    std::uint32_t flags;
    std::uint64_t reserved;
};
struct OnDiskProvenance {
    char magic[8];  // "DAV2META"
    std::uint32_t version;
    std::uint32_t bytes;
    std::uint32_t model_format_version;
    std::uint32_t encoder;
    std::uint32_t flags;     // bit 0: metric head
    std::uint32_t reserved;  // metric head: float maximum depth
    std::uint8_t canonical_sha256[32];
    char converter[64];
};
#pragma pack(pop)
static_assert(sizeof(OnDiskHeader) == 64 && sizeof(OnDiskTensor) == 192 && sizeof(OnDiskProvenance) == 128,
              ".dav2 record sizes");

constexpr std::uint64_t kPayloadAlignment = 64;
constexpr std::uint32_t kMaxTensors = 2048;

[[noreturn]] void fail(const char* message) { throw std::runtime_error(message); }

// [offset, offset + length) lies inside [0, limit), without overflow.
bool fits(std::uint64_t offset, std::uint64_t length, std::uint64_t limit) {
    return offset <= limit && length <= limit - offset;
}

template <typename T>
T load_at(const std::byte* base, std::uint64_t offset) {
    T value;
    std::memcpy(&value, base + offset, sizeof(T));
    return value;
}

void check_header(const OnDiskHeader& h, std::uint64_t file_bytes, dav2_encoder expected) {
    const bool header_ok = std::memcmp(h.magic, "DAV2MOD\0", 8) == 0 && h.version == 1 && h.endian == 0x01020304u;
    if (!header_ok) fail("invalid DAV2 model header");
    if (h.encoder != static_cast<std::uint32_t>(expected)) fail("model encoder does not match create options");
    if (h.tensor_count == 0 || h.tensor_count > kMaxTensors || h.file_bytes != file_bytes)
        fail("invalid DAV2 model bounds");
    const std::uint64_t table_bytes = std::uint64_t(h.tensor_count) * sizeof(OnDiskTensor);
    const bool table_ok = h.directory_bytes == table_bytes && fits(h.directory_offset, table_bytes, file_bytes) &&
                          h.data_offset % kPayloadAlignment == 0 &&
                          h.data_offset >= h.directory_offset + table_bytes && h.data_offset <= file_bytes;
    if (!table_ok) fail("invalid DAV2 tensor directory");
}

ModelProvenance read_provenance(const std::byte* base, const OnDiskHeader& h) {
    ModelProvenance out;
    if (h.metadata_offset == 0) return out;  // files from before the record existed
    if (h.metadata_offset != h.directory_offset + h.directory_bytes ||
        !fits(h.metadata_offset, sizeof(OnDiskProvenance), h.data_offset))
        fail("invalid DAV2 derivation metadata bounds");
    const auto p = load_at<OnDiskProvenance>(base, h.metadata_offset);
    const bool record_ok = std::memcmp(p.magic, "DAV2META", 8) == 0 && p.version == 1 &&
                           p.bytes == sizeof(OnDiskProvenance) && p.model_format_version == 1 &&
                           p.encoder == h.encoder && (p.flags & ~1u) == 0 &&
                           std::memchr(p.converter, '\0', sizeof(p.converter)) != nullptr;
    if (!record_ok) fail("invalid DAV2 derivation metadata");
    out.recorded = true;
    out.converter = p.converter;
    out.metric = (p.flags & 1u) != 0;
    if (out.metric) {
        if (out.converter != "dav2-export-pytorch-metric-v1") fail("invalid DAV2 metric converter identity");
        std::memcpy(&out.metric_max_depth, &p.reserved, sizeof(float));
        if (out.metric_max_depth != 20.0f && out.metric_max_depth != 80.0f)
            fail("invalid DAV2 metric maximum depth");
    } else {
        if (p.reserved != 0) fail("invalid DAV2 relative derivation metadata");
        if (out.converter != "dav2-export-pytorch-v1") fail("invalid DAV2 relative converter identity");
    }
    return out;
}

WeightRecord read_tensor(const std::byte* base, std::uint64_t record_offset, const OnDiskHeader& h,
                         std::uint64_t file_bytes) {
    const auto t = load_at<OnDiskTensor>(base, record_offset);
    const char* name = reinterpret_cast<const char*>(base + record_offset);  // the record's first field
    const void* nul = std::memchr(name, '\0', sizeof(t.name));
    const bool record_ok = nul != nullptr && name[0] != '\0' && t.dtype == 1 && t.rank >= 1 && t.rank <= 4 &&
                           t.flags == 0 && t.reserved == 0 && t.data_offset >= h.data_offset &&
                           t.data_offset % kPayloadAlignment == 0 && fits(t.data_offset, t.data_bytes, file_bytes);
    if (!record_ok) fail("invalid DAV2 tensor record");
    WeightRecord w;
    w.rank = t.rank;
    w.count = 1;
    for (std::uint32_t d = 0; d < 4; ++d) {
        const std::uint64_t extent = t.dimensions[d];
        if (d >= t.rank) {
            if (extent != 0) fail("invalid DAV2 unused dimension");
            continue;
        }
        if (extent == 0 || w.count > std::numeric_limits<std::uint64_t>::max() / extent)
            fail("invalid DAV2 tensor dimensions");
        w.count *= extent;
        w.shape[d] = extent;
    }
    if (w.count != t.element_count || w.count > std::numeric_limits<std::uint64_t>::max() / 4 ||
        w.count * 4 != t.data_bytes)
        fail("invalid DAV2 tensor byte count");
    w.name = std::string_view(name, static_cast<std::size_t>(static_cast<const char*>(nul) - name));
    w.values = reinterpret_cast<const float*>(base + t.data_offset);
    w.checksum = t.crc32;
    return w;
}

}  // namespace

MappedModel::MappedModel(const std::string& path, dav2_encoder expected_encoder) {
    if (path.empty()) throw std::invalid_argument("model path is empty");
    try {
        fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd_ < 0) fail("failed to open model file");
        struct stat info {};
        if (::fstat(fd_, &info) != 0 || info.st_size < 0) fail("failed to query model file size");
        bytes_ = static_cast<std::uint64_t>(info.st_size);
        if (bytes_ < sizeof(OnDiskHeader)) fail("model file is truncated or too large");
        void* view = ::mmap(nullptr, static_cast<std::size_t>(bytes_), PROT_READ, MAP_PRIVATE, fd_, 0);
        if (view == MAP_FAILED) fail("failed to map model file");
        base_ = static_cast<const std::byte*>(view);

        const auto header = load_at<OnDiskHeader>(base_, 0);
        check_header(header, bytes_, expected_encoder);
        provenance_ = read_provenance(base_, header);
        // Records are checked in file order; a repeated name is reported at
        // the record that repeats it, before any later record is looked at.
        records_.reserve(header.tensor_count);
        std::unordered_set<std::string_view> seen;
        seen.reserve(header.tensor_count);
        for (std::uint32_t i = 0; i < header.tensor_count; ++i) {
            records_.push_back(read_tensor(base_, header.directory_offset + std::uint64_t(i) * sizeof(OnDiskTensor),
                                           header, bytes_));
            if (!seen.insert(records_.back().name).second) fail("duplicate DAV2 tensor name");
        }
        by_name_.resize(records_.size());
        for (std::uint32_t i = 0; i < by_name_.size(); ++i) by_name_[i] = i;
        std::sort(by_name_.begin(), by_name_.end(),
                  [&](std::uint32_t a, std::uint32_t b) { return records_[a].name < records_[b].name; });
    } catch (...) {
        unmap();
        throw;
    }
}

MappedModel::~MappedModel() { unmap(); }

void MappedModel::unmap() noexcept {
    records_.clear();
    by_name_.clear();
    if (base_) ::munmap(const_cast<std::byte*>(base_), static_cast<std::size_t>(bytes_));
    base_ = nullptr;
    if (fd_ >= 0) ::close(fd_);
    fd_ = -1;
    bytes_ = 0;
}

const WeightRecord* MappedModel::find(std::string_view name) const {
    const auto it = std::lower_bound(by_name_.begin(), by_name_.end(), name,
                                     [&](std::uint32_t i, std::string_view key) { return records_[i].name < key; });
    if (it == by_name_.end() || records_[*it].name != name) return nullptr;
    return &records_[*it];
}

const WeightRecord& MappedModel::at(std::string_view name) const {
    const WeightRecord* w = find(name);
    if (!w) throw std::runtime_error("model is missing tensor: " + std::string(name));
    return *w;
}

}  // namespace dav2
