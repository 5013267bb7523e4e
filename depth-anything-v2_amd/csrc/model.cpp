#include "model.h"

#include <cstring>
#include <limits>
#include <stdexcept>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace dav2 {
namespace {

// On-disk layout (little-endian, packed). Field order and sizes are fixed by
// the format: src/model.cpp:27-69, tools/export_model.py:25-38.
#pragma pack(push, 1)
struct FileHeader {
    char magic[8];  // "DAV2MOD\0"
    std::uint32_t version;
    std::uint32_t endian;
    std::uint32_t encoder;
    std::uint32_t tensor_count;
    std::uint64_t directory_offset;
    std::uint64_t directory_bytes;
    std::uint64_t data_offset;
    std::uint64_t file_bytes;
    std::uint64_t metadata_offset;  // 0 = no derivation record
};
struct TensorRecord {
    char name[112];
    std::uint32_t dtype;  // 1 = float32
    std::uint32_t rank;
    std::uint64_t dimensions[4];
    std::uint64_t data_offset;
    std::uint64_t data_bytes;
    std::uint64_t element_count;
    std::uint32_t crc32;
    std::uint32_t flags;
    std::uint64_t reserved;
};
struct DerivationRecord {
    char magic[8];  // "DAV2META"
    std::uint32_t version;
    std::uint32_t bytes;
    std::uint32_t model_format_version;
    std::uint32_t encoder;
    std::uint32_t flags;     // bit 0: metric model
    std::uint32_t reserved;  // metric: float max depth bits
    std::uint8_t canonical_sha256[32];
    char converter[64];
};
#pragma pack(pop)
static_assert(sizeof(FileHeader) == 64, "header is 64 bytes");
static_assert(sizeof(TensorRecord) == 192, "record is 192 bytes");
static_assert(sizeof(DerivationRecord) == 128, "derivation record is 128 bytes");

constexpr std::uint64_t kAlignment = 64;

bool in_range(std::uint64_t offset, std::uint64_t bytes, std::uint64_t limit) {
    return offset <= limit && bytes <= limit - offset;
}

[[noreturn]] void reject(const char* why) { throw std::runtime_error(why); }

}  // namespace

std::uint32_t crc32(const void* data, std::size_t bytes) {
    if (bytes != 0 && data == nullptr) throw std::invalid_argument("CRC32 input is null");
    static const auto table = [] {
        std::array<std::uint32_t, 256> t{};
        for (std::uint32_t i = 0; i < 256; ++i) {
            std::uint32_t c = i;
            for (int k = 0; k < 8; ++k) c = (c >> 1) ^ ((c & 1u) ? 0xedb88320u : 0u);
            t[i] = c;
        }
        return t;
    }();
    const auto* p = static_cast<const unsigned char*>(data);
    std::uint32_t c = 0xffffffffu;
    for (std::size_t i = 0; i < bytes; ++i) c = table[(c ^ p[i]) & 0xffu] ^ (c >> 8);
    return ~c;
}

ModelFile::ModelFile(const std::string& path, dav2_encoder expected_encoder) {
    try {
        if (path.empty()) throw std::invalid_argument("model path is empty");
        fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd_ < 0) reject("failed to open model file");
        struct stat st {};
        if (::fstat(fd_, &st) != 0 || st.st_size < 0) reject("failed to query model file size");
        size_ = static_cast<std::uint64_t>(st.st_size);
        if (size_ < sizeof(FileHeader)) reject("model file is truncated or too large");
        void* mapped = ::mmap(nullptr, static_cast<std::size_t>(size_), PROT_READ, MAP_PRIVATE, fd_, 0);
        if (mapped == MAP_FAILED) reject("failed to map model file");
        view_ = static_cast<const std::byte*>(mapped);

        FileHeader header;
        std::memcpy(&header, view_, sizeof(header));
        if (std::memcmp(header.magic, "DAV2MOD\0", 8) != 0 || header.version != 1 ||
            header.endian != 0x01020304u)
            reject("invalid DAV2 model header");
        if (header.encoder != static_cast<std::uint32_t>(expected_encoder))
            reject("model encoder does not match create options");
        if (header.tensor_count == 0 || header.tensor_count > 2048 || header.file_bytes != size_)
            reject("invalid DAV2 model bounds");
        const std::uint64_t directory_bytes = static_cast<std::uint64_t>(header.tensor_count) * sizeof(TensorRecord);
        if (header.directory_bytes != directory_bytes ||
            !in_range(header.directory_offset, header.directory_bytes, size_) ||
            header.data_offset % kAlignment != 0 ||
            header.data_offset < header.directory_offset + header.directory_bytes || header.data_offset > size_)
            reject("invalid DAV2 tensor directory");

        if (header.metadata_offset != 0) {
            if (header.metadata_offset != header.directory_offset + header.directory_bytes ||
                !in_range(header.metadata_offset, sizeof(DerivationRecord), header.data_offset))
                reject("invalid DAV2 derivation metadata bounds");
            DerivationRecord meta;
            std::memcpy(&meta, view_ + header.metadata_offset, sizeof(meta));
            if (std::memcmp(meta.magic, "DAV2META", 8) != 0 || meta.version != 1 ||
                meta.bytes != sizeof(DerivationRecord) || meta.model_format_version != 1 ||
                meta.encoder != header.encoder || (meta.flags & ~1u) != 0 ||
                std::memchr(meta.converter, '\0', sizeof(meta.converter)) == nullptr)
                reject("invalid DAV2 derivation metadata");
            derivation_.present = true;
            std::memcpy(derivation_.canonical_sha256.data(), meta.canonical_sha256, 32);
            derivation_.converter = meta.converter;
            derivation_.format_version = meta.model_format_version;
            derivation_.encoder = static_cast<dav2_encoder>(meta.encoder);
            if (meta.flags & 1u) {
                if (derivation_.converter != "dav2-export-pytorch-metric-v1")
                    reject("invalid DAV2 metric converter identity");
                float max_depth = 0.0f;
                std::memcpy(&max_depth, &meta.reserved, sizeof(max_depth));
                if (max_depth != 20.0f && max_depth != 80.0f) reject("invalid DAV2 metric maximum depth");
                derivation_.metric_max_depth = max_depth;
            } else if (meta.reserved != 0) {
                reject("invalid DAV2 relative derivation metadata");
            } else if (derivation_.converter != "dav2-export-pytorch-v1") {
                reject("invalid DAV2 relative converter identity");
            }
        }

        tensors_.reserve(header.tensor_count);
        names_.reserve(header.tensor_count);
        for (std::uint32_t i = 0; i < header.tensor_count; ++i) {
            const auto* record_bytes = view_ + header.directory_offset + static_cast<std::uint64_t>(i) * sizeof(TensorRecord);
            TensorRecord record;
            std::memcpy(&record, record_bytes, sizeof(record));
            const auto* name_bytes = reinterpret_cast<const char*>(record_bytes);  // name is the first field
            const void* terminator = std::memchr(name_bytes, '\0', sizeof(record.name));
            if (!terminator || name_bytes[0] == '\0' || record.dtype != 1 || record.rank == 0 || record.rank > 4 ||
                record.flags != 0 || record.reserved != 0 || record.data_offset < header.data_offset ||
                record.data_offset % kAlignment != 0 || !in_range(record.data_offset, record.data_bytes, size_))
                reject("invalid DAV2 tensor record");
            std::uint64_t elements = 1;
            for (std::uint32_t d = 0; d < 4; ++d) {
                const std::uint64_t v = record.dimensions[d];
                if (d < record.rank) {
                    if (v == 0 || elements > std::numeric_limits<std::uint64_t>::max() / v)
                        reject("invalid DAV2 tensor dimensions");
                    elements *= v;
                } else if (v != 0) {
                    reject("invalid DAV2 unused dimension");
                }
            }
            if (elements != record.element_count || elements > std::numeric_limits<std::uint64_t>::max() / 4 ||
                elements * 4 != record.data_bytes)
                reject("invalid DAV2 tensor byte count");
            const std::string_view name(name_bytes,
                                        static_cast<std::size_t>(static_cast<const char*>(terminator) - name_bytes));
            TensorView t;
            t.data = reinterpret_cast<const float*>(view_ + record.data_offset);
            for (int d = 0; d < 4; ++d) t.dimensions[d] = record.dimensions[d];
            t.rank = record.rank;
            t.elements = record.element_count;
            t.crc32 = record.crc32;
            if (!tensors_.emplace(name, t).second) reject("duplicate DAV2 tensor name");
            names_.push_back(name);
        }
    } catch (...) {
        close();
        throw;
    }
}

ModelFile::~ModelFile() { close(); }

void ModelFile::close() noexcept {
    tensors_.clear();
    names_.clear();
    if (view_) {
        ::munmap(const_cast<std::byte*>(view_), static_cast<std::size_t>(size_));
        view_ = nullptr;
    }
    if (fd_ >= 0) {
        ::close(fd_);
        fd_ = -1;
    }
    size_ = 0;
}

const TensorView& ModelFile::tensor(std::string_view name) const {
    const auto it = tensors_.find(name);
    if (it == tensors_.end()) throw std::runtime_error("model is missing tensor: " + std::string(name));
    return it->second;
}

bool ModelFile::contains(std::string_view name) const { return tensors_.count(name) != 0; }

}  // namespace dav2
