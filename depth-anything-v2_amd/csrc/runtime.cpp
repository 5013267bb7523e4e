#include "runtime.h"

#include <algorithm>
#include <cstring>

#include "dav2_hip.h"

#include <cstdio>
#include <new>
#include <utility>

namespace dav2 {

void hip_check(hipError_t error, const char* what) {
    if (error == hipSuccess) return;
    if (error == hipErrorOutOfMemory || error == hipErrorMemoryAllocation) throw std::bad_alloc();
    throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(error));
}

DeviceBuffer::DeviceBuffer(std::size_t bytes) : bytes_(bytes), owned_(true) {
    if (bytes == 0) return;
    hip_check(hipMalloc(&pointer_, bytes), "hipMalloc");
}

DeviceBuffer::~DeviceBuffer() { reset(); }

DeviceBuffer::DeviceBuffer(DeviceBuffer&& other) noexcept
    : pointer_(std::exchange(other.pointer_, nullptr)),
      bytes_(std::exchange(other.bytes_, 0)),
      owned_(std::exchange(other.owned_, false)) {}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& other) noexcept {
    if (this != &other) {
        reset();
        pointer_ = std::exchange(other.pointer_, nullptr);
        bytes_ = std::exchange(other.bytes_, 0);
        owned_ = std::exchange(other.owned_, false);
    }
    return *this;
}

DeviceBuffer DeviceBuffer::view(void* pointer, std::size_t bytes) {
    DeviceBuffer b;
    b.pointer_ = pointer;
    b.bytes_ = pointer ? bytes : 0;
    b.owned_ = false;
    return b;
}

void DeviceBuffer::reset() {
    if (owned_ && pointer_) (void)hipFree(pointer_);
    pointer_ = nullptr;
    bytes_ = 0;
    owned_ = false;
}

Profiler::~Profiler() {
    for (auto& r : pending_) {
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.stop);
    }
    for (hipEvent_t e : free_) (void)hipEventDestroy(e);
}

hipEvent_t Profiler::take_event() {
    if (!free_.empty()) {
        hipEvent_t e = free_.back();
        free_.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    hip_check(hipEventCreate(&e), "hipEventCreate");
    return e;
}

int Profiler::begin(const char* name, double work, const char* unit, hipStream_t stream, bool dispatch_events) {
    if (!enabled_) return -1;
    Record r{name, unit, work, take_event(), take_event(), dispatch_events, true, {}};
    if (dispatch_events)
        dav2_hip_launch_events(r.start, r.stop);
    else
        hip_check(hipEventRecord(r.start, stream), "hipEventRecord");
    pending_.push_back(r);
    return static_cast<int>(pending_.size() - 1);
}

void Profiler::end(int id, hipStream_t stream) {
    if (id < 0 || static_cast<std::size_t>(id) >= pending_.size()) return;
    if (pending_[id].dispatch)
        // the operation's launches are done; an operation that launched
        // nothing (an empty range) left the events as an earlier one set them
        pending_[id].launched = dav2_hip_launch_events(nullptr, nullptr) != 0;
    else
        (void)hipEventRecord(pending_[id].stop, stream);
}

void Profiler::set_shape(int id, std::uint32_t m, std::uint32_t n, std::uint32_t k, const char* tag) {
    if (id < 0 || static_cast<std::size_t>(id) >= pending_.size()) return;
    char buf[96];
    std::snprintf(buf, sizeof(buf), "%ux%ux%u:%s", m, n, k, tag);
    pending_[id].shape = buf;
}

std::string Profiler::report() {
    hip_check(hipDeviceSynchronize(), "profile synchronize");
    for (auto& r : pending_) {
        float ms = 0.0f;
        // an event pair a launch never recorded (it failed, or the operation
        // launched nothing) has no time
        if (!r.launched || hipEventElapsedTime(&ms, r.start, r.stop) != hipSuccess) {
            (void)hipGetLastError();
            free_.push_back(r.start);
            free_.push_back(r.stop);
            continue;
        }
        Total& t = totals_[r.name];
        t.launches += 1;
        t.ms += ms;
        t.work += r.work;
        t.unit = r.unit;
        if (!r.shape.empty()) {
            Total& ts = totals_[r.name + "@" + r.shape];
            ts.launches += 1;
            ts.ms += ms;
            ts.work += r.work;
            ts.unit = r.unit;
        }
        free_.push_back(r.start);
        free_.push_back(r.stop);
    }
    pending_.clear();
    std::string out = "{";
    bool first = true;
    for (const auto& kv : totals_) {
        char buf[256];
        std::snprintf(buf, sizeof(buf), "%s\"%s\": {\"launches\": %llu, \"ms\": %.6f, \"work\": %.6e, \"unit\": \"%s\"}",
                      first ? "" : ", ", kv.first.c_str(), static_cast<unsigned long long>(kv.second.launches),
                      kv.second.ms, kv.second.work, kv.second.unit.c_str());
        out += buf;
        first = false;
    }
    out += "}";
    totals_.clear();
    return out;
}

HipContext::HipContext(int device_index) : device_(device_index) {
    int count = 0;
    hip_check(hipGetDeviceCount(&count), "hipGetDeviceCount");
    if (device_index < 0 || device_index >= count)
        throw std::runtime_error("HIP device index " + std::to_string(device_index) + " is not available");
    hip_check(hipSetDevice(device_), "hipSetDevice");
    hipDeviceProp_t props{};
    hip_check(hipGetDeviceProperties(&props, device_), "hipGetDeviceProperties");
    device_name_ = props.name;
    compute_units_ = props.multiProcessorCount;
    // Default priority, non-blocking with respect to the null stream.
    hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
    active_ = stream_;
    hip_check(hipEventCreateWithFlags(&in_copied_, hipEventDisableTiming), "staging event");
}

HipContext::~HipContext() {
    (void)hipSetDevice(device_);
    if (stream_) (void)hipStreamSynchronize(stream_);
    if (in_copied_) {
        (void)hipEventSynchronize(in_copied_);
        (void)hipEventDestroy(in_copied_);
    }
    if (in_stage_.data) (void)hipHostFree(in_stage_.data);
    if (out_stage_.data) (void)hipHostFree(out_stage_.data);
    if (stream_) (void)hipStreamDestroy(stream_);
}

void* HipContext::pinned(Pinned& buffer, std::size_t bytes) {
    if (buffer.bytes >= bytes) return buffer.data;
    if (buffer.data) hip_check(hipHostFree(buffer.data), "hipHostFree");
    buffer.data = nullptr;
    buffer.bytes = 0;
    const std::size_t grow = (bytes + (std::size_t(1) << 20) - 1) & ~((std::size_t(1) << 20) - 1);
    hip_check(hipHostMalloc(&buffer.data, grow, hipHostMallocDefault), "hipHostMalloc (staging)");
    buffer.bytes = grow;
    return buffer.data;
}

void* HipContext::input_staging(std::size_t bytes) {
    if (in_pending_) hip_check(hipEventSynchronize(in_copied_), "staging wait");
    in_pending_ = false;
    return pinned(in_stage_, bytes);
}

void HipContext::upload_staged(DeviceBuffer& destination, std::size_t bytes) {
    if (bytes > destination.size() || bytes > in_stage_.bytes) throw std::invalid_argument("staged upload too large");
    if (bytes == 0) return;
    hip_check(hipMemcpyAsync(destination.data(), in_stage_.data, bytes, hipMemcpyHostToDevice, active_), "upload");
    hip_check(hipEventRecord(in_copied_, active_), "staging event");
    in_pending_ = true;
    upload_bytes_ += bytes;
}

void HipContext::upload_staged(DeviceBuffer& destination, const void* source, std::size_t bytes) {
    if (bytes > destination.size()) throw std::invalid_argument("upload exceeds device buffer");
    if (bytes == 0) return;
    // In pieces of about 1 MiB: the DMA of one piece runs while the host
    // copies the next into pinned memory.
    auto* stage = static_cast<std::uint8_t*>(input_staging(bytes));
    const auto* src = static_cast<const std::uint8_t*>(source);
    auto* dst = static_cast<std::uint8_t*>(destination.data());
    const std::size_t pieces = std::min<std::size_t>(8, (bytes + (std::size_t(1) << 20) - 1) >> 20);
    const std::size_t piece = ((bytes + pieces - 1) / pieces + 63) & ~std::size_t(63);
    for (std::size_t off = 0; off < bytes; off += piece) {
        const std::size_t n = std::min(piece, bytes - off);
        std::memcpy(stage + off, src + off, n);
        hip_check(hipMemcpyAsync(dst + off, stage + off, n, hipMemcpyHostToDevice, active_), "upload");
    }
    hip_check(hipEventRecord(in_copied_, active_), "staging event");
    in_pending_ = true;
    upload_bytes_ += bytes;
}

void HipContext::download_staged(const DeviceBuffer& source, void* destination, std::size_t bytes) {
    if (bytes > source.size()) throw std::invalid_argument("download exceeds device buffer");
    if (bytes == 0) return;
    void* stage = pinned(out_stage_, bytes);
    hip_check(hipMemcpyAsync(stage, source.data(), bytes, hipMemcpyDeviceToHost, active_), "download");
    hip_check(hipStreamSynchronize(active_), "download synchronize");
    std::memcpy(destination, stage, bytes);
    download_bytes_ += bytes;
}

void HipContext::make_current() const { hip_check(hipSetDevice(device_), "hipSetDevice"); }

void HipContext::upload(DeviceBuffer& destination, const void* source, std::size_t bytes) {
    if (bytes > destination.size()) throw std::invalid_argument("upload exceeds device buffer");
    if (bytes == 0) return;
    hip_check(hipMemcpyAsync(destination.data(), source, bytes, hipMemcpyHostToDevice, active_), "upload");
    // Asynchronous: the caller keeps the host source alive and unchanged until
    // it synchronises the stream (create and infer both end with a sync).
    upload_bytes_ += bytes;
}

void HipContext::download(const DeviceBuffer& source, void* destination, std::size_t bytes) {
    if (bytes > source.size()) throw std::invalid_argument("download exceeds device buffer");
    if (bytes == 0) return;
    hip_check(hipMemcpyAsync(destination, source.data(), bytes, hipMemcpyDeviceToHost, active_), "download");
    hip_check(hipStreamSynchronize(active_), "download synchronize");
    download_bytes_ += bytes;
}

void HipContext::synchronize() { hip_check(hipStreamSynchronize(active_), "hipStreamSynchronize"); }

}  // namespace dav2
