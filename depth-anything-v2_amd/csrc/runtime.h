// HIP device runtime: device buffers, one in-order stream per context,
// transfers with byte counters, and per-launch error checking.
// Role of the reference's src/vulkan.{h,cpp} (buffers, dispatch, batch,
// transfer counters) without any of its Vulkan objects: a single in-order HIP
// stream already orders every kernel after the one before it, so there are
// no barriers or hazard tracking to manage.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

namespace dav2 {

// Throws std::bad_alloc for out-of-memory and std::runtime_error otherwise.
void hip_check(hipError_t error, const char* what);
inline void hip_check(int error, const char* what) { hip_check(static_cast<hipError_t>(error), what); }

class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(std::size_t bytes);
    ~DeviceBuffer();
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& other) noexcept;
    DeviceBuffer& operator=(DeviceBuffer&& other) noexcept;

    // Non-owning view of caller memory (the FFI operator surface uses this).
    static DeviceBuffer view(void* pointer, std::size_t bytes);

    void* data() const { return pointer_; }
    std::size_t size() const { return bytes_; }
    template <typename T>
    T* as() const { return static_cast<T*>(pointer_); }
    explicit operator bool() const { return pointer_ != nullptr; }
    void reset();

private:
    void* pointer_ = nullptr;
    std::size_t bytes_ = 0;
    bool owned_ = false;
};

// Per-launch HIP-event timing, aggregated per kernel family (role of the
// reference's DAV2_VULKAN_PROFILE timestamp queries, src/vulkan.cpp:874-960).
// Off by default; when on, every operator launch is bracketed by two events on
// the stream it runs on, together with its algorithmic work (ops or bytes).
class Profiler {
public:
    ~Profiler();
    void set_enabled(bool on) { enabled_ = on; }
    bool enabled() const { return enabled_; }
    // Returns a record id, or -1 when disabled. With dispatch_events (the
    // default) the events go to the operation's kernel dispatches
    // (dav2_hip_launch_events): the first kernel records the start as it
    // begins, the last one the stop as it ends, so gaps before the first
    // kernel are not counted; otherwise they are recorded on the stream
    // around the enqueued work.
    int begin(const char* name, double work, const char* unit, hipStream_t stream, bool dispatch_events = true);
    void end(int id, hipStream_t stream);
    // Adds a per-shape total "name@MxNxK:tag" for record `id` (GEMMs), beside
    // the family total.
    void set_shape(int id, std::uint32_t m, std::uint32_t n, std::uint32_t k, const char* tag);
    // Synchronises, folds pending records into the totals and returns them as
    // a JSON object {name: {"launches", "ms", "work", "unit"}}; then clears.
    std::string report();

private:
    struct Record {
        std::string name;
        const char* unit;
        double work;
        hipEvent_t start, stop;
        bool dispatch;
        bool launched;  // false: the operation launched no kernel, nothing to time
        std::string shape;
    };
    struct Total {
        std::uint64_t launches = 0;
        double ms = 0.0, work = 0.0;
        std::string unit;
    };
    hipEvent_t take_event();
    bool enabled_ = false;
    std::vector<Record> pending_;
    std::vector<hipEvent_t> free_;
    std::map<std::string, Total> totals_;
};

class ProfileScope {
public:
    ProfileScope(Profiler& p, const char* name, double work, const char* unit, hipStream_t s,
                 bool dispatch_events = true)
        : p_(p), s_(s), id_(p.begin(name, work, unit, s, dispatch_events)) {}
    ~ProfileScope() { p_.end(id_, s_); }
    void shape(std::uint32_t m, std::uint32_t n, std::uint32_t k, const char* tag) {
        if (id_ >= 0) p_.set_shape(id_, m, n, k, tag);
    }

private:
    Profiler& p_;
    hipStream_t s_;
    int id_;
};

class HipContext {
public:
    explicit HipContext(int device_index);
    ~HipContext();
    HipContext(const HipContext&) = delete;
    HipContext& operator=(const HipContext&) = delete;

    int device() const { return device_; }
    hipStream_t stream() const { return stream_; }
    // Runs subsequent work on an external stream (nullptr restores the own one).
    void use_stream(hipStream_t stream) { active_ = stream ? stream : stream_; }
    hipStream_t active_stream() const { return active_; }

    DeviceBuffer create_device_buffer(std::size_t bytes) { return DeviceBuffer(bytes); }
    void upload(DeviceBuffer& destination, const void* source, std::size_t bytes);
    void download(const DeviceBuffer& source, void* destination, std::size_t bytes);
    // Host I/O of the inference entries through pinned buffers owned by the
    // context. A pageable hipMemcpyAsync stages the data itself and returns
    // only when the copy is done; a host copy into pinned memory takes a few
    // microseconds per MB and the DMA from it runs on the stream, so the
    // kernels are enqueued while the input is in flight (ViT-L 518: 3.2 MB
    // up 0.12 -> 0.08 ms, 1.1 MB down 0.08 -> 0.04 ms).
    // input_staging: the pinned input buffer, at least `bytes` long, once the
    // previous staged upload has left it; upload_staged(destination, bytes)
    // then copies its first `bytes` to the device on the active stream.
    void* input_staging(std::size_t bytes);
    void upload_staged(DeviceBuffer& destination, std::size_t bytes);
    void upload_staged(DeviceBuffer& destination, const void* source, std::size_t bytes);
    // Copies to the pinned output buffer on the active stream, synchronises
    // the stream, then copies to `destination`.
    void download_staged(const DeviceBuffer& source, void* destination, std::size_t bytes);
    void synchronize();
    void make_current() const;

    std::uint64_t upload_bytes() const { return upload_bytes_; }
    std::uint64_t download_bytes() const { return download_bytes_; }
    const std::string& device_name() const { return device_name_; }
    int compute_units() const { return compute_units_; }
    Profiler& profiler() { return profiler_; }

private:
    struct Pinned {
        void* data = nullptr;
        std::size_t bytes = 0;
    };
    void* pinned(Pinned& buffer, std::size_t bytes);

    Profiler profiler_;
    int device_ = 0;
    hipStream_t stream_ = nullptr;
    hipStream_t active_ = nullptr;
    Pinned in_stage_, out_stage_;
    hipEvent_t in_copied_ = nullptr;  // recorded after each staged upload
    bool in_pending_ = false;
    std::uint64_t upload_bytes_ = 0;
    std::uint64_t download_bytes_ = 0;
    std::string device_name_;
    int compute_units_ = 0;
};

// RAII switch of the context's active stream.
class ScopedStream {
public:
    ScopedStream(HipContext& context, hipStream_t stream) : context_(context), previous_(context.active_stream()) {
        context_.use_stream(stream);
    }
    ~ScopedStream() { context_.use_stream(previous_); }

private:
    HipContext& context_;
    hipStream_t previous_;
};

}  // namespace dav2
