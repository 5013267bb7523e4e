// The HIP executor behind the C ABI (role of the reference's Executor /
// VulkanExecutor, src/executor.h:87-121, src/vulkan_executor.cpp:534-634).
#pragma once

#include "graph.h"
#include "model.h"

#include <atomic>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

namespace dav2 {

// A submitted GPU inference (dav2_submit_hip): its completion event, the IPC
// mappings and event it holds until release, and the cancel flag.
class HipJob {
public:
    ~HipJob();
    // DAV2_GPU_JOB_* state: RUNNING while the GPU work is in flight, then
    // COMPLETE (or CANCELLED once cancel() has been called).
    dav2_gpu_job_state state() const;
    void cancel() { cancelled_.store(true, std::memory_order_release); }
    void wait() const;

private:
    friend class HipExecutor;
    int device_ = 0;
    hipEvent_t done_ = nullptr;
    void* mapped_input_ = nullptr;
    void* mapped_output_ = nullptr;
    std::atomic<bool> cancelled_{false};
};

class HipExecutor {
public:
    HipExecutor(const std::string& model_path, dav2_encoder encoder, int device_index, std::uint32_t flags);

    void prepare(int image_width, int image_height, int input_size);
    // Host buffers: normalised RGB CHW in, width*height raw depth out.
    void infer(const float* input, int width, int height, float* output);
    // Device buffers, batch images; enqueued on `stream` (nullptr = own stream).
    void infer_device(const float* input, int batch, int width, int height, float* output, hipStream_t stream,
                      float* pre_relu = nullptr);
    void normalize_relative_device(float* depth, std::uint64_t count, hipStream_t stream);
    // Host image paths (src/dav2.cpp:630-665, :754-802), preprocessing and
    // post-processing on the device. bgr8: interleaved BGR rows, inference at
    // network_width x network_height, raw depth resized back to the image
    // (bilinear, align corners) into output [height][width]. bgra8: BGRA rows,
    // nearest resize to network_width x network_height, output min/max
    // normalised at the network size.
    void infer_bgr8(const std::uint8_t* bgr, int width, int height, std::size_t stride, int network_width,
                    int network_height, float* output);
    void infer_bgra8_normalized(const std::uint8_t* bgra, int width, int height, std::size_t stride,
                                int network_width, int network_height, float* output);
    // dav2_submit_hip: enqueue the zero-copy GPU path; the request has been
    // validated by the caller.
    std::unique_ptr<HipJob> submit_hip(const dav2_hip_submit_request& request, int network_width,
                                       int network_height);

private:
    // Uploads `height` rows of `row_bytes` (`stride` bytes apart) into the
    // arena slot `slot` with one copy; returns the device row stride, which
    // is `stride` only if keep_stride allows it.
    std::size_t upload_image(const char* slot, const std::uint8_t* image, std::size_t row_bytes, int height,
                             std::size_t stride, bool keep_stride, DeviceBuffer*& device);

public:

    dav2_encoder encoder() const { return encoder_; }
    float metric_max_depth() const { return model_.provenance().metric_max_depth; }
    void transfer_counters(std::uint64_t& upload, std::uint64_t& download) const {
        upload = context_.upload_bytes();
        download = context_.download_bytes();
    }
    AttentionMode attention_mode() const { return attention_mode_; }
    Precision precision() const { return precision_; }
    HipContext& context() { return context_; }
    std::uint64_t arena_bytes() const { return arena_.bytes(); }

private:
    void run(const float* input, int batch, int width, int height, float* output, float* pre_relu);
    // run() through a HIP graph: the first call with a given (input, output,
    // pre_relu, size, stream) runs eagerly and sizes every buffer, the next
    // one captures the enqueued work (both streams) into a graph, later ones
    // replay it, when DAV2_HIP_GRAPHS=1 is set at creation. Batch > 1 and
    // profiling always run eagerly.
    void run_graph(const float* input, int batch, int width, int height, float* output, float* pre_relu);

public:
    ~HipExecutor();
    HipExecutor(const HipExecutor&) = delete;
    HipExecutor& operator=(const HipExecutor&) = delete;

private:

    dav2_encoder encoder_;
    MappedModel model_;  // validated before any HIP call, as the reference's member order does
    HipContext context_;
    Precision precision_;  // int8, or fp32 / fp16 under FORCE_FP32 / FORCE_FP16
    AttentionMode attention_mode_;
    GpuModel weights_;
    HipOperators operators_;
    // Second operator set with its own workspaces on side_stream_: the DPT
    // levels whose encoder features are ready run there while the encoder
    // continues (batch 1).
    HipOperators side_operators_;
    hipStream_t side_stream_ = nullptr;
    hipEvent_t captured_[4] = {nullptr, nullptr, nullptr, nullptr};
    hipEvent_t side_done_ = nullptr;
    // End of the previous call's work on whichever stream it ran: every call
    // waits for it first, since all calls share the arena buffers.
    hipEvent_t call_done_ = nullptr;
    struct GraphKey {
        const float* input = nullptr;
        float* output = nullptr;
        float* pre_relu = nullptr;
        int width = 0, height = 0;
        hipStream_t stream = nullptr;
        bool operator==(const GraphKey& o) const {
            return input == o.input && output == o.output && pre_relu == o.pre_relu && width == o.width &&
                   height == o.height && stream == o.stream;
        }
    };
    bool graphs_enabled_ = true;
    bool warm_valid_ = false;
    GraphKey warm_key_;   // last eager run (buffers sized for it)
    GraphKey graph_key_;  // what graph_exec_ replays
    hipGraphExec_t graph_exec_ = nullptr;
    DinoEncoder dino_;
    DptHead dpt_;
    Arena arena_;
    std::mutex mutex_;  // one inference at a time per context (docs/architecture.md:254-256)
};

}  // namespace dav2

// Opaque handles of the public ABI.
struct dav2_context {
    std::unique_ptr<dav2::HipExecutor> executor;
};
struct dav2_gpu_job {
    std::unique_ptr<dav2::HipJob> implementation;
    std::uint64_t source_frame_id = 0;
};
