#include "executor.h"

#include "dav2_hip.h"

#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>

namespace dav2 {

namespace {
// Orders a call's work after the previous call's (which may have been
// enqueued on another stream: the context's own or a caller's) and marks the
// call's end for the next one.
class CallOrder {
public:
    CallOrder(hipEvent_t done, hipStream_t stream) : done_(done), stream_(stream) {
        hip_check(hipStreamWaitEvent(stream_, done_, 0), "order after the previous call");
    }
    ~CallOrder() { (void)hipEventRecord(done_, stream_); }
    CallOrder(const CallOrder&) = delete;
    CallOrder& operator=(const CallOrder&) = delete;

private:
    hipEvent_t done_;
    hipStream_t stream_;
};

AttentionMode attention_mode_for(std::uint32_t flags) {
    // src/encoder.cpp:389-396: int8 and fp16 modes run the reference's
    // binary16 attention unless FORCE_FP32(_ATTENTION) asks for fp32 scores.
    // Here the int8-mode default is the integer-exact fused attention; the
    // reference's binary16 arithmetic is DAV2_CREATE_REFERENCE_FP16_ATTENTION
    // (and the fp16 mode's default).
    if (flags & (DAV2_CREATE_FORCE_FP32 | DAV2_CREATE_FORCE_FP32_ATTENTION)) return AttentionMode::fp32;
    // operators.cpp:1137-1148: devices with cooperative_matrix_fp16 take the
    // scores from bmm_score_coop_fp16.glsl
    if (flags & DAV2_CREATE_REFERENCE_FP16_COOP_ATTENTION) return AttentionMode::binary16_coop;
    if (flags & (DAV2_CREATE_REFERENCE_FP16_ATTENTION | DAV2_CREATE_FORCE_FP16)) return AttentionMode::binary16;
    return AttentionMode::exact;
}

Precision precision_for(std::uint32_t flags) {
    if (flags & DAV2_CREATE_FORCE_FP32) return Precision::fp32;
    if (flags & DAV2_CREATE_FORCE_FP16) return Precision::fp16;
    return Precision::int8;
}
}  // namespace

HipExecutor::HipExecutor(const std::string& model_path, dav2_encoder encoder, int device_index,
                         std::uint32_t flags)
    : encoder_(encoder),
      model_(model_path, encoder),
      context_(device_index),
      precision_(precision_for(flags)),
      attention_mode_(attention_mode_for(flags)),
      weights_(model_, context_, precision_),
      operators_(context_),
      side_operators_(context_),
      dino_(encoder, weights_, operators_, attention_mode_, precision_),
      dpt_(encoder, weights_, operators_, precision_) {
    context_.make_current();
    hip_check(hipStreamCreateWithFlags(&side_stream_, hipStreamNonBlocking), "side stream");
    for (hipEvent_t& e : captured_) hip_check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "capture event");
    hip_check(hipEventCreateWithFlags(&side_done_, hipEventDisableTiming), "side event");
    hip_check(hipEventCreateWithFlags(&call_done_, hipEventDisableTiming), "call event");
    side_operators_.set_stream(side_stream_);
    // Graph replay is opt-in: on MI355X the eager launches of the ViT-L 518
    // inference measured 2-3% faster than replaying its captured graph.
    const char* env = std::getenv("DAV2_HIP_GRAPHS");
    graphs_enabled_ = env && std::string(env) == "1";
    context_.synchronize();
}

HipExecutor::~HipExecutor() {
    context_.make_current();
    if (side_stream_) (void)hipStreamSynchronize(side_stream_);
    (void)hipStreamSynchronize(context_.stream());
    if (graph_exec_) (void)hipGraphExecDestroy(graph_exec_);
    for (hipEvent_t e : captured_)
        if (e) (void)hipEventDestroy(e);
    if (side_done_) (void)hipEventDestroy(side_done_);
    if (call_done_) (void)hipEventDestroy(call_done_);
    if (side_stream_) (void)hipStreamDestroy(side_stream_);
}

void HipExecutor::prepare(int image_width, int image_height, int input_size) {
    (void)image_width;
    (void)image_height;
    (void)input_size;
    // Buffers are sized on the first inference at a resolution; nothing is
    // compiled or autotuned ahead of time.
}

void HipExecutor::run(const float* input, int batch, int width, int height, float* output, float* pre_relu) {
    DeviceBuffer* features[4] = {nullptr, nullptr, nullptr, nullptr};
    const std::uint32_t w = static_cast<std::uint32_t>(width), h = static_cast<std::uint32_t>(height);
    const std::uint32_t pw = w / 14, ph = h / 14;
    const hipStream_t main = operators_.stream();
    if (batch != 1) {
        // The encoder runs the batch at once; then the images' DPT heads
        // alternate between the main and the side stream (own operator set,
        // workspaces and arena slots each), two in flight at a time.
        dino_.forward(input, w, h, static_cast<std::uint32_t>(batch), arena_, features);
        hip_check(hipEventRecord(captured_[0], main), "encoder event");
        hip_check(hipStreamWaitEvent(side_stream_, captured_[0], 0), "side wait");
        for (std::uint32_t b = 0; b < static_cast<std::uint32_t>(batch); ++b) {
            const bool side = (b & 1u) != 0;
            HipOperators& ops = side ? side_operators_ : operators_;
            dpt_.set_slot_suffix(side ? "@side" : "");
            FeatureMap refined[4];
            for (std::uint32_t i = 0; i < 4; ++i) refined[i] = dpt_.prepare_level(i, *features[i], b, pw, ph, arena_, ops);
            dpt_.refine_and_head(refined, b, pw, ph, arena_, output,
                                 b + 1 == static_cast<std::uint32_t>(batch) ? pre_relu : nullptr, &ops);
        }
        dpt_.set_slot_suffix("");
        hip_check(hipEventRecord(side_done_, side_stream_), "side event");
        hip_check(hipStreamWaitEvent(main, side_done_, 0), "main wait");
        return;
    }
    // Levels 0-2 of the DPT head only need their own captured feature: each
    // runs on the side stream as soon as the encoder has produced it, beside
    // the remaining encoder blocks. Level 3 (the last block's feature) runs
    // on the main stream, which then waits for the side stream before the
    // refinenets read all four levels.
    FeatureMap refined[4];
    dino_.forward(input, w, h, 1u, arena_, features, [&](std::uint32_t level) {
        if (level >= 3) return;
        hip_check(hipEventRecord(captured_[level], main), "capture event");
        hip_check(hipStreamWaitEvent(side_stream_, captured_[level], 0), "side wait");
        refined[level] = dpt_.prepare_level(level, *features[level], 0, pw, ph, arena_, side_operators_);
    });
    refined[3] = dpt_.prepare_level(3, *features[3], 0, pw, ph, arena_, operators_);
    hip_check(hipEventRecord(side_done_, side_stream_), "side event");
    hip_check(hipStreamWaitEvent(main, side_done_, 0), "main wait");
    dpt_.refine_and_head(refined, 0, pw, ph, arena_, output, pre_relu);
}

void HipExecutor::run_graph(const float* input, int batch, int width, int height, float* output, float* pre_relu) {
    const hipStream_t main = operators_.stream();
    if (!graphs_enabled_ || batch != 1 || context_.profiler().enabled()) {
        run(input, batch, width, height, output, pre_relu);
        return;
    }
    GraphKey key;
    key.input = input;
    key.output = output;
    key.pre_relu = pre_relu;
    key.width = width;
    key.height = height;
    key.stream = main;
    if (graph_exec_ && key == graph_key_) {
        hip_check(hipGraphLaunch(graph_exec_, main), "graph launch");
        return;
    }
    if (!warm_valid_ || !(key == warm_key_)) {
        // First run at this key: eager, so every arena slot and workspace is
        // allocated (nothing may allocate or synchronise during a capture).
        run(input, batch, width, height, output, pre_relu);
        warm_key_ = key;
        warm_valid_ = true;
        return;
    }
    hipGraph_t graph = nullptr;
    hip_check(hipStreamBeginCapture(main, hipStreamCaptureModeThreadLocal), "begin capture");
    try {
        run(input, batch, width, height, output, pre_relu);
    } catch (...) {
        (void)hipStreamEndCapture(main, &graph);
        if (graph) (void)hipGraphDestroy(graph);
        throw;
    }
    hip_check(hipStreamEndCapture(main, &graph), "end capture");
    hipGraphExec_t exec = nullptr;
    const hipError_t inst = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    hip_check(inst, "graph instantiate");
    if (graph_exec_) {
        hip_check(hipStreamSynchronize(main), "graph replace");
        (void)hipGraphExecDestroy(graph_exec_);
    }
    graph_exec_ = exec;
    graph_key_ = key;
    hip_check(hipGraphLaunch(graph_exec_, main), "graph launch");
}

void HipExecutor::infer(const float* input, int width, int height, float* output) {
    std::lock_guard<std::mutex> lock(mutex_);
    context_.make_current();
    ScopedStream scoped(context_, nullptr);
    CallOrder order(call_done_, context_.active_stream());
    const std::uint64_t in_elems = std::uint64_t(width) * height * 3;
    const std::uint64_t out_elems = std::uint64_t(width) * height;
    DeviceBuffer& in = arena_.get("io.input", in_elems * sizeof(float));
    DeviceBuffer& out = arena_.get("io.output", out_elems * sizeof(float));
    context_.upload_staged(in, input, in_elems * sizeof(float));
    run_graph(in.as<float>(), 1, width, height, out.as<float>(), nullptr);
    context_.download_staged(out, output, out_elems * sizeof(float));
}

void HipExecutor::infer_device(const float* input, int batch, int width, int height, float* output,
                               hipStream_t stream, float* pre_relu) {
    std::lock_guard<std::mutex> lock(mutex_);
    context_.make_current();
    ScopedStream scoped(context_, stream);
    CallOrder order(call_done_, context_.active_stream());
    run_graph(input, batch, width, height, output, pre_relu);
}

void HipExecutor::normalize_relative_device(float* depth, std::uint64_t count, hipStream_t stream) {
    std::lock_guard<std::mutex> lock(mutex_);
    context_.make_current();
    ScopedStream scoped(context_, stream);
    CallOrder order(call_done_, context_.active_stream());
    if (count == 0 || count > 0xffffffffull) throw std::invalid_argument("invalid relative depth count");
    DeviceBuffer d = DeviceBuffer::view(depth, count * sizeof(float));
    DeviceBuffer& range = arena_.get("io.range", 2 * sizeof(float));
    operators_.reduce_minmax(d, range, static_cast<std::uint32_t>(count));
    operators_.normalize_relative(d, range, static_cast<std::uint32_t>(count));
}

std::size_t HipExecutor::upload_image(const char* slot, const std::uint8_t* image, std::size_t row_bytes,
                                      int height, std::size_t stride, bool keep_stride, DeviceBuffer*& device) {
    // One host-to-device copy either way (a pitched copy from pageable memory
    // goes row by row), through the context's pinned input buffer: the rows
    // with their padding when it is small, else the rows packed.
    const std::size_t rows = static_cast<std::size_t>(height);
    const std::size_t span = (rows - 1) * stride + row_bytes, packed = rows * row_bytes;
    if (keep_stride && span <= packed + packed / 4) {
        device = &arena_.get(slot, span);
        context_.upload_staged(*device, image, span);
        return stride;
    }
    auto* stage = static_cast<std::uint8_t*>(context_.input_staging(packed));
    for (std::size_t r = 0; r < rows; ++r) std::memcpy(stage + r * row_bytes, image + r * stride, row_bytes);
    device = &arena_.get(slot, packed);
    context_.upload_staged(*device, packed);
    return row_bytes;
}

HipJob::~HipJob() {
    // the job's device current for the calls below, the caller's afterwards
    int previous = -1;
    (void)hipGetDevice(&previous);
    (void)hipSetDevice(device_);
    if (done_) {
        (void)hipEventSynchronize(done_);
        (void)hipEventDestroy(done_);
    }
    if (mapped_input_) (void)hipIpcCloseMemHandle(mapped_input_);
    if (mapped_output_) (void)hipIpcCloseMemHandle(mapped_output_);
    if (previous >= 0) (void)hipSetDevice(previous);
}

dav2_gpu_job_state HipJob::state() const {
    // vulkan_executor.cpp:450-457: CANCELLED, else COMPLETE once the
    // submission has finished, else RUNNING.
    if (cancelled_.load(std::memory_order_acquire)) return DAV2_GPU_JOB_CANCELLED;
    const hipError_t e = hipEventQuery(done_);
    if (e == hipSuccess) return DAV2_GPU_JOB_COMPLETE;
    if (e == hipErrorNotReady) return DAV2_GPU_JOB_RUNNING;
    return DAV2_GPU_JOB_FAILED;
}

void HipJob::wait() const { hip_check(hipEventSynchronize(done_), "GPU job wait"); }

std::unique_ptr<HipJob> HipExecutor::submit_hip(const dav2_hip_submit_request& r, int network_width,
                                                int network_height) {
    std::lock_guard<std::mutex> lock(mutex_);
    context_.make_current();
    ScopedStream scoped(context_, nullptr);
    CallOrder order(call_done_, context_.active_stream());
    const hipStream_t main = context_.active_stream();
    auto job = std::make_unique<HipJob>();
    job->device_ = context_.device();
    hip_check(hipEventCreateWithFlags(&job->done_, hipEventDisableTiming), "job event");
    // Buffers: this process's pointers, or the other process's allocations
    // mapped through their IPC handles (held by the job until release).
    const std::uint8_t* input = static_cast<const std::uint8_t*>(r.input);
    if (!input) {
        hipIpcMemHandle_t h;
        std::memcpy(&h, r.input_ipc, sizeof(h));
        hip_check(hipIpcOpenMemHandle(&job->mapped_input_, h, hipIpcMemLazyEnablePeerAccess), "open input IPC handle");
        input = static_cast<const std::uint8_t*>(job->mapped_input_) + r.input_offset;
    }
    float* output = r.output;
    if (!output) {
        hipIpcMemHandle_t h;
        std::memcpy(&h, r.output_ipc, sizeof(h));
        hip_check(hipIpcOpenMemHandle(&job->mapped_output_, h, hipIpcMemLazyEnablePeerAccess),
                  "open output IPC handle");
        output = reinterpret_cast<float*>(static_cast<std::uint8_t*>(job->mapped_output_) + r.output_offset);
    }
    if (r.wait_event) {
        hip_check(hipStreamWaitEvent(main, static_cast<hipEvent_t>(r.wait_event), 0), "wait for the producer");
    }
    // vulkan_executor.cpp:694-787: GPU preprocessing, inference, min/max
    // normalisation at the network size, bilinear resize into the output
    const std::uint64_t net = std::uint64_t(network_width) * network_height;
    const std::uint64_t pixels = std::uint64_t(r.width) * r.height;
    DeviceBuffer& in = arena_.get("io.input", net * 3 * sizeof(float));
    DeviceBuffer& depth = arena_.get("io.output", net * sizeof(float));
    DeviceBuffer& range = arena_.get("io.range", 2 * sizeof(float));
    hip_check(dav2_hip_preprocess_rgba8(reinterpret_cast<const std::uint32_t*>(input), r.width, r.height,
                                        r.row_stride_bytes, static_cast<std::uint32_t>(network_width),
                                        static_cast<std::uint32_t>(network_height),
                                        r.pixel_format == DAV2_GPU_PIXEL_RGBA8 ? 1u : 0u, in.as<float>(), main),
              "preprocess_rgba8");
    run_graph(in.as<float>(), 1, network_width, network_height, depth.as<float>(), nullptr);
    operators_.reduce_minmax(depth, range, static_cast<std::uint32_t>(net));
    operators_.normalize_relative(depth, range, static_cast<std::uint32_t>(net));
    DeviceBuffer out = DeviceBuffer::view(output, pixels * sizeof(float));
    operators_.bilinear_align_true(out, depth, static_cast<std::uint32_t>(network_width),
                                   static_cast<std::uint32_t>(network_height), r.width, r.height, 1);
    hip_check(hipEventRecord(job->done_, main), "job event");
    return job;
}

void HipExecutor::infer_bgr8(const std::uint8_t* bgr, int width, int height, std::size_t stride, int network_width,
                             int network_height, float* output) {
    std::lock_guard<std::mutex> lock(mutex_);
    context_.make_current();
    ScopedStream scoped(context_, nullptr);
    CallOrder order(call_done_, context_.active_stream());
    const std::uint64_t row_bytes = std::uint64_t(width) * 3;
    const std::uint64_t net = std::uint64_t(network_width) * network_height;
    const std::uint64_t pixels = std::uint64_t(width) * height;
    DeviceBuffer* image = nullptr;
    const std::size_t device_stride = upload_image("io.bgr8", bgr, row_bytes, height, stride, true, image);
    DeviceBuffer& in = arena_.get("io.input", net * 3 * sizeof(float));
    DeviceBuffer& depth = arena_.get("io.output", net * sizeof(float));
    hip_check(dav2_hip_preprocess_bgr8(image->as<std::uint8_t>(), static_cast<std::uint32_t>(width),
                                       static_cast<std::uint32_t>(height), device_stride,
                                       static_cast<std::uint32_t>(network_width),
                                       static_cast<std::uint32_t>(network_height), in.as<float>(),
                                       context_.active_stream()),
              "preprocess_bgr8");
    run_graph(in.as<float>(), 1, network_width, network_height, depth.as<float>(), nullptr);
    if (network_width == width && network_height == height) {
        context_.download_staged(depth, output, pixels * sizeof(float));
        return;
    }
    // vulkan_executor.cpp:586-598: bilinear (align corners) back to the image
    DeviceBuffer& resized = arena_.get("io.resized", pixels * sizeof(float));
    operators_.bilinear_align_true(resized, depth, static_cast<std::uint32_t>(network_width),
                                   static_cast<std::uint32_t>(network_height), static_cast<std::uint32_t>(width),
                                   static_cast<std::uint32_t>(height), 1);
    context_.download_staged(resized, output, pixels * sizeof(float));
}

void HipExecutor::infer_bgra8_normalized(const std::uint8_t* bgra, int width, int height, std::size_t stride,
                                         int network_width, int network_height, float* output) {
    std::lock_guard<std::mutex> lock(mutex_);
    context_.make_current();
    ScopedStream scoped(context_, nullptr);
    CallOrder order(call_done_, context_.active_stream());
    const std::uint64_t row_bytes = std::uint64_t(width) * 4;
    const std::uint64_t net = std::uint64_t(network_width) * network_height;
    if (net > 0xffffffffull) throw std::invalid_argument("network size too large");
    // the kernel reads whole pixels: a stride that is not a multiple of 4 is packed
    DeviceBuffer* image = nullptr;
    const std::size_t device_stride = upload_image("io.bgra8", bgra, row_bytes, height, stride, stride % 4 == 0, image);
    DeviceBuffer& in = arena_.get("io.input", net * 3 * sizeof(float));
    DeviceBuffer& depth = arena_.get("io.output", net * sizeof(float));
    DeviceBuffer& normalized = arena_.get("io.normalized", net * sizeof(float));
    DeviceBuffer& range = arena_.get("io.range", 2 * sizeof(float));
    hip_check(dav2_hip_preprocess_bgra8_nearest(image->as<std::uint8_t>(), static_cast<std::uint32_t>(width),
                                                static_cast<std::uint32_t>(height), device_stride,
                                                static_cast<std::uint32_t>(network_width),
                                                static_cast<std::uint32_t>(network_height), in.as<float>(),
                                                context_.active_stream()),
              "preprocess_bgra8_nearest");
    run_graph(in.as<float>(), 1, network_width, network_height, depth.as<float>(), nullptr);
    operators_.reduce_minmax(depth, range, static_cast<std::uint32_t>(net));
    hip_check(dav2_hip_normalize_span(depth.as<float>(), range.as<float>(), net, normalized.as<float>(),
                                      context_.active_stream()),
              "normalize_span");
    context_.download_staged(normalized, output, net * sizeof(float));
}

}  // namespace dav2
