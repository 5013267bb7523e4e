// Public C ABI (include/depth_anything_v2.h). Argument checks, their order,
// messages and the exception -> status mapping follow src/dav2.cpp of the
// reference (protect() :71-90, create :158-213, infer :603-628).

#include "depth_anything_v2.h"

#include "executor.h"

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstddef>
#include <cstring>
#include <memory>
#include <new>
#include <stdexcept>
#include <string>

namespace {

thread_local std::string last_error;

class ApiError final : public std::runtime_error {
public:
    ApiError(dav2_status status, const char* message) : std::runtime_error(message), status_(status) {}
    dav2_status status() const { return status_; }

private:
    dav2_status status_;
};

dav2_status fail(dav2_status status, const char* message) {
    last_error = message ? message : "";
    return status;
}

template <typename Function>
dav2_status protect(Function&& function) {
    try {
        function();
        last_error.clear();
        return DAV2_STATUS_OK;
    } catch (const ApiError& e) {
        return fail(e.status(), e.what());
    } catch (const std::bad_alloc&) {
        return fail(DAV2_STATUS_OUT_OF_MEMORY, "out of memory");
    } catch (const std::invalid_argument& e) {
        return fail(DAV2_STATUS_INVALID_ARGUMENT, e.what());
    } catch (const std::exception& e) {
        return fail(DAV2_STATUS_INTERNAL_ERROR, e.what());
    } catch (...) {
        return fail(DAV2_STATUS_INTERNAL_ERROR, "unknown internal error");
    }
}

bool supported_encoder(dav2_encoder e) {
    return e == DAV2_ENCODER_VITS || e == DAV2_ENCODER_VITB || e == DAV2_ENCODER_VITL;
}

// src/image.cpp:15-19, :138-161 (numpy.round ties-to-even == nearbyint).
int round_to_multiple(double value, int multiple) {
    return static_cast<int>(std::nearbyint(value / multiple)) * multiple;
}

dav2_image_shape network_shape(int width, int height, int input_size) {
    if (width <= 0 || height <= 0 || input_size <= 0)
        throw std::invalid_argument("image dimensions and input_size must be positive");
    constexpr int patch = 14;
    const double scale = std::max(static_cast<double>(input_size) / height, static_cast<double>(input_size) / width);
    int oh = std::max(round_to_multiple(scale * height, patch), input_size);
    int ow = std::max(round_to_multiple(scale * width, patch), input_size);
    if (oh % patch != 0) oh = ((oh + patch - 1) / patch) * patch;
    if (ow % patch != 0) ow = ((ow + patch - 1) / patch) * patch;
    return {ow, oh};
}

}  // namespace

extern "C" {

uint32_t DAV2_CALL dav2_abi_version(void) { return DAV2_ABI_VERSION; }

const char* DAV2_CALL dav2_version_string(void) { return "0.1.0-mi355x"; }

const char* DAV2_CALL dav2_status_string(dav2_status status) {
    switch (status) {
        case DAV2_STATUS_OK: return "ok";
        case DAV2_STATUS_INVALID_ARGUMENT: return "invalid argument";
        case DAV2_STATUS_MODEL_IO: return "model I/O error";
        case DAV2_STATUS_MODEL_FORMAT: return "invalid model format";
        case DAV2_STATUS_VULKAN_UNAVAILABLE: return "Vulkan unavailable";
        case DAV2_STATUS_OUT_OF_MEMORY: return "out of memory";
        case DAV2_STATUS_INFERENCE_FAILED: return "inference failed";
        case DAV2_STATUS_BUFFER_TOO_SMALL: return "buffer too small";
        case DAV2_STATUS_UNSUPPORTED: return "unsupported";
        case DAV2_STATUS_INTERNAL_ERROR: return "internal error";
        case DAV2_STATUS_INVALID_STATE: return "invalid state";
        case DAV2_STATUS_CANCELLED: return "cancelled";
    }
    return "unknown status";
}

const char* DAV2_CALL dav2_last_error(void) { return last_error.c_str(); }

dav2_status DAV2_CALL dav2_get_network_shape(int32_t image_width, int32_t image_height, int32_t input_size,
                                             dav2_image_shape* shape) {
    if (shape == nullptr) return fail(DAV2_STATUS_INVALID_ARGUMENT, "network_shape is null");
    return protect([&] { *shape = network_shape(image_width, image_height, input_size); });
}

dav2_status DAV2_CALL dav2_get_inferbridge_shape(int32_t image_width, int32_t image_height, int32_t input_size,
                                                 dav2_image_shape* shape) {
    if (shape == nullptr) return fail(DAV2_STATUS_INVALID_ARGUMENT, "output_shape is null");
    return protect([&] {
        const dav2_image_shape s = network_shape(image_width, image_height, input_size);
        shape->width = s.height;
        shape->height = s.width;
    });
}

dav2_status DAV2_CALL dav2_create(const char* model_path_utf8, const dav2_create_options* options,
                                  dav2_context** context) {
    if (context == nullptr) return fail(DAV2_STATUS_INVALID_ARGUMENT, "context is null");
    *context = nullptr;
    if (model_path_utf8 == nullptr || model_path_utf8[0] == '\0')
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "model_path_utf8 is empty");
    constexpr size_t legacy_size = offsetof(dav2_create_options, cache_path_utf8);
    if (options == nullptr || options->struct_size < legacy_size)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "invalid create options");
    if (options->abi_version != DAV2_ABI_VERSION) return fail(DAV2_STATUS_INVALID_ARGUMENT, "ABI version mismatch");
    if (!supported_encoder(options->encoder)) return fail(DAV2_STATUS_INVALID_ARGUMENT, "unsupported encoder");
    constexpr uint32_t supported = DAV2_CREATE_FORCE_FP32 | DAV2_CREATE_FORCE_FP32_WEIGHTS |
                                   DAV2_CREATE_FORCE_FP32_ATTENTION | DAV2_CREATE_FORCE_FP16 |
                                   DAV2_CREATE_FORCE_INT8 | DAV2_CREATE_FORCE_METAL | DAV2_CREATE_FORCE_VULKAN |
                                   DAV2_CREATE_REFERENCE_FP16_ATTENTION | DAV2_CREATE_REFERENCE_FP16_COOP_ATTENTION;
    if ((options->flags & ~supported) != 0) return fail(DAV2_STATUS_INVALID_ARGUMENT, "unsupported create flags");
    if ((options->flags & (DAV2_CREATE_REFERENCE_FP16_ATTENTION | DAV2_CREATE_REFERENCE_FP16_COOP_ATTENTION)) &&
        (options->flags & (DAV2_CREATE_FORCE_FP32 | DAV2_CREATE_FORCE_FP32_ATTENTION)))
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "binary16 attention needs the int8 execution precision");
    const uint32_t precision = options->flags & (DAV2_CREATE_FORCE_FP32 | DAV2_CREATE_FORCE_FP16 | DAV2_CREATE_FORCE_INT8);
    if (precision != 0 && (precision & (precision - 1u)) != 0)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "multiple DAV2 execution precisions were requested");
    if (options->vulkan_device_index < 0) return fail(DAV2_STATUS_INVALID_ARGUMENT, "invalid device index");
    // This build executes the int8 operator path (the default) and the fp32
    // and fp16 precision modes (FORCE_FP32, FORCE_FP16). FORCE_FP32_WEIGHTS is
    // accepted and has no further effect, as in the reference (dav2.cpp:182
    // is its only use).
    if (options->flags & DAV2_CREATE_FORCE_METAL)
        return fail(DAV2_STATUS_UNSUPPORTED, "the Metal executor is not available on this platform");
    return protect([&] {
        auto result = std::make_unique<dav2_context>();
        result->executor = std::make_unique<dav2::HipExecutor>(model_path_utf8, options->encoder,
                                                               options->vulkan_device_index, options->flags);
        if (result->executor->metric_max_depth() > 0.0f)
            throw ApiError(DAV2_STATUS_UNSUPPORTED, "metric-depth heads are not part of this build");
        *context = result.release();
    });
}

dav2_status DAV2_CALL dav2_prepare(dav2_context* context, int32_t image_width, int32_t image_height,
                                   int32_t input_size) {
    if (context == nullptr || image_width <= 0 || image_height <= 0 || input_size <= 0)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "invalid prepare request");
    return protect([&] { context->executor->prepare(image_width, image_height, input_size); });
}

void DAV2_CALL dav2_destroy(dav2_context* context) { delete context; }

dav2_status DAV2_CALL dav2_get_model_info(const dav2_context* context, dav2_model_info* info) {
    if (context == nullptr || info == nullptr || info->struct_size < sizeof(*info))
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "invalid model info query");
    return protect([&] {
        const float max_depth = context->executor->metric_max_depth();
        *info = {};
        info->struct_size = sizeof(*info);
        info->abi_version = DAV2_ABI_VERSION;
        info->encoder = context->executor->encoder();
        info->is_metric = max_depth > 0.0f ? 1u : 0u;
        info->metric_max_depth = max_depth;
    });
}

dav2_status DAV2_CALL dav2_probe_gpu_capabilities(int32_t device_index, dav2_gpu_capabilities* caps) {
    if (caps == nullptr) return fail(DAV2_STATUS_INVALID_ARGUMENT, "GPU capabilities are null");
    if (caps->struct_size < sizeof(*caps) || device_index < 0)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "invalid GPU capability probe");
    // No D3D12/Metal interop on this platform: no capability flags
    // (src/vulkan_executor.cpp:1057-1065 on Linux).
    *caps = {};
    caps->struct_size = sizeof(*caps);
    caps->abi_version = DAV2_ABI_VERSION;
    last_error.clear();
    return DAV2_STATUS_OK;
}

dav2_status DAV2_CALL dav2_get_gpu_capabilities(const dav2_context* context, dav2_gpu_capabilities* caps) {
    if (context == nullptr || caps == nullptr) return fail(DAV2_STATUS_INVALID_ARGUMENT, "null GPU capability argument");
    if (caps->struct_size < sizeof(*caps))
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "GPU capabilities struct is too small");
    *caps = {};
    caps->struct_size = sizeof(*caps);
    caps->abi_version = DAV2_ABI_VERSION;
    last_error.clear();
    return DAV2_STATUS_OK;
}

dav2_status DAV2_CALL dav2_get_transfer_counters(const dav2_context* context, dav2_transfer_counters* counters) {
    if (context == nullptr || counters == nullptr)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "null transfer counter argument");
    if (counters->struct_size < sizeof(*counters))
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "transfer counters struct is too small");
    return protect([&] {
        std::uint64_t up = 0, down = 0;
        context->executor->transfer_counters(up, down);
        *counters = {};
        counters->struct_size = sizeof(*counters);
        counters->tensor_upload_bytes = up;
        counters->tensor_download_bytes = down;
    });
}

// ---- D3D12 / Metal interop: not available (src/dav2.cpp:329-601) ----------
dav2_status DAV2_CALL dav2_submit_d3d12(dav2_context* context, const dav2_d3d12_submit_request* request,
                                       dav2_gpu_job** job) {
    if (context == nullptr || request == nullptr || job == nullptr)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "null D3D12 submit argument");
    *job = nullptr;
    if (request->struct_size < sizeof(*request) || request->abi_version != DAV2_ABI_VERSION)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "invalid D3D12 submit request");
    return fail(DAV2_STATUS_UNSUPPORTED, "complete D3D12/Vulkan GPU interop is unavailable");
}

dav2_status DAV2_CALL dav2_submit_d3d12_texture(dav2_context* context,
                                               const dav2_d3d12_texture_submit_request* request,
                                               dav2_gpu_job** job) {
    if (context == nullptr || request == nullptr || job == nullptr)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "null D3D12 texture submit argument");
    *job = nullptr;
    if (request->struct_size < sizeof(*request) || request->abi_version != DAV2_ABI_VERSION)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "invalid D3D12 texture submit request");
    return fail(DAV2_STATUS_UNSUPPORTED, "complete D3D12/Vulkan texture interop is unavailable");
}

dav2_status DAV2_CALL dav2_submit_d3d12_texture_binding(dav2_context* context,
                                                       const dav2_d3d12_texture_binding_request* request,
                                                       dav2_gpu_job** job) {
    if (!context || !request || !job) return fail(DAV2_STATUS_INVALID_ARGUMENT, "null D3D12 texture binding argument");
    *job = nullptr;
    if (request->struct_size < offsetof(dav2_d3d12_texture_binding_request, input_texture_identity) ||
        request->abi_version != DAV2_ABI_VERSION)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "invalid D3D12 texture binding request");
    return fail(DAV2_STATUS_UNSUPPORTED, "D3D12 texture bindings are only available on Windows");
}

dav2_status DAV2_CALL dav2_submit_metal_texture_binding(dav2_context* context,
                                                       const dav2_metal_texture_binding_request* request,
                                                       dav2_gpu_job** job) {
    if (!context || !request || !job) return fail(DAV2_STATUS_INVALID_ARGUMENT, "null Metal texture binding argument");
    *job = nullptr;
    if (request->struct_size < sizeof(*request) || request->abi_version != DAV2_ABI_VERSION)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "invalid Metal texture binding request");
    return fail(DAV2_STATUS_UNSUPPORTED, "Metal texture bindings are only available on Apple platforms");
}

// GPU jobs come from dav2_submit_hip (src/dav2.cpp:429-473 semantics).
dav2_status DAV2_CALL dav2_gpu_job_poll(const dav2_gpu_job* job, dav2_gpu_job_status* status) {
    if (job == nullptr || status == nullptr) return fail(DAV2_STATUS_INVALID_ARGUMENT, "null GPU job poll argument");
    if (status->struct_size < sizeof(*status))
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "GPU job status struct is too small");
    return protect([&] {
        const dav2_gpu_job_state state = job->implementation->state();
        *status = {};
        status->struct_size = sizeof(*status);
        status->state = state;
        status->output_count = state == DAV2_GPU_JOB_CANCELLED ? 0u : 1u;
        status->source_frame_id = job->source_frame_id;
    });
}

dav2_status DAV2_CALL dav2_gpu_job_cancel(dav2_gpu_job* job) {
    if (job == nullptr) return fail(DAV2_STATUS_INVALID_ARGUMENT, "GPU job is null");
    return protect([&] {
        if (job->implementation->state() == DAV2_GPU_JOB_COMPLETE)
            throw ApiError(DAV2_STATUS_INVALID_STATE, "completed GPU job cannot be cancelled");
        job->implementation->cancel();
    });
}

void DAV2_CALL dav2_gpu_job_release(dav2_gpu_job* job) { delete job; }

dav2_status DAV2_CALL dav2_submit_hip(dav2_context* context, const dav2_hip_submit_request* request,
                                     dav2_gpu_job** job) {
    if (!context || !request || !job) return fail(DAV2_STATUS_INVALID_ARGUMENT, "null HIP submit argument");
    *job = nullptr;
    if (request->struct_size < sizeof(*request) || request->abi_version != DAV2_ABI_VERSION)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "invalid HIP submit request");
    return protect([&] {
        // vulkan_executor.cpp:669-690
        const dav2_hip_submit_request& r = *request;
        if (r.width == 0 || r.height == 0 || r.row_stride_bytes < r.width * 4ull || r.row_stride_bytes % 4u ||
            (r.pixel_format != DAV2_GPU_PIXEL_BGRA8 && r.pixel_format != DAV2_GPU_PIXEL_RGBA8) ||
            (r.flags & ~static_cast<uint32_t>(DAV2_HIP_SUBMIT_WAIT_EVENT_IPC)) != 0)
            throw std::invalid_argument("invalid HIP GPU inference request");
        // Waiting on another process's event: hipEventRecord of an
        // interprocess event was refused by the runtime on the hardware this
        // was built for, so the form could never be exercised; it is
        // reported as unsupported rather than shipped untested. Producers in
        // another process synchronise before publishing their handles.
        if (r.flags & DAV2_HIP_SUBMIT_WAIT_EVENT_IPC)
            throw ApiError(DAV2_STATUS_UNSUPPORTED, "waiting on an interprocess HIP event is not supported");
        if (static_cast<uint64_t>(r.row_stride_bytes) * r.height > r.input_byte_size ||
            r.width > static_cast<uint32_t>(INT32_MAX) || r.height > static_cast<uint32_t>(INT32_MAX))
            throw std::invalid_argument("HIP GPU input dimensions exceed the buffer");
        if (r.output_byte_size < static_cast<uint64_t>(r.width) * r.height * sizeof(float))
            throw ApiError(DAV2_STATUS_BUFFER_TOO_SMALL, "output buffer is too small");
        if ((r.input && (reinterpret_cast<uintptr_t>(r.input) & 3u)) || (r.input == nullptr && (r.input_offset & 3u)) ||
            (r.output && (reinterpret_cast<uintptr_t>(r.output) & 3u)) || (r.output == nullptr && (r.output_offset & 3u)))
            throw std::invalid_argument("HIP GPU buffers must be 4-byte aligned");
        const dav2_image_shape shape =
            network_shape(static_cast<int>(r.width), static_cast<int>(r.height), r.input_size);
        auto result = std::make_unique<dav2_gpu_job>();
        result->source_frame_id = r.source_frame_id;
        result->implementation = context->executor->submit_hip(r, shape.width, shape.height);
        *job = result.release();
    });
}

dav2_status DAV2_CALL dav2_gpu_output_acquire(dav2_gpu_job* job, uint32_t, dav2_d3d12_output_descriptor* descriptor,
                                             dav2_gpu_output_lease** lease) {
    if (job == nullptr || descriptor == nullptr || lease == nullptr)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "null GPU output acquire argument");
    *lease = nullptr;
    return fail(DAV2_STATUS_UNSUPPORTED, "GPU jobs are not available on this platform");
}

dav2_status DAV2_CALL dav2_gpu_texture_output_acquire(dav2_gpu_job* job, uint32_t,
                                                     dav2_d3d12_texture_output_descriptor* descriptor,
                                                     dav2_gpu_output_lease** lease) {
    if (job == nullptr || descriptor == nullptr || lease == nullptr)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "null GPU texture output acquire argument");
    *lease = nullptr;
    return fail(DAV2_STATUS_UNSUPPORTED, "GPU jobs are not available on this platform");
}

void DAV2_CALL dav2_gpu_output_release(dav2_gpu_output_lease*) {}

// ---- host-image paths -------------------------------------------------------
// src/dav2.cpp:630-665: network_shape, BGR8 cubic preprocessing, inference,
// bilinear resize of the raw depth back to the image; here the
// preprocessing and the resize run on the device.
dav2_status DAV2_CALL dav2_infer_bgr8(dav2_context* context, const uint8_t* bgr, int32_t image_width,
                                     int32_t image_height, ptrdiff_t row_stride_bytes, int32_t input_size,
                                     float* output_depth, size_t output_count) {
    if (context == nullptr || bgr == nullptr || output_depth == nullptr)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "null inference argument");
    const size_t required =
        image_width > 0 && image_height > 0 ? static_cast<size_t>(image_width) * static_cast<size_t>(image_height) : 0;
    if (output_count < required) return fail(DAV2_STATUS_BUFFER_TOO_SMALL, "output buffer is too small");
    return protect([&] {
        const dav2_image_shape shape = network_shape(image_width, image_height, input_size);
        // image.cpp:171-175
        if (row_stride_bytes < static_cast<ptrdiff_t>(image_width) * 3)
            throw std::invalid_argument("invalid source image");
        context->executor->infer_bgr8(bgr, image_width, image_height, static_cast<size_t>(row_stride_bytes),
                                      shape.width, shape.height, output_depth);
    });
}

// src/dav2.cpp:754-802: the InferBridge contract -- BGRA bytes kept in BGR
// order as model channels, nearest resize to the transposed network shape,
// depth min/max normalised at that size. (Metric models, which take a fixed
// 25 m span there, are refused at dav2_create by this build.)
dav2_status DAV2_CALL dav2_inferbridge_bgra8_f32(dav2_context* context, const uint8_t* bgra, int32_t image_width,
                                                int32_t image_height, ptrdiff_t row_stride_bytes, int32_t input_size,
                                                float* output_depth, size_t output_count) {
    if (context == nullptr || bgra == nullptr || output_depth == nullptr)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "null inference argument");
    return protect([&] {
        const dav2_image_shape upstream = network_shape(image_width, image_height, input_size);
        const int out_w = upstream.height, out_h = upstream.width;
        const size_t required = static_cast<size_t>(out_w) * out_h;
        if (output_count < required) throw ApiError(DAV2_STATUS_BUFFER_TOO_SMALL, "output buffer is too small");
        // image.cpp:296-300
        if (row_stride_bytes < static_cast<ptrdiff_t>(image_width) * 4)
            throw std::invalid_argument("invalid InferBridge source image");
        context->executor->infer_bgra8_normalized(bgra, image_width, image_height,
                                                  static_cast<size_t>(row_stride_bytes), out_w, out_h, output_depth);
    });
}

// ---- the hot path ------------------------------------------------------------
dav2_status DAV2_CALL dav2_infer_tensor_f32(dav2_context* context, const float* normalized_rgb_chw,
                                           int32_t network_width, int32_t network_height, float* output_depth,
                                           size_t output_count) {
    if (context == nullptr || normalized_rgb_chw == nullptr || output_depth == nullptr)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "null inference argument");
    if (network_width <= 0 || network_height <= 0 || network_width % 14 != 0 || network_height % 14 != 0)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "network dimensions must be positive multiples of 14");
    const size_t required = static_cast<size_t>(network_width) * static_cast<size_t>(network_height);
    if (output_count < required) return fail(DAV2_STATUS_BUFFER_TOO_SMALL, "output buffer is too small");
    return protect([&] {
        context->executor->infer(normalized_rgb_chw, network_width, network_height, output_depth);
    });
}

dav2_status DAV2_CALL dav2_infer_tensor_f32_device(dav2_context* context, const float* device_input, int32_t batch,
                                                  int32_t network_width, int32_t network_height,
                                                  float* device_output, size_t output_count, void* hip_stream) {
    if (context == nullptr || device_input == nullptr || device_output == nullptr)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "null inference argument");
    if (batch <= 0) return fail(DAV2_STATUS_INVALID_ARGUMENT, "batch must be positive");
    if (network_width <= 0 || network_height <= 0 || network_width % 14 != 0 || network_height % 14 != 0)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "network dimensions must be positive multiples of 14");
    const size_t required =
        static_cast<size_t>(network_width) * static_cast<size_t>(network_height) * static_cast<size_t>(batch);
    if (output_count < required) return fail(DAV2_STATUS_BUFFER_TOO_SMALL, "output buffer is too small");
    return protect([&] {
        context->executor->infer_device(device_input, batch, network_width, network_height, device_output,
                                        static_cast<hipStream_t>(hip_stream));
    });
}

dav2_status DAV2_CALL dav2_normalize_relative_device(dav2_context* context, float* device_depth, size_t count,
                                                    void* hip_stream) {
    if (context == nullptr || device_depth == nullptr || count == 0)
        return fail(DAV2_STATUS_INVALID_ARGUMENT, "invalid normalisation request");
    return protect([&] {
        context->executor->normalize_relative_device(device_depth, count, static_cast<hipStream_t>(hip_stream));
    });
}

dav2_status DAV2_CALL dav2_profile_enable(dav2_context* context, int32_t enable) {
    if (context == nullptr) return fail(DAV2_STATUS_INVALID_ARGUMENT, "context is null");
    return protect([&] { context->executor->context().profiler().set_enabled(enable != 0); });
}

dav2_status DAV2_CALL dav2_profile_report(dav2_context* context, char* json, size_t capacity) {
    if (context == nullptr || json == nullptr) return fail(DAV2_STATUS_INVALID_ARGUMENT, "null profile argument");
    std::string text;
    const dav2_status st = protect([&] {
        context->executor->context().make_current();
        text = context->executor->context().profiler().report();
    });
    if (st != DAV2_STATUS_OK) return st;
    if (text.size() + 1 > capacity) return fail(DAV2_STATUS_BUFFER_TOO_SMALL, "profile report buffer is too small");
    std::memcpy(json, text.c_str(), text.size() + 1);
    return DAV2_STATUS_OK;
}

}  // extern "C"
