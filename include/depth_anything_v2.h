/*
 * Depth-Anything-V2 inference library, MI355X (gfx950) build.
 *
 * Public C ABI. Every type, enumerator value, struct layout and function
 * signature here is the one the reference runtime exports from
 * include/depth_anything_v2.h (ABI version 1), so that a program linked
 * against the reference DLL links against libdepth_anything_v2.so unchanged.
 * Entry points that exist only for D3D12/Metal interop are exported and
 * return DAV2_STATUS_UNSUPPORTED on this platform.
 *
 * Additive entry points (no counterpart in the reference) are declared at the
 * end of this file under "MI355X extensions".
 */
#ifndef DEPTH_ANYTHING_V2_H
#define DEPTH_ANYTHING_V2_H

#include <stddef.h>
#include <stdint.h>

#define DAV2_API __attribute__((visibility("default")))
#define DAV2_CALL

#ifdef __cplusplus
extern "C" {
#endif

#define DAV2_ABI_VERSION 1u

typedef struct dav2_context dav2_context;
typedef struct dav2_gpu_job dav2_gpu_job;
typedef struct dav2_gpu_output_lease dav2_gpu_output_lease;

/* Reference: include/depth_anything_v2.h:29-42 */
typedef enum dav2_status {
    DAV2_STATUS_OK = 0,
    DAV2_STATUS_INVALID_ARGUMENT = 1,
    DAV2_STATUS_MODEL_IO = 2,
    DAV2_STATUS_MODEL_FORMAT = 3,
    DAV2_STATUS_VULKAN_UNAVAILABLE = 4,
    DAV2_STATUS_OUT_OF_MEMORY = 5,
    DAV2_STATUS_INFERENCE_FAILED = 6,
    DAV2_STATUS_BUFFER_TOO_SMALL = 7,
    DAV2_STATUS_UNSUPPORTED = 8,
    DAV2_STATUS_INTERNAL_ERROR = 9,
    DAV2_STATUS_INVALID_STATE = 10,
    DAV2_STATUS_CANCELLED = 11
} dav2_status;

/* Reference: include/depth_anything_v2.h:44-48 */
typedef enum dav2_encoder {
    DAV2_ENCODER_VITS = 0,
    DAV2_ENCODER_VITB = 1,
    DAV2_ENCODER_VITL = 2
} dav2_encoder;

/*
 * Reference: include/depth_anything_v2.h:50-58. vulkan_device_index keeps its
 * name for ABI compatibility and selects the HIP device ordinal here.
 */
typedef struct dav2_create_options {
    uint32_t struct_size;
    uint32_t abi_version;
    dav2_encoder encoder;
    int32_t vulkan_device_index;
    uint32_t flags;
    const char* cache_path_utf8; /* accepted and ignored: nothing is JIT-compiled */
} dav2_create_options;

/* Reference: include/depth_anything_v2.h:60-74 */
enum {
    DAV2_CREATE_FORCE_FP32 = 1u << 0u,
    DAV2_CREATE_FORCE_FP32_WEIGHTS = 1u << 1u,
    DAV2_CREATE_FORCE_FP32_ATTENTION = 1u << 2u,
    DAV2_CREATE_FORCE_FP16 = 1u << 3u,
    DAV2_CREATE_FORCE_INT8 = 1u << 4u,
    DAV2_CREATE_FORCE_METAL = 1u << 5u,
    DAV2_CREATE_FORCE_VULKAN = 1u << 6u
};

/* Reference: include/depth_anything_v2.h:76-83 */
typedef struct dav2_model_info {
    uint32_t struct_size;
    uint32_t abi_version;
    dav2_encoder encoder;
    uint32_t is_metric;
    float metric_max_depth;
    uint32_t reserved[3];
} dav2_model_info;

typedef struct dav2_image_shape {
    int32_t width;
    int32_t height;
} dav2_image_shape;

/* Reference: include/depth_anything_v2.h:90-105 */
enum {
    DAV2_GPU_CAP_D3D12_SHARED_INPUT = 1ull << 0u,
    DAV2_GPU_CAP_D3D12_FENCE_WAIT = 1ull << 1u,
    DAV2_GPU_CAP_D3D12_SHARED_OUTPUT = 1ull << 2u,
    DAV2_GPU_CAP_D3D12_FENCE_SIGNAL = 1ull << 3u,
    DAV2_GPU_CAP_ASYNC_SUBMIT = 1ull << 4u,
    DAV2_GPU_CAP_CANCELLATION = 1ull << 5u,
    DAV2_GPU_CAP_NO_HOST_PIXEL_STAGING = 1ull << 6u,
    DAV2_GPU_CAP_NO_HOST_DEPTH_STAGING = 1ull << 7u,
    DAV2_GPU_CAP_D3D12_SHARED_TEXTURE_INPUT = 1ull << 8u,
    DAV2_GPU_CAP_D3D12_SHARED_TEXTURE_OUTPUT = 1ull << 9u,
    DAV2_GPU_CAP_METAL_TEXTURE_INPUT = 1ull << 10u,
    DAV2_GPU_CAP_METAL_SHARED_EVENT_WAIT = 1ull << 11u,
    DAV2_GPU_CAP_METAL_TEXTURE_OUTPUT = 1ull << 12u,
    DAV2_GPU_CAP_METAL_SHARED_EVENT_SIGNAL = 1ull << 13u
};

typedef enum dav2_gpu_pixel_format {
    DAV2_GPU_PIXEL_BGRA8 = 1,
    DAV2_GPU_PIXEL_RGBA8 = 2,
    DAV2_GPU_PIXEL_DEPTH_FLOAT32 = 3
} dav2_gpu_pixel_format;

typedef enum dav2_gpu_job_state {
    DAV2_GPU_JOB_QUEUED = 0,
    DAV2_GPU_JOB_RUNNING = 1,
    DAV2_GPU_JOB_COMPLETE = 2,
    DAV2_GPU_JOB_FAILED = 3,
    DAV2_GPU_JOB_CANCELLED = 4
} dav2_gpu_job_state;

typedef struct dav2_gpu_capabilities {
    uint32_t struct_size;
    uint32_t abi_version;
    uint64_t flags;
    uint64_t adapter_luid;
    uint32_t maximum_in_flight_jobs;
    uint32_t reserved;
} dav2_gpu_capabilities;

/* Windows interop request layouts (reference: include/depth_anything_v2.h:138-269). */
typedef struct dav2_d3d12_submit_request {
    uint32_t struct_size;
    uint32_t abi_version;
    uint64_t shared_resource_handle;
    uint64_t resource_byte_size;
    uint32_t width;
    uint32_t height;
    uint32_t row_stride_bytes;
    uint32_t pixel_format;
    int32_t input_size;
    uint32_t reserved;
    uint64_t wait_fence_handle;
    uint64_t wait_fence_value;
    uint64_t source_frame_id;
    uint64_t timestamp_ns;
} dav2_d3d12_submit_request;

typedef struct dav2_d3d12_texture_submit_request {
    uint32_t struct_size;
    uint32_t abi_version;
    uint64_t shared_texture_handle;
    uint32_t width;
    uint32_t height;
    uint32_t pixel_format;
    int32_t input_size;
    uint64_t wait_fence_handle;
    uint64_t wait_fence_value;
    uint64_t source_frame_id;
    uint64_t timestamp_ns;
} dav2_d3d12_texture_submit_request;

typedef struct dav2_d3d12_texture_binding_request {
    uint32_t struct_size;
    uint32_t abi_version;
    uint64_t input_texture_handle;
    uint32_t input_width;
    uint32_t input_height;
    uint32_t input_pixel_format;
    int32_t input_size;
    uint64_t wait_fence_handle;
    uint64_t wait_fence_value;
    uint64_t output_texture_handle;
    uint32_t output_width;
    uint32_t output_height;
    uint64_t signal_fence_handle;
    uint64_t signal_fence_value;
    uint64_t source_frame_id;
    uint64_t timestamp_ns;
    uint64_t input_texture_identity;
    uint64_t output_texture_identity;
} dav2_d3d12_texture_binding_request;

typedef struct dav2_metal_texture_binding_request {
    uint32_t struct_size;
    uint32_t abi_version;
    uint64_t input_texture;
    uint32_t input_width;
    uint32_t input_height;
    uint32_t input_pixel_format;
    int32_t input_size;
    uint64_t wait_shared_event;
    uint64_t wait_value;
    uint64_t output_texture;
    uint32_t output_width;
    uint32_t output_height;
    uint64_t signal_shared_event;
    uint64_t signal_value;
    uint64_t source_frame_id;
    uint64_t timestamp_ns;
} dav2_metal_texture_binding_request;

typedef struct dav2_gpu_job_status {
    uint32_t struct_size;
    uint32_t state;
    uint32_t output_count;
    uint32_t reserved;
    uint64_t source_frame_id;
} dav2_gpu_job_status;

typedef struct dav2_d3d12_output_descriptor {
    uint32_t struct_size;
    uint32_t abi_version;
    uint32_t pixel_format;
    uint32_t reserved;
    uint32_t width;
    uint32_t height;
    uint32_t row_stride_bytes;
    uint32_t reserved2;
    uint64_t byte_size;
    uint64_t shared_resource_handle;
    uint64_t ready_fence_handle;
    uint64_t ready_fence_value;
    uint64_t source_frame_id;
    uint64_t timestamp_ns;
} dav2_d3d12_output_descriptor;

typedef struct dav2_d3d12_texture_output_descriptor {
    uint32_t struct_size;
    uint32_t abi_version;
    uint32_t pixel_format;
    uint32_t reserved;
    uint32_t width;
    uint32_t height;
    uint32_t reserved2;
    uint32_t reserved3;
    uint64_t shared_texture_handle;
    uint64_t ready_fence_handle;
    uint64_t ready_fence_value;
    uint64_t source_frame_id;
    uint64_t timestamp_ns;
} dav2_d3d12_texture_output_descriptor;

typedef struct dav2_transfer_counters {
    uint32_t struct_size;
    uint32_t reserved;
    uint64_t tensor_upload_bytes;
    uint64_t tensor_download_bytes;
} dav2_transfer_counters;

/* Reference: include/depth_anything_v2.h:278-281, src/dav2.cpp:96-124 */
DAV2_API uint32_t DAV2_CALL dav2_abi_version(void);
DAV2_API const char* DAV2_CALL dav2_version_string(void);
DAV2_API const char* DAV2_CALL dav2_status_string(dav2_status status);
DAV2_API const char* DAV2_CALL dav2_last_error(void);

/* Reference: include/depth_anything_v2.h:283-293, src/image.cpp:138-161 */
DAV2_API dav2_status DAV2_CALL dav2_get_network_shape(
    int32_t image_width, int32_t image_height, int32_t input_size,
    dav2_image_shape* network_shape);
DAV2_API dav2_status DAV2_CALL dav2_get_inferbridge_shape(
    int32_t image_width, int32_t image_height, int32_t input_size,
    dav2_image_shape* output_shape);

/* Reference: include/depth_anything_v2.h:295-310, src/dav2.cpp:158-229 */
DAV2_API dav2_status DAV2_CALL dav2_create(
    const char* model_path_utf8, const dav2_create_options* options,
    dav2_context** context);
DAV2_API dav2_status DAV2_CALL dav2_get_model_info(
    const dav2_context* context, dav2_model_info* info);
DAV2_API dav2_status DAV2_CALL dav2_prepare(
    dav2_context* context, int32_t image_width, int32_t image_height,
    int32_t input_size);
DAV2_API void DAV2_CALL dav2_destroy(dav2_context* context);

/* Reference: include/depth_anything_v2.h:312-322 */
DAV2_API dav2_status DAV2_CALL dav2_probe_gpu_capabilities(
    int32_t vulkan_device_index, dav2_gpu_capabilities* capabilities);
DAV2_API dav2_status DAV2_CALL dav2_get_gpu_capabilities(
    const dav2_context* context, dav2_gpu_capabilities* capabilities);
DAV2_API dav2_status DAV2_CALL dav2_get_transfer_counters(
    const dav2_context* context, dav2_transfer_counters* counters);

/* Interop (reference: include/depth_anything_v2.h:324-364): UNSUPPORTED here. */
DAV2_API dav2_status DAV2_CALL dav2_submit_d3d12(
    dav2_context* context, const dav2_d3d12_submit_request* request,
    dav2_gpu_job** job);
DAV2_API dav2_status DAV2_CALL dav2_submit_d3d12_texture(
    dav2_context* context, const dav2_d3d12_texture_submit_request* request,
    dav2_gpu_job** job);
DAV2_API dav2_status DAV2_CALL dav2_submit_d3d12_texture_binding(
    dav2_context* context, const dav2_d3d12_texture_binding_request* request,
    dav2_gpu_job** job);
DAV2_API dav2_status DAV2_CALL dav2_submit_metal_texture_binding(
    dav2_context* context, const dav2_metal_texture_binding_request* request,
    dav2_gpu_job** job);
DAV2_API dav2_status DAV2_CALL dav2_gpu_job_poll(
    const dav2_gpu_job* job, dav2_gpu_job_status* status);
DAV2_API dav2_status DAV2_CALL dav2_gpu_job_cancel(dav2_gpu_job* job);
DAV2_API void DAV2_CALL dav2_gpu_job_release(dav2_gpu_job* job);
DAV2_API dav2_status DAV2_CALL dav2_gpu_output_acquire(
    dav2_gpu_job* job, uint32_t output_index,
    dav2_d3d12_output_descriptor* descriptor, dav2_gpu_output_lease** lease);
DAV2_API dav2_status DAV2_CALL dav2_gpu_texture_output_acquire(
    dav2_gpu_job* job, uint32_t output_index,
    dav2_d3d12_texture_output_descriptor* descriptor,
    dav2_gpu_output_lease** lease);
DAV2_API void DAV2_CALL dav2_gpu_output_release(dav2_gpu_output_lease* lease);

/* Host-image paths (reference: include/depth_anything_v2.h:373-397). */
DAV2_API dav2_status DAV2_CALL dav2_infer_bgr8(
    dav2_context* context, const uint8_t* bgr, int32_t image_width,
    int32_t image_height, ptrdiff_t row_stride_bytes, int32_t input_size,
    float* output_depth, size_t output_count);
DAV2_API dav2_status DAV2_CALL dav2_inferbridge_bgra8_f32(
    dav2_context* context, const uint8_t* bgra, int32_t image_width,
    int32_t image_height, ptrdiff_t row_stride_bytes, int32_t input_size,
    float* output_depth, size_t output_count);

/*
 * The hot path. Reference: include/depth_anything_v2.h:399-410,
 * src/dav2.cpp:603-628. Input is normalised RGB planar float32 (CHW, batch 1);
 * width and height must be positive multiples of 14; output is
 * width*height float32 raw (ReLU) relative depth.
 */
DAV2_API dav2_status DAV2_CALL dav2_infer_tensor_f32(
    dav2_context* context, const float* normalized_rgb_chw,
    int32_t network_width, int32_t network_height, float* output_depth,
    size_t output_count);

/* ------------------------------------------------------------------------
 * MI355X extensions. No counterpart in the reference.
 * ------------------------------------------------------------------------ */

/*
 * Create flag (int8 mode): run the attention in the reference shaders'
 * binary16 arithmetic order -- bmm_score_fp16.glsl, softmax_lastdim_half.glsl
 * and bmm_value_fp16.glsl, every product rounded to binary16 and every sum in
 * the shaders' order (the reference's int8-mode attention on devices without
 * its cooperative-matrix score shader, src/encoder.cpp:389-396) -- instead of
 * this build's default integer-exact fused attention. The results equal the
 * CPU oracle's restatement of those shaders bit for bit; that restatement
 * uses this build's own exp (exp_cw) where the shaders call the Vulkan
 * driver's exp, and devices with the cooperative-matrix score shader sum the
 * scores in another order, so bit equality with a given Vulkan device is not
 * established. Slower than the default (about half the images per second).
 * Not combinable with FORCE_FP32 / FORCE_FP32_ATTENTION.
 */
enum { DAV2_CREATE_REFERENCE_FP16_ATTENTION = 1u << 16u };

/*
 * Create flag (int8 or fp16 mode): the reference's binary16 attention as it
 * runs on devices with cooperative_matrix_fp16 (src/operators.cpp:1137-1148):
 * the scores of bmm_score_coop_fp16.glsl -- binary16 operands, exact
 * products, fp32 sums in the matrix unit's order (here the MFMA's), each
 * score stored as binary16 -- then softmax_lastdim_half.glsl and
 * bmm_value_fp16.glsl as under DAV2_CREATE_REFERENCE_FP16_ATTENTION. The
 * shader leaves the order of the sums to the device, so the results are held
 * to the CPU oracle's restatement (products summed exactly) within a
 * tolerance, not bit for bit. Takes precedence over
 * DAV2_CREATE_REFERENCE_FP16_ATTENTION; not combinable with FORCE_FP32 /
 * FORCE_FP32_ATTENTION.
 */
enum { DAV2_CREATE_REFERENCE_FP16_COOP_ATTENTION = 1u << 17u };

/*
 * Device-resident, batched variant of dav2_infer_tensor_f32 for callers whose
 * images already live in HBM (serving loops, benchmarks). device_input holds
 * batch images, each 3*H*W float32 CHW, back to back; device_output receives
 * batch*W*H float32. hip_stream is a hipStream_t (NULL = the context's own
 * stream). The call enqueues work and returns without synchronising; the
 * output is valid once the stream has drained. Same argument checks and
 * statuses as dav2_infer_tensor_f32.
 */
DAV2_API dav2_status DAV2_CALL dav2_infer_tensor_f32_device(
    dav2_context* context, const float* device_input, int32_t batch,
    int32_t network_width, int32_t network_height, float* device_output,
    size_t output_count, void* hip_stream);

/*
 * HIP counterpart of dav2_submit_d3d12 (the reference's zero-copy GPU
 * submission, src/vulkan_executor.cpp:656-800; request layout after
 * dav2_d3d12_submit_request). The input is a device buffer of BGRA8 or RGBA8
 * pixels and the output a device buffer of width*height float32, each given
 * as a pointer in this process or, when the pointer is NULL, as a HIP IPC
 * memory handle exported by another process (plus a byte offset into that
 * allocation). The work waits for an optional HIP event of this process
 * (wait_event; DAV2_HIP_SUBMIT_WAIT_EVENT_IPC, a wait on another process's
 * event, returns DAV2_STATUS_UNSUPPORTED: a producer in another process
 * finishes its writes before it publishes the handles), then runs the
 * GPU preprocessing (float32 cubic resize to network_shape(width, height,
 * input_size)), the inference, min/max normalisation and the bilinear resize
 * back to width x height, on the device and without host copies. The returned
 * job works with dav2_gpu_job_poll (RUNNING until the GPU work has finished,
 * then COMPLETE), dav2_gpu_job_cancel (CANCELLED: the GPU work still runs,
 * its output is not to be used) and dav2_gpu_job_release (waits for the GPU
 * work, closes IPC mappings, frees the job).
 */
typedef struct dav2_hip_submit_request {
    uint32_t struct_size;
    uint32_t abi_version;
    const void* input;          /* device pointer, or NULL: input_ipc */
    uint64_t input_byte_size;   /* readable bytes from input (or from the mapping + input_offset) */
    uint32_t width;
    uint32_t height;
    uint32_t row_stride_bytes;  /* multiple of 4, >= 4 * width */
    uint32_t pixel_format;      /* DAV2_GPU_PIXEL_BGRA8 or DAV2_GPU_PIXEL_RGBA8 */
    int32_t input_size;
    uint32_t flags;             /* DAV2_HIP_SUBMIT_* */
    void* wait_event;           /* hipEvent_t, or NULL */
    float* output;              /* device pointer, or NULL: output_ipc */
    uint64_t output_byte_size;  /* >= 4 * width * height */
    uint64_t input_offset;
    uint64_t output_offset;
    uint8_t input_ipc[64];      /* hipIpcMemHandle_t */
    uint8_t output_ipc[64];     /* hipIpcMemHandle_t */
    uint8_t wait_event_ipc[64]; /* reserved: DAV2_HIP_SUBMIT_WAIT_EVENT_IPC is unsupported */
    uint64_t source_frame_id;
    uint64_t timestamp_ns;
} dav2_hip_submit_request;

enum { DAV2_HIP_SUBMIT_WAIT_EVENT_IPC = 1u };

DAV2_API dav2_status DAV2_CALL dav2_submit_hip(
    dav2_context* context, const dav2_hip_submit_request* request, dav2_gpu_job** job);

/*
 * Relative-depth normalisation on device: reduce_minmax + normalize_relative
 * over count floats in place (reference semantics: src/operators.cpp:2050-2071,
 * used by src/vulkan_executor.cpp:759-787).
 */
DAV2_API dav2_status DAV2_CALL dav2_normalize_relative_device(
    dav2_context* context, float* device_depth, size_t count,
    void* hip_stream);

/*
 * Per-launch kernel timing (role of the reference's DAV2_VULKAN_PROFILE,
 * src/vulkan.cpp:874-960). While enabled, every kernel launch of the context
 * is bracketed by HIP events on its stream. dav2_profile_report synchronises
 * and writes a JSON object {kernel: {"launches", "ms", "work", "unit"}} with
 * the totals since the previous report (work = algorithmic ops or bytes),
 * then clears them. BUFFER_TOO_SMALL if capacity cannot hold the text.
 */
DAV2_API dav2_status DAV2_CALL dav2_profile_enable(dav2_context* context, int32_t enable);
DAV2_API dav2_status DAV2_CALL dav2_profile_report(dav2_context* context, char* json, size_t capacity);

#ifdef __cplusplus
}
#endif

#endif /* DEPTH_ANYTHING_V2_H */
