// C ABI over dav2::HipOperators (include/dav2_ops.h).

#include "dav2_hip.h"
#include "dav2_ops.h"

#include "executor.h"
#include "operators.h"

#include <algorithm>
#include <atomic>
#include <memory>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>

struct dav2_ops {
    std::unique_ptr<dav2::HipContext> context;
    std::unique_ptr<dav2::HipOperators> ops;
    // int8 weights of the reference layout repacked to the GEMM layout when
    // their row length is not a multiple of 64 (grown on demand)
    dav2::DeviceBuffer padded_weight;
};

namespace {

thread_local std::string ops_error;

// Status mapping of the public ABI (src/dav2.cpp:71-90). The last error text
// is published through dav2_last_error() via the public entry points only, so
// keep a separate message here and mirror it there.
template <typename Function>
dav2_status guard(dav2_ops* ops, Function&& f) {
    if (ops == nullptr) return DAV2_STATUS_INVALID_ARGUMENT;
    try {
        ops->context->make_current();
        f(*ops->ops);
        return DAV2_STATUS_OK;
    } catch (const std::bad_alloc&) {
        ops_error = "out of memory";
        return DAV2_STATUS_OUT_OF_MEMORY;
    } catch (const std::invalid_argument& e) {
        ops_error = e.what();
        return DAV2_STATUS_INVALID_ARGUMENT;
    } catch (const std::exception& e) {
        ops_error = e.what();
        return DAV2_STATUS_INTERNAL_ERROR;
    }
}

dav2::DeviceBuffer v(const dav2_device_buffer& b) { return dav2::DeviceBuffer::view(b.data, b.data ? b.bytes : 0); }

std::uint32_t ld64(std::uint64_t columns) { return static_cast<std::uint32_t>((columns + 63) & ~63ull); }

// int8 weights as the reference's GpuModel hands them to its operators:
// [rows][columns] bytes, i.e. [rows][columns/4] little-endian words of four
// int8 (src/gpu_model.cpp:241-284, quantize_rows_int8_fused.glsl:51). The
// operators take rows of roundup(columns, 64) bytes with zero padding; for
// columns % 64 == 0 that is the same memory, otherwise the rows are copied
// into the instance's padded buffer (enqueued on its stream).
dav2::DeviceBuffer reference_int8_weight(dav2_ops& o, const dav2_device_buffer& w, std::uint64_t rows,
                                         std::uint64_t columns, const char* what) {
    if (rows == 0 || columns == 0 || columns % 4 != 0 || rows > 0xffffffffull || columns > 0xffffffffull)
        throw std::invalid_argument(std::string("invalid ") + what + " dimensions");
    if (w.data == nullptr || w.bytes < rows * columns) throw std::invalid_argument(std::string(what) + " is too small");
    if (columns % 64 == 0) return v(w);
    const std::uint64_t ld = ld64(columns);
    if (o.padded_weight.size() < rows * ld) {
        o.context->synchronize();  // work already queued may still read the old buffer
        o.padded_weight.reset();
        o.padded_weight = dav2::DeviceBuffer(rows * ld);
    }
    for (std::uint64_t r0 = 0; r0 < rows; r0 += 65535) {
        const std::uint64_t n = std::min<std::uint64_t>(65535, rows - r0);
        dav2::hip_check(dav2_hip_pad_rows_i8(static_cast<const std::int8_t*>(w.data) + r0 * columns,
                                             static_cast<std::uint32_t>(n), static_cast<std::uint32_t>(columns),
                                             o.padded_weight.as<std::int8_t>() + r0 * ld, static_cast<std::uint32_t>(ld),
                                             o.ops->stream()),
                        "pad int8 weight rows");
    }
    return dav2::DeviceBuffer::view(o.padded_weight.data(), rows * ld);
}

// ---------------------------------------------------------------------------
// Scratch of dav2_ops_linear_int8_noalloc: a file-scope device array, one
// copy per GPU, held from module load until the process ends. Host code
// never passes the array's name to a kernel (in host code it is a stand-in,
// not a device address): the entry point's first call on a device looks up
// that device's address of it with hipGetSymbolAddress, and every call
// passes that.
constexpr std::uint64_t kNoAllocScratchBytes = 32ull << 20;
static __device__ __align__(256) std::uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<std::uint8_t*> scratch_address[kMaxDevices];
std::mutex scratch_lookup;

// Order of the no-allocation calls on one GPU: every instance has its own
// stream, and all of them share the device's scratch, so each call makes its
// stream wait for the previous call's last kernel (an event per device,
// created with the first instance on that device) and records the event
// after its own. The mutex keeps wait + enqueue + record of one call
// together. Streams under graph capture are left alone (their work runs when
// the graph is launched, and a wait on an event recorded outside the capture
// is not allowed there).
struct NoAllocOrder {
    std::mutex mutex;
    hipEvent_t done = nullptr;
};
NoAllocOrder noalloc_order[kMaxDevices];

// Address of the current device's copy of `scratch` (the caller made
// `device` current).
std::uint8_t* device_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) throw std::runtime_error("device ordinal beyond the scratch table");
    std::uint8_t* p = scratch_address[device].load(std::memory_order_acquire);
    if (p) return p;
    std::lock_guard<std::mutex> lock(scratch_lookup);
    p = scratch_address[device].load(std::memory_order_relaxed);
    if (!p) {
        void* address = nullptr;
        const hipError_t e = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
        if (e != hipSuccess || address == nullptr)
            throw std::runtime_error(std::string("no-allocation scratch: hipGetSymbolAddress failed: ") +
                                     hipGetErrorString(e));
        p = static_cast<std::uint8_t*>(address);
        scratch_address[device].store(p, std::memory_order_release);
    }
    return p;
}

std::uint64_t align256(std::uint64_t n) { return (n + 255u) & ~255ull; }

}  // namespace

extern "C" {

DAV2_API const char* DAV2_CALL dav2_ops_last_error(void) { return ops_error.c_str(); }

dav2_ops* DAV2_CALL dav2_ops_create(int32_t device_index) {
    try {
        auto o = std::make_unique<dav2_ops>();
        o->context = std::make_unique<dav2::HipContext>(device_index);
        o->ops = std::make_unique<dav2::HipOperators>(*o->context);
        o->context->make_current();
        const int device = o->context->device();
        if (device >= 0 && device < kMaxDevices) {
            std::lock_guard<std::mutex> lock(noalloc_order[device].mutex);
            if (!noalloc_order[device].done)
                dav2::hip_check(hipEventCreateWithFlags(&noalloc_order[device].done, hipEventDisableTiming),
                                "no-allocation call order event");
        }
        return o.release();
    } catch (const std::exception& e) {
        ops_error = e.what();
        return nullptr;
    }
}

void DAV2_CALL dav2_ops_destroy(dav2_ops* ops) { delete ops; }

void* DAV2_CALL dav2_ops_stream(dav2_ops* ops) { return ops ? ops->context->stream() : nullptr; }

dav2_status DAV2_CALL dav2_ops_synchronize(dav2_ops* ops) {
    return guard(ops, [&](dav2::HipOperators& o) { o.context().synchronize(); });
}

dav2_status DAV2_CALL dav2_ops_linear_int8(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer input,
                                          dav2_device_buffer w8, dav2_device_buffer ws, dav2_device_buffer bias,
                                          uint32_t rows, uint32_t ic, uint32_t oc, int32_t gelu,
                                          int32_t weight_transposed) {
    return guard(ops, [&](dav2::HipOperators& o) {
        auto out = v(output);
        if (weight_transposed) {
            // [ic][oc] bytes, turned into rows by the operator itself
            o.linear_int8(out, v(input), v(w8), v(ws), v(bias), rows, ic, oc, gelu != 0, true);
            return;
        }
        const auto w = reference_int8_weight(*ops, w8, oc, ic, "packed INT8 weight buffer");
        o.linear_int8(out, v(input), w, v(ws), v(bias), rows, ic, oc, gelu != 0);
    });
}

// linear_int8 without allocating: the quantized rows (rows x roundup(ic, 64)
// bytes), their scales and, when ic % 64 != 0 or the weight comes transposed,
// the weight rows in the GEMM layout live in this GPU's copy of `scratch`,
// laid out [packed][scales][weight], each part 256-byte aligned. Every byte a
// kernel reads there was written earlier in the same call (the quantizer
// writes the zero padding of each row itself), so nothing needs clearing.
// Calls on one GPU are ordered through the device's event (NoAllocOrder);
// calls under graph capture are not, and captured graphs replayed while
// another call runs on the same GPU race on the array.
dav2_status DAV2_CALL dav2_ops_linear_int8_noalloc(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer input,
                                                  dav2_device_buffer w8, dav2_device_buffer ws,
                                                  dav2_device_buffer bias, uint32_t rows, uint32_t ic, uint32_t oc,
                                                  int32_t gelu, int32_t weight_transposed) {
    return guard(ops, [&](dav2::HipOperators& o) {
        if (rows == 0 || ic == 0 || oc == 0 || ic % 4 != 0)
            throw std::invalid_argument("invalid INT8 linear dimensions");
        if (w8.data == nullptr || w8.bytes < std::uint64_t(oc) * ic)
            throw std::invalid_argument(weight_transposed ? "transposed INT8 weight buffer is too small"
                                                          : "packed INT8 weight buffer is too small");
        const std::uint64_t ld = ld64(ic);
        const std::uint64_t packed_bytes = align256(std::uint64_t(rows) * ld);
        const std::uint64_t scale_bytes = align256(std::uint64_t(rows) * sizeof(float));
        const std::uint64_t weight_bytes = (ic % 64 || weight_transposed) ? align256(std::uint64_t(oc) * ld) : 0;
        if (packed_bytes + scale_bytes + weight_bytes > kNoAllocScratchBytes)
            throw std::invalid_argument(
                "linear_int8_noalloc: rows x roundup(input_columns, 64) bytes of quantized rows, their scales and "
                "the weight rows exceed the 32 MiB scratch");
        const int device = ops->context->device();
        std::uint8_t* base = device_scratch(device);
        NoAllocOrder& order = noalloc_order[device];
        std::lock_guard<std::mutex> lock(order.mutex);
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        dav2::hip_check(hipStreamIsCapturing(o.stream(), &capture), "capture status");
        const bool ordered = capture == hipStreamCaptureStatusNone && order.done != nullptr;
        if (ordered) dav2::hip_check(hipStreamWaitEvent(o.stream(), order.done, 0), "wait for the previous call");
        auto weight = v(w8);
        if (weight_bytes) {
            std::uint8_t* rows_layout = base + packed_bytes + scale_bytes;
            if (weight_transposed) {
                dav2::hip_check(dav2_hip_transpose_rows_i8(static_cast<const std::int8_t*>(w8.data), ic, oc,
                                                           reinterpret_cast<std::int8_t*>(rows_layout),
                                                           static_cast<std::uint32_t>(ld), o.stream()),
                                "transpose int8 weight");
            } else {
                for (std::uint64_t r0 = 0; r0 < oc; r0 += 65535) {
                    const std::uint64_t n = std::min<std::uint64_t>(65535, oc - r0);
                    dav2::hip_check(dav2_hip_pad_rows_i8(static_cast<const std::int8_t*>(w8.data) + r0 * ic,
                                                         static_cast<std::uint32_t>(n), ic,
                                                         reinterpret_cast<std::int8_t*>(rows_layout + r0 * ld),
                                                         static_cast<std::uint32_t>(ld), o.stream()),
                                    "pad int8 weight rows");
                }
            }
            weight = dav2::DeviceBuffer::view(rows_layout, std::uint64_t(oc) * ld);
        }
        auto out = v(output);
        o.linear_int8_in(out, v(input), weight, v(ws), v(bias), rows, ic, oc, gelu != 0,
                         dav2::DeviceBuffer::view(base, std::uint64_t(rows) * ld),
                         dav2::DeviceBuffer::view(base + packed_bytes, std::uint64_t(rows) * sizeof(float)));
        if (ordered) dav2::hip_check(hipEventRecord(order.done, o.stream()), "record the call's end");
    });
}

dav2_status DAV2_CALL dav2_ops_layer_norm(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer input,
                                         dav2_device_buffer weight, dav2_device_buffer bias, uint32_t rows,
                                         uint32_t columns, float epsilon) {
    return guard(ops, [&](dav2::HipOperators& o) {
        auto out = v(output);
        o.layer_norm(out, v(input), v(weight), v(bias), rows, columns, epsilon);
    });
}

dav2_status DAV2_CALL dav2_ops_add_scaled(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer residual,
                                         dav2_device_buffer addend, dav2_device_buffer scale, uint32_t count,
                                         uint32_t columns) {
    return guard(ops, [&](dav2::HipOperators& o) {
        auto out = v(output);
        o.add_scaled(out, v(residual), v(addend), v(scale), count, columns);
    });
}

dav2_status DAV2_CALL dav2_ops_attention_head64(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer qkv,
                                               uint32_t tokens, uint32_t heads, dav2_device_buffer scratch,
                                               int32_t precision) {
    return guard(ops, [&](dav2::HipOperators& o) {
        if (precision != DAV2_PRECISION_FP32 && precision != DAV2_PRECISION_FP16)
            throw std::invalid_argument("attention precision must be fp32 or fp16");
        auto out = v(output);
        auto s = v(scratch);
        o.attention_head64(out, v(qkv), tokens, heads, scratch.data ? &s : nullptr,
                           precision == DAV2_PRECISION_FP16 ? dav2::Precision::fp16 : dav2::Precision::fp32);
    });
}

dav2_status DAV2_CALL dav2_ops_prepare_tokens(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer image,
                                             dav2_device_buffer w8, dav2_device_buffer ws, dav2_device_buffer bias,
                                             dav2_device_buffer cls, dav2_device_buffer position, uint32_t width,
                                             uint32_t height, uint32_t embedding) {
    return guard(ops, [&](dav2::HipOperators& o) {
        auto out = v(output);
        const auto w = reference_int8_weight(*ops, w8, embedding, 3 * 14 * 14, "INT8 patch weight buffer");
        o.prepare_tokens(out, v(image), dav2::DeviceBuffer(), dav2::DeviceBuffer(), w, v(ws), v(bias), v(cls),
                         v(position), width, height, embedding, dav2::Precision::int8);
    });
}

dav2_status DAV2_CALL dav2_ops_project_tokens_int8(dav2_ops* ops, dav2_device_buffer output,
                                                  dav2_device_buffer tokens, dav2_device_buffer w8,
                                                  dav2_device_buffer ws, dav2_device_buffer bias, uint32_t width,
                                                  uint32_t height, uint32_t embedding, uint32_t channels) {
    return guard(ops, [&](dav2::HipOperators& o) {
        auto out = v(output);
        const auto w = reference_int8_weight(*ops, w8, channels, embedding, "INT8 projection weight");
        o.project_tokens_int8(out, v(tokens), w, v(ws), v(bias), width, height, embedding, channels);
    });
}

dav2_status DAV2_CALL dav2_ops_conv2d_int8(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer input,
                                          dav2_device_buffer w8, dav2_device_buffer ws, dav2_device_buffer bias,
                                          uint32_t iw, uint32_t ih, uint32_t ic, uint32_t oc, uint32_t kernel,
                                          uint32_t stride, uint32_t padding, int32_t has_bias) {
    return guard(ops, [&](dav2::HipOperators& o) {
        auto out = v(output);
        const auto w = reference_int8_weight(*ops, w8, oc, std::uint64_t(ic) * kernel * kernel, "INT8 convolution weight");
        o.conv2d_int8(out, v(input), w, v(ws), v(bias), iw, ih, ic, oc, kernel, stride, padding, has_bias != 0);
    });
}

dav2_status DAV2_CALL dav2_ops_conv_transpose_nonoverlap_int8(dav2_ops* ops, dav2_device_buffer output,
                                                             dav2_device_buffer input, dav2_device_buffer w8,
                                                             dav2_device_buffer ws, dav2_device_buffer bias,
                                                             uint32_t iw, uint32_t ih, uint32_t ic, uint32_t oc,
                                                             uint32_t kernel) {
    return guard(ops, [&](dav2::HipOperators& o) {
        auto out = v(output);
        const auto w =
            reference_int8_weight(*ops, w8, std::uint64_t(kernel) * kernel * oc, ic, "INT8 transposed weight");
        o.conv_transpose_nonoverlap_int8(out, v(input), w, v(ws), v(bias), iw, ih, ic, oc, kernel);
    });
}

dav2_status DAV2_CALL dav2_ops_linear(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer input,
                                      dav2_device_buffer weight, dav2_device_buffer bias, uint32_t rows,
                                      uint32_t input_columns, uint32_t output_columns, int32_t gelu) {
    return guard(ops, [&](dav2::HipOperators& o) {
        auto out = v(output);
        o.linear(out, v(input), v(weight), v(bias), rows, input_columns, output_columns, gelu != 0);
    });
}

dav2_status DAV2_CALL dav2_ops_project_tokens(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer tokens,
                                              dav2_device_buffer weight, dav2_device_buffer bias, uint32_t width,
                                              uint32_t height, uint32_t embedding, uint32_t channels) {
    return guard(ops, [&](dav2::HipOperators& o) {
        auto out = v(output);
        o.project_tokens(out, v(tokens), v(weight), v(bias), width, height, embedding, channels);
    });
}

dav2_status DAV2_CALL dav2_ops_conv2d(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer input,
                                      dav2_device_buffer weight, dav2_device_buffer bias, uint32_t iw, uint32_t ih,
                                      uint32_t ic, uint32_t oc, uint32_t kernel, uint32_t stride, uint32_t padding,
                                      int32_t has_bias) {
    return guard(ops, [&](dav2::HipOperators& o) {
        auto out = v(output);
        o.conv2d(out, v(input), v(weight), v(bias), iw, ih, ic, oc, kernel, stride, padding, has_bias != 0);
    });
}

dav2_status DAV2_CALL dav2_ops_conv_transpose_nonoverlap(dav2_ops* ops, dav2_device_buffer output,
                                                         dav2_device_buffer input, dav2_device_buffer weight,
                                                         dav2_device_buffer bias, uint32_t iw, uint32_t ih,
                                                         uint32_t ic, uint32_t oc, uint32_t kernel) {
    return guard(ops, [&](dav2::HipOperators& o) {
        auto out = v(output);
        o.conv_transpose_nonoverlap(out, v(input), v(weight), v(bias), iw, ih, ic, oc, kernel);
    });
}

dav2_status DAV2_CALL dav2_ops_prepare_tokens_f32(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer image,
                                                  dav2_device_buffer weight, dav2_device_buffer bias,
                                                  dav2_device_buffer cls, dav2_device_buffer position,
                                                  uint32_t width, uint32_t height, uint32_t embedding) {
    return guard(ops, [&](dav2::HipOperators& o) {
        auto out = v(output);
        o.prepare_tokens(out, v(image), v(weight), dav2::DeviceBuffer(), dav2::DeviceBuffer(), dav2::DeviceBuffer(),
                         v(bias), v(cls), v(position), width, height, embedding, dav2::Precision::fp32);
    });
}

dav2_status DAV2_CALL dav2_ops_bilinear_align_true(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer input,
                                                  uint32_t iw, uint32_t ih, uint32_t ow, uint32_t oh,
                                                  uint32_t channels) {
    return guard(ops, [&](dav2::HipOperators& o) {
        auto out = v(output);
        o.bilinear_align_true(out, v(input), iw, ih, ow, oh, channels);
    });
}

dav2_status DAV2_CALL dav2_ops_reduce_minmax(dav2_ops* ops, dav2_device_buffer input, dav2_device_buffer range,
                                            uint32_t count) {
    return guard(ops, [&](dav2::HipOperators& o) {
        auto r = v(range);
        o.reduce_minmax(v(input), r, count);
    });
}

dav2_status DAV2_CALL dav2_ops_normalize_relative(dav2_ops* ops, dav2_device_buffer depth, dav2_device_buffer range,
                                                 uint32_t count) {
    return guard(ops, [&](dav2::HipOperators& o) {
        auto d = v(depth);
        o.normalize_relative(d, v(range), count);
    });
}

dav2_status DAV2_CALL dav2_ops_relu(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer input,
                                   uint32_t count) {
    return guard(ops, [&](dav2::HipOperators& o) {
        auto out = v(output);
        o.relu(out, v(input), count);
    });
}

dav2_status DAV2_CALL dav2_ops_add(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer left,
                                  dav2_device_buffer right, uint32_t count) {
    return guard(ops, [&](dav2::HipOperators& o) {
        auto out = v(output);
        o.add(out, v(left), v(right), count);
    });
}

dav2_status DAV2_CALL dav2_ops_gelu(dav2_ops* ops, dav2_device_buffer output, dav2_device_buffer input,
                                   uint32_t count) {
    return guard(ops, [&](dav2::HipOperators& o) {
        auto out = v(output);
        o.gelu(out, v(input), count);
    });
}

dav2_status DAV2_CALL dav2_infer_tensor_f32_device_logits(dav2_context* context, const float* input, int32_t width,
                                                         int32_t height, float* depth, float* logits,
                                                         void* stream) {
    if (context == nullptr || input == nullptr || depth == nullptr || logits == nullptr) return DAV2_STATUS_INVALID_ARGUMENT;
    if (width <= 0 || height <= 0 || width % 14 != 0 || height % 14 != 0) return DAV2_STATUS_INVALID_ARGUMENT;
    try {
        context->executor->infer_device(input, 1, width, height, depth, static_cast<hipStream_t>(stream), logits);
        return DAV2_STATUS_OK;
    } catch (const std::invalid_argument& e) {
        ops_error = e.what();
        return DAV2_STATUS_INVALID_ARGUMENT;
    } catch (const std::exception& e) {
        ops_error = e.what();
        return DAV2_STATUS_INTERNAL_ERROR;
    }
}

}  // extern "C"
