// Host-image paths of the public ABI on the GPU: the reference runs these on
// the CPU (src/image.cpp) around its tensor inference.
//  - preprocess_bgr8_kernel: interleaved BGR bytes -> normalised RGB CHW at
//    the network size, OpenCV-style separable cubic resize (image.cpp:163-270);
//  - preprocess_bgra8_nearest_kernel: BGRA bytes -> channels in byte order,
//    floor-nearest resize (image.cpp:289-339);
//  - preprocess_rgba8_kernel: the GPU submit path's float32 cubic resize of
//    BGRA / RGBA words (preprocess_rgba.glsl);
//  - normalize_span_kernel: (x - min) / (max - min) (dav2.cpp:787-800).
// One thread per destination pixel. Every float32 / float64 step is the same
// IEEE operation, in the same order, as the reference's C++ (the build turns
// contraction off, so no product is fused into a following add), hence the
// same bits.

#include "common.h"
#include "dav2_hip.h"

namespace {

using namespace dav2k;

constexpr uint32_t kTileX = 64, kTileY = 4;  // 256 threads: 64 columns x 4 rows

// OpenCV's interpolateCubic with A = -0.75 in float32 (image.cpp:20-39);
// the last weight closes the partition of unity.
DAV2_DEV void opencv_cubic(float x, float c[4]) {
    const float a = -0.75f;
    const float x1 = x + 1.0f, o = 1.0f - x;
    c[0] = ((a * x1 - 5.0f * a) * x1 + 8.0f * a) * x1 - 4.0f * a;
    c[1] = ((a + 2.0f) * x - (a + 3.0f)) * x * x + 1.0f;
    c[2] = ((a + 2.0f) * o - (a + 3.0f)) * o * o + 1.0f;
    c[3] = 1.0f - c[0] - c[1] - c[2];
}

// Taps of destination index d: half-pixel centres mapped through `scale`
// (source / destination size, float64), the coordinate rounded to float32,
// its floor and the four weights; tap t reads source index base - 1 + t,
// clamped to [0, limit - 1] (image.cpp:187-196, :238-252).
DAV2_DEV void cubic_taps(uint32_t d, double scale, int limit, int idx[4], float c[4]) {
    const float coord = static_cast<float>((static_cast<double>(d) + 0.5) * scale - 0.5);
    const int base = static_cast<int>(floorf(coord));
    opencv_cubic(coord - static_cast<float>(base), c);
#pragma unroll
    for (int t = 0; t < 4; ++t) idx[t] = min(max(base - 1 + t, 0), limit - 1);
}

__global__ __launch_bounds__(kTileX* kTileY) void preprocess_bgr8_kernel(const uint8_t* __restrict__ bgr,
                                                                          uint32_t width, uint32_t height,
                                                                          uint64_t stride, uint32_t dst_width,
                                                                          uint32_t dst_height, double scale_x,
                                                                          double scale_y, float* __restrict__ out) {
    // byte / 255 in float64, once per workgroup
    __shared__ double unit[256];
    unit[threadIdx.x] = static_cast<double>(threadIdx.x) / 255.0;
    __syncthreads();
    const uint32_t dx = blockIdx.x * kTileX + threadIdx.x % kTileX;
    const uint32_t dy = blockIdx.y * kTileY + threadIdx.x / kTileX;
    if (dx >= dst_width || dy >= dst_height) return;
    int xs[4], ys[4];
    float cx[4], cy[4];
    cubic_taps(dx, scale_x, static_cast<int>(width), xs, cx);
    cubic_taps(dy, scale_y, static_cast<int>(height), ys, cy);
    const double mean[3] = {0.485, 0.456, 0.406}, stddev[3] = {0.229, 0.224, 0.225};
    const uint64_t plane = static_cast<uint64_t>(dst_width) * dst_height;
    const uint64_t o = static_cast<uint64_t>(dy) * dst_width + dx;
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) {
        // horizontal pass of source row ys[t] (a float64 sum from 0.0 in tap
        // order), then the vertical combination ((h0 c0 + h1 c1) + h2 c2) + h3 c3
        double v = 0.0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint8_t* row = bgr + static_cast<uint64_t>(ys[t]) * stride + (2 - ch);
            double h = 0.0;
#pragma unroll
            for (int k = 0; k < 4; ++k) h = h + unit[row[3 * xs[k]]] * static_cast<double>(cx[k]);
            const double term = h * static_cast<double>(cy[t]);
            v = t == 0 ? term : v + term;
        }
        out[ch * plane + o] = static_cast<float>((v - mean[ch]) / stddev[ch]);
    }
}

__global__ __launch_bounds__(kTileX* kTileY) void preprocess_bgra8_nearest_kernel(
    const uint8_t* __restrict__ bgra, uint32_t width, uint32_t height, uint64_t stride, uint32_t dst_width,
    uint32_t dst_height, float scale_x, float scale_y, float* __restrict__ out) {
    const uint32_t dx = blockIdx.x * kTileX + threadIdx.x % kTileX;
    const uint32_t dy = blockIdx.y * kTileY + threadIdx.x / kTileX;
    if (dx >= dst_width || dy >= dst_height) return;
    const uint32_t x = min(static_cast<uint32_t>(floorf(static_cast<float>(dx) * scale_x)), width - 1);
    const uint32_t y = min(static_cast<uint32_t>(floorf(static_cast<float>(dy) * scale_y)), height - 1);
    const uchar4 px = *reinterpret_cast<const uchar4*>(bgra + static_cast<uint64_t>(y) * stride + 4ull * x);
    const uint64_t plane = static_cast<uint64_t>(dst_width) * dst_height;
    const uint64_t o = static_cast<uint64_t>(dy) * dst_width + dx;
    const uint8_t bytes[3] = {px.x, px.y, px.z};
    const float mean[3] = {0.485f, 0.456f, 0.406f}, stddev[3] = {0.229f, 0.224f, 0.225f};
#pragma unroll
    for (int ch = 0; ch < 3; ++ch)
        out[ch * plane + o] = div_rn(div_rn(static_cast<float>(bytes[ch]), 255.0f) - mean[ch], stddev[ch]);
}

// preprocess_rgba.glsl (src/gpu_preprocess.cpp:41-104): the GPU submit
// path's resize, all in float32 -- coordinate ((d + 0.5) * src) / dst - 0.5,
// weights cubic2(f + 1), cubic1(f), cubic1(1 - f), cubic2(2 - f), row and
// column sums from 0 in tap order, byte / 255 and (v - mean) / std divided.
DAV2_DEV float rgba_cubic1(float v) { return ((1.25f * v - 2.25f) * v) * v + 1.0f; }
DAV2_DEV float rgba_cubic2(float v) {
    const float a = -0.75f;
    return ((a * v - 5.0f * a) * v + 8.0f * a) * v - 4.0f * a;
}

DAV2_DEV void rgba_taps(uint32_t d, uint32_t src, uint32_t dst, int idx[4], float c[4]) {
    const float coord = div_rn((static_cast<float>(d) + 0.5f) * static_cast<float>(src), static_cast<float>(dst)) - 0.5f;
    const int base = static_cast<int>(floorf(coord));
    const float f = coord - static_cast<float>(base);
    c[0] = rgba_cubic2(f + 1.0f);
    c[1] = rgba_cubic1(f);
    c[2] = rgba_cubic1(1.0f - f);
    c[3] = rgba_cubic2(2.0f - f);
#pragma unroll
    for (int t = 0; t < 4; ++t) idx[t] = min(max(base - 1 + t, 0), static_cast<int>(src) - 1);
}

__global__ __launch_bounds__(kTileX* kTileY) void preprocess_rgba8_kernel(const uint32_t* __restrict__ pixels,
                                                                           uint32_t width, uint32_t height,
                                                                           uint32_t stride_pixels, uint32_t dst_width,
                                                                           uint32_t dst_height, uint32_t rgba_order,
                                                                           float* __restrict__ out) {
    const uint32_t dx = blockIdx.x * kTileX + threadIdx.x % kTileX;
    const uint32_t dy = blockIdx.y * kTileY + threadIdx.x / kTileX;
    if (dx >= dst_width || dy >= dst_height) return;
    int xs[4], ys[4];
    float cx[4], cy[4];
    rgba_taps(dx, width, dst_width, xs, cx);
    rgba_taps(dy, height, dst_height, ys, cy);
    uint32_t px[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int k = 0; k < 4; ++k) px[t][k] = pixels[static_cast<uint64_t>(ys[t]) * stride_pixels + xs[k]];
    const float mean[3] = {0.485f, 0.456f, 0.406f}, stddev[3] = {0.229f, 0.224f, 0.225f};
    // channel 0 is red: byte 0 of an RGBA pixel, byte 2 of a BGRA one
    const uint32_t shifts[3] = {rgba_order ? 0u : 16u, 8u, rgba_order ? 16u : 0u};
    const uint64_t plane = static_cast<uint64_t>(dst_width) * dst_height;
    const uint64_t o = static_cast<uint64_t>(dy) * dst_width + dx;
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) {
        float resized = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float row = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float v = div_rn(static_cast<float>((px[t][k] >> shifts[ch]) & 255u), 255.0f);
                row = row + v * cx[k];
            }
            resized = resized + row * cy[t];
        }
        out[ch * plane + o] = div_rn(resized - mean[ch], stddev[ch]);
    }
}

__global__ __launch_bounds__(256) void normalize_span_kernel(const float* __restrict__ depth,
                                                             const float* __restrict__ range, uint64_t count,
                                                             float* __restrict__ out) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    if (i >= count) return;
    const float minimum = range[0];
    const float span = range[1] - minimum;
    out[i] = span > 0.0f ? div_rn(depth[i] - minimum, span) : 0.0f;
}

}  // namespace

extern "C" {

int dav2_hip_preprocess_bgr8(const uint8_t* bgr, uint32_t width, uint32_t height, uint64_t stride,
                             uint32_t dst_width, uint32_t dst_height, float* out, void* stream) {
    if (!bgr || !out || width == 0 || height == 0 || dst_width == 0 || dst_height == 0 ||
        stride < 3ull * width || width > (1u << 30) || height > (1u << 30) || dst_width > (1u << 24) ||
        dst_height > kTileY * 65535u)
        return hipErrorInvalidValue;
    const dim3 grid(ceil_div(dst_width, kTileX), ceil_div(dst_height, kTileY));
    dispatch(preprocess_bgr8_kernel, grid, dim3(kTileX * kTileY), 0, static_cast<hipStream_t>(stream), bgr,
                       width, height, stride, dst_width, dst_height,
                       static_cast<double>(width) / static_cast<double>(dst_width),
                       static_cast<double>(height) / static_cast<double>(dst_height), out);
    return hipGetLastError();
}

int dav2_hip_preprocess_bgra8_nearest(const uint8_t* bgra, uint32_t width, uint32_t height, uint64_t stride,
                                      uint32_t dst_width, uint32_t dst_height, float* out, void* stream) {
    if (!bgra || !out || width == 0 || height == 0 || dst_width == 0 || dst_height == 0 || stride < 4ull * width ||
        stride % 4u || (reinterpret_cast<uintptr_t>(bgra) & 3u) || width > (1u << 24) || height > (1u << 24) ||
        dst_width > (1u << 24) || dst_height > kTileY * 65535u)
        return hipErrorInvalidValue;
    const dim3 grid(ceil_div(dst_width, kTileX), ceil_div(dst_height, kTileY));
    dispatch(preprocess_bgra8_nearest_kernel, grid, dim3(kTileX * kTileY), 0,
                       static_cast<hipStream_t>(stream), bgra, width, height, stride, dst_width, dst_height,
                       static_cast<float>(width) / static_cast<float>(dst_width),
                       static_cast<float>(height) / static_cast<float>(dst_height), out);
    return hipGetLastError();
}

int dav2_hip_preprocess_rgba8(const uint32_t* pixels, uint32_t width, uint32_t height, uint64_t stride_bytes,
                              uint32_t dst_width, uint32_t dst_height, uint32_t rgba_order, float* out, void* stream) {
    // gpu_preprocess.cpp:50-88
    if (!pixels || !out || width == 0 || height == 0 || dst_width == 0 || dst_height == 0 || stride_bytes % 4u ||
        stride_bytes < 4ull * width || stride_bytes / 4u > 0xffffffffull || width > (1u << 24) ||
        height > (1u << 24) || dst_width > (1u << 24) || dst_height > kTileY * 65535u)
        return hipErrorInvalidValue;
    const dim3 grid(ceil_div(dst_width, kTileX), ceil_div(dst_height, kTileY));
    dispatch(preprocess_rgba8_kernel, grid, dim3(kTileX * kTileY), 0, static_cast<hipStream_t>(stream),
                       pixels, width, height, static_cast<uint32_t>(stride_bytes / 4u), dst_width, dst_height,
                       rgba_order, out);
    return hipGetLastError();
}

int dav2_hip_normalize_span(const float* depth, const float* range, uint64_t count, float* out, void* stream) {
    if (count == 0) return hipSuccess;
    if (!depth || !range || !out) return hipErrorInvalidValue;
    dispatch(normalize_span_kernel, dim3(ceil_div(count, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), depth, range, count, out);
    return hipGetLastError();
}

}  // extern "C"
