// Bandwidth-bound kernels: GELU, LayerScale residual, add, ReLU, bilinear
// (align_corners=True), global min/max, relative-depth normalisation and the
// patch-token position embedding (bicubic pos-embed + class token).

#include "common.h"
#include "dav2_hip.h"

using namespace dav2k;

namespace {

constexpr int kBlock = 256;

// Grid-stride launch size: enough workgroups to cover the whole chip a few
// times over without creating millions of tiny groups.
unsigned grid_for(uint64_t items) {
    const uint64_t g = (items + kBlock - 1) / kBlock;
    return static_cast<unsigned>(g < 65536u ? (g == 0 ? 1 : g) : 65536u);
}

// gelu.glsl:16-49 (erfc fit and operation order of the shader).
__global__ __launch_bounds__(kBlock) void gelu_kernel(float* out, const float* in, uint64_t n) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * kBlock) {
        const float v = in[i];
        out[i] = gelu_erfcc(v);
    }
}

// add_scaled.glsl:23-32
__global__ __launch_bounds__(kBlock) void add_scaled_kernel(float* out, const float* residual,
                                                            const float* addend, const float* scale,
                                                            uint64_t n, uint32_t columns) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * kBlock) {
        const float scaled = addend[i] * scale[i % columns];
        out[i] = residual[i] + scaled;
    }
}

// add.glsl / relu.glsl, float4 body + scalar tail.
__global__ __launch_bounds__(kBlock) void add_kernel(float* out, const float* l, const float* r, uint64_t n) {
    const uint64_t n4 = n / 4;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    const bool vec = ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(l) |
                       reinterpret_cast<uintptr_t>(r)) & 15) == 0;
    uint64_t i = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (vec) {
        for (; i < n4; i += stride) {
            const float4 a = reinterpret_cast<const float4*>(l)[i];
            const float4 b = reinterpret_cast<const float4*>(r)[i];
            reinterpret_cast<float4*>(out)[i] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
        }
        i = n4 * 4 + static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x;
    }
    for (; i < n; i += stride) out[i] = l[i] + r[i];
}

// data[i] = the binary16 value nearest data[i] (round to nearest even), as a
// float: the reference's float_to_half weight conversion (gpu_model.cpp:51-98).
__global__ __launch_bounds__(kBlock) void round_half_kernel(float* data, uint64_t n) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        data[i] = round_half(data[i]);
}

__global__ __launch_bounds__(kBlock) void relu_kernel(float* out, const float* in, uint64_t n) {
    const uint64_t n4 = n / 4;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    const bool vec = ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(in)) & 15) == 0;
    uint64_t i = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (vec) {
        for (; i < n4; i += stride) {
            const float4 a = reinterpret_cast<const float4*>(in)[i];
            reinterpret_cast<float4*>(out)[i] =
                make_float4(fmaxf(a.x, 0.f), fmaxf(a.y, 0.f), fmaxf(a.z, 0.f), fmaxf(a.w, 0.f));
        }
        i = n4 * 4 + static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x;
    }
    for (; i < n; i += stride) out[i] = fmaxf(in[i], 0.0f);
}

// bilinear_align_true.glsl:27-63. One thread per output pixel and
// kBilinearChannels channels: the source coordinates and weights are formed
// once (the shader's operation order) and reused for every channel, and all
// the channels' gathers are issued before the first blend.
constexpr uint32_t kBilinearChannels = 8;

// CPT channels per thread; with a maxima buffer (CPT = 32, channels % 32 ==
// 0) the thread also writes max |out| of its 32-channel group.
template <uint32_t CPT>
__global__ __launch_bounds__(kBlock) void bilinear_kernel(float* __restrict__ out, const float* __restrict__ in,
                                                          uint32_t iw, uint32_t ih, uint32_t ow, uint32_t oh,
                                                          uint32_t channels, float* __restrict__ maxima) {
    constexpr uint32_t kBilinearChannels = CPT;
    const uint32_t ox = blockIdx.x * 64u + (threadIdx.x & 63u);
    const uint32_t oy = blockIdx.y * 4u + (threadIdx.x >> 6);
    const uint32_t c0 = blockIdx.z * kBilinearChannels;
    if (ox >= ow || oy >= oh) return;
    const float sx = ow > 1 ? static_cast<float>(ox) * static_cast<float>(iw - 1) / static_cast<float>(ow - 1) : 0.0f;
    const float sy = oh > 1 ? static_cast<float>(oy) * static_cast<float>(ih - 1) / static_cast<float>(oh - 1) : 0.0f;
    const uint32_t x0 = static_cast<uint32_t>(floorf(sx));
    const uint32_t y0 = static_cast<uint32_t>(floorf(sy));
    const uint32_t x1 = min(x0 + 1u, iw - 1u);
    const uint32_t y1 = min(y0 + 1u, ih - 1u);
    const float fx = sx - static_cast<float>(x0);
    const float fy = sy - static_cast<float>(y0);
    const uint64_t iplane = static_cast<uint64_t>(ih) * iw, oplane = static_cast<uint64_t>(oh) * ow;
    const uint32_t n = min(kBilinearChannels, channels - c0);
    const float* src = in + static_cast<uint64_t>(c0) * iplane;
    float a[kBilinearChannels], b[kBilinearChannels], c[kBilinearChannels], d[kBilinearChannels];
#pragma unroll
    for (uint32_t k = 0; k < kBilinearChannels; ++k) {
        const float* p = src + static_cast<uint64_t>(min(k, n - 1u)) * iplane;  // clamped: every load valid
        a[k] = p[y0 * iw + x0];
        b[k] = p[y0 * iw + x1];
        c[k] = p[y1 * iw + x0];
        d[k] = p[y1 * iw + x1];
    }
    float* dst = out + static_cast<uint64_t>(c0) * oplane + static_cast<uint64_t>(oy) * ow + ox;
    float m = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < kBilinearChannels; ++k) {
        const float top = a[k] * (1.0f - fx) + b[k] * fx;
        const float bottom = c[k] * (1.0f - fx) + d[k] * fx;
        const float v = top * (1.0f - fy) + bottom * fy;
        if (k < n) dst[static_cast<uint64_t>(k) * oplane] = v;
        m = fmaxf(m, fabsf(v));
    }
    if (CPT == 32 && maxima) maxima[static_cast<uint64_t>(blockIdx.z) * oplane + static_cast<uint64_t>(oy) * ow + ox] = m;
}

// reduce_minmax.glsl as a grid reduction. Stage 1: each workgroup folds a
// grid-stride slice into one (min, max) pair; stage 2: one workgroup folds the
// partials. min/max are exact, so the result does not depend on the order.
constexpr uint32_t kMinMaxGroups = 1024;

__global__ __launch_bounds__(kBlock) void minmax_stage1(const float* in, uint64_t n, float* partials) {
    __shared__ float smin[kBlock / 64], smax[kBlock / 64];
    float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * kBlock) {
        const float v = in[i];
        mn = fminf(mn, v);
        mx = fmaxf(mx, v);
    }
    mn = wave_min(mn);
    mx = wave_max(mx);
    if ((threadIdx.x & 63u) == 0) {
        smin[threadIdx.x >> 6] = mn;
        smax[threadIdx.x >> 6] = mx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kBlock / 64; ++w) {
            mn = fminf(mn, smin[w]);
            mx = fmaxf(mx, smax[w]);
        }
        partials[2 * blockIdx.x] = mn;
        partials[2 * blockIdx.x + 1] = mx;
    }
}

__global__ __launch_bounds__(kBlock) void minmax_stage2(const float* partials, uint32_t groups, float* range) {
    __shared__ float smin[kBlock / 64], smax[kBlock / 64];
    float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
    for (uint32_t i = threadIdx.x; i < groups; i += kBlock) {
        mn = fminf(mn, partials[2 * i]);
        mx = fmaxf(mx, partials[2 * i + 1]);
    }
    mn = wave_min(mn);
    mx = wave_max(mx);
    if ((threadIdx.x & 63u) == 0) {
        smin[threadIdx.x >> 6] = mn;
        smax[threadIdx.x >> 6] = mx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kBlock / 64; ++w) {
            mn = fminf(mn, smin[w]);
            mx = fmaxf(mx, smax[w]);
        }
        range[0] = mn;
        range[1] = mx;
    }
}

// normalize_relative.glsl:8-16
__global__ __launch_bounds__(kBlock) void normalize_relative_kernel(float* depth, const float* range, uint64_t n) {
    const float minimum = range[0];
    const float span = range[1] - minimum;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * kBlock)
        depth[i] = span > 1.0e-12f ? fminf(fmaxf((depth[i] - minimum) / span, 0.0f), 1.0f) : 0.0f;
}

// position_bicubic.glsl:39-105 (A = -0.75, align_corners=False, clamped taps)
// reading the 37x37 patch grid of pos_embed (rows 1..1369 of [1370][D]).
DAV2_DEV void cubic_coeffs(float t, float c[4]) {
    const float a = -0.75f;
    const float x1 = t, x2 = 1.0f - t;
    const float u0 = x1 + 1.0f, u3 = x2 + 1.0f;
    c[0] = ((a * u0 - 5.0f * a) * u0 + 8.0f * a) * u0 - 4.0f * a;
    c[1] = ((a + 2.0f) * x1 - (a + 3.0f)) * x1 * x1 + 1.0f;
    c[2] = ((a + 2.0f) * x2 - (a + 3.0f)) * x2 * x2 + 1.0f;
    c[3] = ((a * u3 - 5.0f * a) * u3 + 8.0f * a) * u3 - 4.0f * a;
}

__global__ __launch_bounds__(kBlock) void position_bicubic_kernel(float* out, const float* position, uint32_t pw,
                                                                  uint32_t ph, uint32_t D, float scale_x,
                                                                  float scale_y) {
    const uint64_t spatial = static_cast<uint64_t>(pw) * ph;
    const uint64_t total = spatial * D;
    for (uint64_t idx = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; idx < total;
         idx += static_cast<uint64_t>(gridDim.x) * kBlock) {
        const uint32_t d = static_cast<uint32_t>(idx / spatial);
        const uint32_t s = static_cast<uint32_t>(idx - static_cast<uint64_t>(d) * spatial);
        const uint32_t y = s / pw, x = s - y * pw;
        const float srcx = (static_cast<float>(x) + 0.5f) * scale_x - 0.5f;
        const float srcy = (static_cast<float>(y) + 0.5f) * scale_y - 0.5f;
        const int bx = static_cast<int>(floorf(srcx));
        const int by = static_cast<int>(floorf(srcy));
        const float tx = srcx - static_cast<float>(bx);
        const float ty = srcy - static_cast<float>(by);
        float cx[4], cy[4];
        cubic_coeffs(tx, cx);
        cubic_coeffs(ty, cy);
        float rows[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int yy = min(max(by - 1 + k, 0), 36);
            float v[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int xx = min(max(bx - 1 + m, 0), 36);
                v[m] = position[static_cast<uint64_t>(xx) * D + static_cast<uint64_t>(yy) * 37u * D + d + D];
            }
            rows[k] = v[0] * cx[0] + v[1] * cx[1] + v[2] * cx[2] + v[3] * cx[3];
        }
        out[idx] = rows[0] * cy[0] + rows[1] * cy[1] + rows[2] * cy[2] + rows[3] * cy[3];
    }
}

// copy_class_token.glsl + add_position.glsl for a batch of token matrices.
__global__ __launch_bounds__(kBlock) void finish_tokens_kernel(float* tokens, const float* interp,
                                                               const float* position, const float* cls,
                                                               uint32_t spatial, uint32_t D, uint32_t batch) {
    const uint64_t per_image = static_cast<uint64_t>(spatial + 1u) * D;
    const uint64_t total = per_image * batch;
    for (uint64_t idx = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; idx < total;
         idx += static_cast<uint64_t>(gridDim.x) * kBlock) {
        const uint64_t local = idx % per_image;
        const uint32_t token = static_cast<uint32_t>(local / D);
        const uint32_t f = static_cast<uint32_t>(local - static_cast<uint64_t>(token) * D);
        if (token == 0) tokens[idx] = cls[f] + position[f];
        else tokens[idx] = tokens[idx] + interp[static_cast<uint64_t>(f) * spatial + (token - 1u)];
    }
}

}  // namespace

LaunchEvents& dav2k::launch_events() {
    thread_local LaunchEvents events{nullptr, nullptr, false};
    return events;
}

extern "C" {

int dav2_hip_launch_events(void* start, void* stop) {
    LaunchEvents& e = launch_events();
    const int launched = e.launched ? 1 : 0;
    e = LaunchEvents{static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop), false};
    return launched;
}

int dav2_hip_gelu(float* out, const float* input, uint64_t count, void* stream) {
    if (count == 0) return hipSuccess;
    if (!out || !input) return hipErrorInvalidValue;
    dispatch(gelu_kernel, dim3(grid_for(count)), dim3(kBlock), 0, static_cast<hipStream_t>(stream), out,
                       input, count);
    return hipGetLastError();
}

int dav2_hip_add_scaled(float* out, const float* residual, const float* addend, const float* scale,
                        uint64_t count, uint32_t columns, void* stream) {
    if (count == 0) return hipSuccess;
    if (!out || !residual || !addend || !scale || columns == 0) return hipErrorInvalidValue;
    dispatch(add_scaled_kernel, dim3(grid_for(count)), dim3(kBlock), 0, static_cast<hipStream_t>(stream),
                       out, residual, addend, scale, count, columns);
    return hipGetLastError();
}

int dav2_hip_add(float* out, const float* left, const float* right, uint64_t count, void* stream) {
    if (count == 0) return hipSuccess;
    if (!out || !left || !right) return hipErrorInvalidValue;
    dispatch(add_kernel, dim3(grid_for((count + 3) / 4)), dim3(kBlock), 0,
                       static_cast<hipStream_t>(stream), out, left, right, count);
    return hipGetLastError();
}

int dav2_hip_round_half(float* data, uint64_t count, void* stream) {
    if (count == 0) return hipSuccess;
    if (!data) return hipErrorInvalidValue;
    dispatch(round_half_kernel, dim3(grid_for(count)), dim3(kBlock), 0, static_cast<hipStream_t>(stream),
                       data, count);
    return hipGetLastError();
}

int dav2_hip_relu(float* out, const float* input, uint64_t count, void* stream) {
    if (count == 0) return hipSuccess;
    if (!out || !input) return hipErrorInvalidValue;
    dispatch(relu_kernel, dim3(grid_for((count + 3) / 4)), dim3(kBlock), 0,
                       static_cast<hipStream_t>(stream), out, input, count);
    return hipGetLastError();
}

int dav2_hip_bilinear_align_true(float* out, const float* input, uint32_t iw, uint32_t ih, uint32_t ow,
                                 uint32_t oh, uint32_t channels, void* stream) {
    if (ow == 0 || oh == 0 || channels == 0) return hipSuccess;
    if (!out || !input || iw == 0 || ih == 0 || channels > 65535u) return hipErrorInvalidValue;
    const dim3 grid(ceil_div(ow, 64), ceil_div(oh, 4), ceil_div(channels, kBilinearChannels));
    dispatch(bilinear_kernel<kBilinearChannels>, grid, dim3(kBlock), 0, static_cast<hipStream_t>(stream),
                       out, input, iw, ih, ow, oh, channels, nullptr);
    return hipGetLastError();
}

int dav2_hip_bilinear_align_true_maxima(float* out, float* partial, const float* input, uint32_t iw, uint32_t ih,
                                        uint32_t ow, uint32_t oh, uint32_t channels, void* stream) {
    if (ow == 0 || oh == 0 || channels == 0) return hipSuccess;
    if (!out || !partial || !input || iw == 0 || ih == 0 || channels % 32u || channels > 65535u)
        return hipErrorInvalidValue;
    const dim3 grid(ceil_div(ow, 64), ceil_div(oh, 4), channels / 32u);
    dispatch(bilinear_kernel<32>, grid, dim3(kBlock), 0, static_cast<hipStream_t>(stream), out, input, iw,
                       ih, ow, oh, channels, partial);
    return hipGetLastError();
}

uint32_t dav2_hip_minmax_partials(uint64_t count) {
    const uint64_t g = (count + kBlock - 1) / kBlock;
    return static_cast<uint32_t>(g == 0 ? 1 : (g < kMinMaxGroups ? g : kMinMaxGroups));
}

int dav2_hip_reduce_minmax(const float* input, uint64_t count, float* range, float* partials, void* stream) {
    if (!input || !range || !partials || count == 0) return hipErrorInvalidValue;
    const uint32_t groups = dav2_hip_minmax_partials(count);
    hipStream_t s = static_cast<hipStream_t>(stream);
    dispatch(minmax_stage1, dim3(groups), dim3(kBlock), 0, s, input, count, partials);
    dispatch(minmax_stage2, dim3(1), dim3(kBlock), 0, s, partials, groups, range);
    return hipGetLastError();
}

int dav2_hip_normalize_relative(float* depth, const float* range, uint64_t count, void* stream) {
    if (count == 0) return hipSuccess;
    if (!depth || !range) return hipErrorInvalidValue;
    dispatch(normalize_relative_kernel, dim3(grid_for(count)), dim3(kBlock), 0,
                       static_cast<hipStream_t>(stream), depth, range, count);
    return hipGetLastError();
}

int dav2_hip_position_bicubic(float* out, const float* position, uint32_t pw, uint32_t ph, uint32_t D,
                              void* stream) {
    if (pw == 0 || ph == 0 || D == 0) return hipSuccess;
    if (!out || !position) return hipErrorInvalidValue;
    // operators.cpp:1346-1364: exact copy scale at 37x37, else 1/((P+0.1)/37)
    // computed in double and rounded to float.
    const bool identity = pw == 37 && ph == 37;
    const float sx = identity ? 1.0f : static_cast<float>(1.0 / ((static_cast<double>(pw) + 0.1) / 37.0));
    const float sy = identity ? 1.0f : static_cast<float>(1.0 / ((static_cast<double>(ph) + 0.1) / 37.0));
    const uint64_t total = static_cast<uint64_t>(pw) * ph * D;
    dispatch(position_bicubic_kernel, dim3(grid_for(total)), dim3(kBlock), 0,
                       static_cast<hipStream_t>(stream), out, position, pw, ph, D, sx, sy);
    return hipGetLastError();
}

int dav2_hip_finish_tokens(float* tokens, const float* interpolated, const float* position,
                           const float* class_token, uint32_t pw, uint32_t ph, uint32_t D, uint32_t batch,
                           void* stream) {
    if (D == 0 || batch == 0) return hipSuccess;
    if (!tokens || !interpolated || !position || !class_token) return hipErrorInvalidValue;
    const uint64_t total = (static_cast<uint64_t>(pw) * ph + 1u) * D * batch;
    dispatch(finish_tokens_kernel, dim3(grid_for(total)), dim3(kBlock), 0,
                       static_cast<hipStream_t>(stream), tokens, interpolated, position, class_token, pw * ph, D,
                       batch);
    return hipGetLastError();
}

const char* dav2_hip_error_string(int error) { return hipGetErrorString(static_cast<hipError_t>(error)); }

}  // extern "C"
