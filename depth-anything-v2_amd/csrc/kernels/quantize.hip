// Per-token dynamic int8 quantization, im2col + quantization, LayerNorm and
// fused LayerNorm + quantization for gfx950.
//
// Output int8 matrices are row-major [rows][ldq] bytes with ldq a multiple of
// 64 and bytes [K, ldq) zeroed, so the MFMA GEMM can stream whole 64-byte K
// steps. The first K bytes of each row are exactly the reference's packed
// 4x int8 words (little-endian byte c%4 of word c/4 = column c).

#include "common.h"
#include "dav2_hip.h"

using namespace dav2k;

namespace {

// Rows are handled one wave each; kRowsPerBlock waves per workgroup.
constexpr int kRowsPerBlock = 4;

// Scale rule shared by every activation quantizer:
// quantize_rows_int8_fused.glsl:37 and im2col_quantize_int8.glsl:63.
DAV2_DEV float row_scale(float absmax) { return fmaxf(absmax / 127.0f, 1.0e-8f); }

// ---------------------------------------------------------------------------
// a1: quantize_rows_int8_fused.glsl:20-55. q = rne(clamp(x / s)).
// Lane l owns float4 chunks at columns 4l + 256j; CH = chunks kept in VGPRs.
template <int CH>
__global__ __launch_bounds__(64 * kRowsPerBlock) void quantize_rows_kernel(
    const float* __restrict__ input, uint64_t input_offset, uint32_t rows,
    uint32_t columns, int8_t* __restrict__ q, uint32_t ldq,
    float* __restrict__ scales) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* x = input + input_offset + static_cast<uint64_t>(row) * columns;
    const uint32_t words = columns >> 2;
    float4 v[CH];
    float absmax = 0.0f;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
        const uint32_t w = lane + 64u * j;
        v[j] = w < words ? *reinterpret_cast<const float4*>(x + 4u * w) : make_float4(0.f, 0.f, 0.f, 0.f);
        absmax = fmaxf(absmax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
    }
    absmax = wave_max(absmax);
    const float s = row_scale(absmax);
    if (lane == 0) scales[row] = s;
    uint32_t* out = reinterpret_cast<uint32_t*>(q + static_cast<uint64_t>(row) * ldq);
#pragma unroll
    for (int j = 0; j < CH; ++j) {
        const uint32_t w = lane + 64u * j;
        if (w < words)
            out[w] = pack4(quantize_rne(v[j].x / s), quantize_rne(v[j].y / s),
                           quantize_rne(v[j].z / s), quantize_rne(v[j].w / s));
    }
    for (uint32_t w = words + lane; w < (ldq >> 2); w += 64u) out[w] = 0u;
}

// Rows too long to hold in registers: read twice.
__global__ __launch_bounds__(64 * kRowsPerBlock) void quantize_rows_long_kernel(
    const float* __restrict__ input, uint64_t input_offset, uint32_t rows,
    uint32_t columns, int8_t* __restrict__ q, uint32_t ldq,
    float* __restrict__ scales) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* x = input + input_offset + static_cast<uint64_t>(row) * columns;
    const uint32_t words = columns >> 2;
    float absmax = 0.0f;
    for (uint32_t w = lane; w < words; w += 64u) {
        const float4 v = *reinterpret_cast<const float4*>(x + 4u * w);
        absmax = fmaxf(absmax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    absmax = wave_max(absmax);
    const float s = row_scale(absmax);
    if (lane == 0) scales[row] = s;
    uint32_t* out = reinterpret_cast<uint32_t*>(q + static_cast<uint64_t>(row) * ldq);
    for (uint32_t w = lane; w < words; w += 64u) {
        const float4 v = *reinterpret_cast<const float4*>(x + 4u * w);
        out[w] = pack4(quantize_rne(v.x / s), quantize_rne(v.y / s), quantize_rne(v.z / s),
                       quantize_rne(v.w / s));
    }
    for (uint32_t w = words + lane; w < (ldq >> 2); w += 64u) out[w] = 0u;
}

// ---------------------------------------------------------------------------
// a2: im2col_quantize_int8.glsl:26-83. Column c of output row r reads
// input[ic][oy*stride+ky-pad][ox*stride+kx-pad] with ic = c / k^2,
// ky = (c % k^2) / k, kx = c % k, zero outside the image; the row is scaled
// by s = max(absmax/127, 1e-8) and quantized as rne(clamp(x * (1/s))).

struct FastDivU32 {
    // Exact floor(n / d) for n < 2^24 via a float reciprocal and one fix-up.
    uint32_t d;
    float inv;
    DAV2_DEV uint32_t div(uint32_t n) const {
        uint32_t q = static_cast<uint32_t>(static_cast<float>(n) * inv);
        if (q * d > n) --q;
        else if ((q + 1u) * d <= n) ++q;
        return q;
    }
};

struct Im2colGeometry {
    const float* input;
    uint32_t iw, ih, ow, k, stride;
    int32_t pad;
    uint32_t columns;  // ic*k*k
    FastDivU32 div_ow, div_area, div_k;
    uint64_t plane;    // iw*ih
};

DAV2_DEV float im2col_value(const Im2colGeometry& g, uint32_t oy, uint32_t ox, uint32_t c) {
    const uint32_t ic = g.div_area.div(c);
    const uint32_t kidx = c - ic * g.div_area.d;
    const uint32_t ky = g.div_k.div(kidx);
    const uint32_t kx = kidx - ky * g.k;
    const int32_t ix = static_cast<int32_t>(ox * g.stride + kx) - g.pad;
    const int32_t iy = static_cast<int32_t>(oy * g.stride + ky) - g.pad;
    if (ix < 0 || iy < 0 || ix >= static_cast<int32_t>(g.iw) || iy >= static_cast<int32_t>(g.ih)) return 0.0f;
    return g.input[ic * g.plane + static_cast<uint64_t>(iy) * g.iw + static_cast<uint32_t>(ix)];
}

// Pass 1: one wave per output row computes the row scale.
__global__ __launch_bounds__(64 * kRowsPerBlock) void im2col_scale_kernel(
    Im2colGeometry g, uint32_t rows, float* __restrict__ scales) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint32_t oy = g.div_ow.div(row);
    const uint32_t ox = row - oy * g.ow;
    float absmax = 0.0f;
    for (uint32_t c = lane; c < g.columns; c += 64u) absmax = fmaxf(absmax, fabsf(im2col_value(g, oy, ox, c)));
    absmax = wave_max(absmax);
    if (lane == 0) scales[row] = row_scale(absmax);
}

// Pass 2: one thread per output word (4 columns); words beyond K are zero.
__global__ __launch_bounds__(256) void im2col_quantize_kernel(
    Im2colGeometry g, uint32_t rows, uint32_t ldq_words, const float* __restrict__ scales,
    int8_t* __restrict__ q) {
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    const uint64_t total = static_cast<uint64_t>(rows) * ldq_words;
    if (idx >= total) return;
    const uint32_t row = static_cast<uint32_t>(idx / ldq_words);
    const uint32_t w = static_cast<uint32_t>(idx - static_cast<uint64_t>(row) * ldq_words);
    const uint32_t c0 = 4u * w;
    uint32_t packed = 0u;
    if (c0 < g.columns) {
        const uint32_t oy = g.div_ow.div(row);
        const uint32_t ox = row - oy * g.ow;
        const float inverse = 1.0f / scales[row];
        int b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t c = c0 + i;
            b[i] = c < g.columns ? quantize_rne(im2col_value(g, oy, ox, c) * inverse) : 0;
        }
        packed = pack4(b[0], b[1], b[2], b[3]);
    }
    reinterpret_cast<uint32_t*>(q)[idx] = packed;
}

// ---------------------------------------------------------------------------
// a10: layer_norm.glsl:27-68. One wave per row; lane l accumulates columns
// l, l+64, ... in order and the wave reduction reproduces the 64-entry LDS
// tree, so sums, mean and variance match the reference order exactly.
// CH = ceil(columns / 64) values kept per lane (0 = re-read from memory).
// With QUANT the normalised row is also quantized (a1 rule) into q/scales;
// out may then be null.
template <int CH, bool QUANT>
__global__ __launch_bounds__(64 * kRowsPerBlock) void layer_norm_kernel(
    const float* __restrict__ input, const float* __restrict__ weight,
    const float* __restrict__ bias, uint32_t rows, uint32_t columns, float epsilon,
    float* __restrict__ out, int8_t* __restrict__ q, uint32_t ldq,
    float* __restrict__ scales) {
    extern __shared__ float lds_rows[];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t row = blockIdx.x * kRowsPerBlock + wave;
    if (row >= rows) return;
    const float* x = input + static_cast<uint64_t>(row) * columns;
    float v[CH > 0 ? CH : 1];
    float s = 0.0f, sq = 0.0f;
    if (CH > 0) {
#pragma unroll
        for (int j = 0; j < (CH > 0 ? CH : 1); ++j) {
            const uint32_t c = lane + 64u * j;
            v[j] = c < columns ? x[c] : 0.0f;
            if (c < columns) {
                s = s + v[j];
                sq = sq + v[j] * v[j];
            }
        }
    } else {
        for (uint32_t c = lane; c < columns; c += 64u) {
            const float t = x[c];
            s = s + t;
            sq = sq + t * t;
        }
    }
    s = wave_sum_tree(s);
    sq = wave_sum_tree(sq);
    const float denom = fmaxf(static_cast<float>(columns), 1.0f);
    const float mean = s / denom;
    const float var = fmaxf(sq / denom - mean * mean, 0.0f);
    const float inv = 1.0f / sqrtf(var + epsilon);
    float* y = out ? out + static_cast<uint64_t>(row) * columns : nullptr;
    float* stage = QUANT ? lds_rows + static_cast<size_t>(wave) * columns : nullptr;
    float absmax = 0.0f;
    if (CH > 0) {
#pragma unroll
        for (int j = 0; j < (CH > 0 ? CH : 1); ++j) {
            const uint32_t c = lane + 64u * j;
            if (c < columns) {
                const float r = (v[j] - mean) * inv * weight[c] + bias[c];
                if (y) y[c] = r;
                if (QUANT) {
                    stage[c] = r;
                    absmax = fmaxf(absmax, fabsf(r));
                }
            }
        }
    } else {
        for (uint32_t c = lane; c < columns; c += 64u) {
            const float r = (x[c] - mean) * inv * weight[c] + bias[c];
            if (y) y[c] = r;
            if (QUANT) {
                stage[c] = r;
                absmax = fmaxf(absmax, fabsf(r));
            }
        }
    }
    if (QUANT) {
        absmax = wave_max(absmax);
        const float sc = row_scale(absmax);
        if (lane == 0) scales[row] = sc;
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        uint32_t* qo = reinterpret_cast<uint32_t*>(q + static_cast<uint64_t>(row) * ldq);
        const uint32_t words = columns >> 2;
        for (uint32_t w = lane; w < words; w += 64u) {
            const float4 t = *reinterpret_cast<const float4*>(stage + 4u * w);
            qo[w] = pack4(quantize_rne(t.x / sc), quantize_rne(t.y / sc), quantize_rne(t.z / sc),
                          quantize_rne(t.w / sc));
        }
        for (uint32_t w = words + lane; w < (ldq >> 2); w += 64u) qo[w] = 0u;
    }
}

FastDivU32 make_div(uint32_t d) { return FastDivU32{d, 1.0f / static_cast<float>(d)}; }

template <bool QUANT>
hipError_t launch_layer_norm(const float* in, const float* w, const float* b, uint32_t rows,
                             uint32_t cols, float eps, float* out, int8_t* q, uint32_t ldq,
                             float* scales, hipStream_t stream) {
    const unsigned grid = ceil_div(rows, kRowsPerBlock);
    const size_t lds = QUANT ? static_cast<size_t>(kRowsPerBlock) * cols * sizeof(float) : 0;
    const uint32_t ch = (cols + 63u) / 64u;
#define DAV2_LN_CASE(N)                                                                   \
    hipLaunchKernelGGL((layer_norm_kernel<N, QUANT>), dim3(grid), dim3(64 * kRowsPerBlock), \
                       lds, stream, in, w, b, rows, cols, eps, out, q, ldq, scales)
    if (ch <= 6) DAV2_LN_CASE(6);
    else if (ch <= 12) DAV2_LN_CASE(12);
    else if (ch <= 16) DAV2_LN_CASE(16);
    else DAV2_LN_CASE(0);
#undef DAV2_LN_CASE
    return hipGetLastError();
}

}  // namespace

extern "C" {

int dav2_hip_quantize_rows_i8(const float* input, uint64_t input_offset, uint32_t rows,
                              uint32_t columns, int8_t* q, uint32_t ldq, float* scales,
                              void* stream) {
    if (rows == 0) return hipSuccess;
    if (!input || !q || !scales || columns == 0 || columns % 4u || ldq < columns || ldq % 64u ||
        input_offset % 4u)
        return hipErrorInvalidValue;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const unsigned grid = ceil_div(rows, kRowsPerBlock);
    const uint32_t ch = (columns / 4u + 63u) / 64u;
#define DAV2_QR_CASE(N)                                                                         \
    hipLaunchKernelGGL(quantize_rows_kernel<N>, dim3(grid), dim3(64 * kRowsPerBlock), 0, s, input, \
                       input_offset, rows, columns, q, ldq, scales)
    if (ch <= 1) DAV2_QR_CASE(1);
    else if (ch <= 2) DAV2_QR_CASE(2);
    else if (ch <= 4) DAV2_QR_CASE(4);
    else if (ch <= 8) DAV2_QR_CASE(8);
    else if (ch <= 16) DAV2_QR_CASE(16);
    else
        hipLaunchKernelGGL(quantize_rows_long_kernel, dim3(grid), dim3(64 * kRowsPerBlock), 0, s,
                           input, input_offset, rows, columns, q, ldq, scales);
#undef DAV2_QR_CASE
    return hipGetLastError();
}

int dav2_hip_im2col_quantize_i8(const float* input, uint32_t input_width, uint32_t input_height,
                                uint32_t input_channels, uint32_t output_width,
                                uint32_t output_height, uint32_t kernel, uint32_t stride,
                                int32_t padding, int8_t* q, uint32_t ldq, float* scales,
                                void* stream) {
    const uint64_t rows64 = static_cast<uint64_t>(output_width) * output_height;
    const uint64_t cols64 = static_cast<uint64_t>(input_channels) * kernel * kernel;
    if (rows64 == 0) return hipSuccess;
    if (!input || !q || !scales || kernel == 0 || stride == 0 || padding < 0 || ldq % 64u ||
        ldq < cols64 || rows64 >= (1u << 24) || cols64 >= (1u << 24))
        return hipErrorInvalidValue;
    // Every tap of every output pixel must be addressable (operators.cpp:1752-1756).
    if (static_cast<uint64_t>(output_width - 1) * stride + kernel > input_width + 2ull * padding ||
        static_cast<uint64_t>(output_height - 1) * stride + kernel > input_height + 2ull * padding)
        return hipErrorInvalidValue;
    hipStream_t s = static_cast<hipStream_t>(stream);
    Im2colGeometry g;
    g.input = input;
    g.iw = input_width;
    g.ih = input_height;
    g.ow = output_width;
    g.k = kernel;
    g.stride = stride;
    g.pad = padding;
    g.columns = static_cast<uint32_t>(cols64);
    g.div_ow = make_div(output_width);
    g.div_area = make_div(kernel * kernel);
    g.div_k = make_div(kernel);
    g.plane = static_cast<uint64_t>(input_width) * input_height;
    const uint32_t rows = static_cast<uint32_t>(rows64);
    hipLaunchKernelGGL(im2col_scale_kernel, dim3(ceil_div(rows, kRowsPerBlock)), dim3(64 * kRowsPerBlock), 0,
                       s, g, rows, scales);
    const uint32_t ldq_words = ldq / 4u;
    const uint64_t total = rows64 * ldq_words;
    hipLaunchKernelGGL(im2col_quantize_kernel, dim3(ceil_div(total, 256)), dim3(256), 0, s, g, rows,
                       ldq_words, scales, q);
    return hipGetLastError();
}

int dav2_hip_layer_norm(float* out, const float* input, const float* weight, const float* bias,
                        uint32_t rows, uint32_t columns, float epsilon, void* stream) {
    if (rows == 0) return hipSuccess;
    if (!out || !input || !weight || !bias || columns == 0) return hipErrorInvalidValue;
    return launch_layer_norm<false>(input, weight, bias, rows, columns, epsilon, out, nullptr, 0,
                                    nullptr, static_cast<hipStream_t>(stream));
}

int dav2_hip_layer_norm_quantize_i8(int8_t* q, uint32_t ldq, float* scales, float* out,
                                    const float* input, const float* weight, const float* bias,
                                    uint32_t rows, uint32_t columns, float epsilon, void* stream) {
    if (rows == 0) return hipSuccess;
    if (!q || !scales || !input || !weight || !bias || columns == 0 || columns % 4u ||
        ldq < columns || ldq % 64u || columns > 4096u)
        return hipErrorInvalidValue;
    return launch_layer_norm<true>(input, weight, bias, rows, columns, epsilon, out, q, ldq, scales,
                                   static_cast<hipStream_t>(stream));
}

}  // extern "C"
