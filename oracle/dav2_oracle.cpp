// CPU oracle for the int8 hot path. TEST INFRASTRUCTURE ONLY: a restatement of
// the reference runtime's operator semantics, used as the checker for the HIP
// implementation and as the timed CPU baseline. Never linked into the product.
//
// Built with -ffp-contract=off so every a*b+c below rounds twice, exactly as
// written; the GPU kernels are compiled the same way where they mirror these
// expressions.

#include "dav2_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <limits>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include <immintrin.h>
#include <omp.h>

namespace {

inline float clamp127(float v) {
    // GLSL clamp(v, -127, 127) == min(max(v, -127), 127)
    return std::min(std::max(v, -127.0f), 127.0f);
}

inline int8_t round_rne(float v) {
    // GLSL round() ties are implementation-defined; the host quantizer uses
    // std::nearbyint (gpu_model.cpp:253). The whole build pins ties-to-even.
    return static_cast<int8_t>(static_cast<int>(std::nearbyint(v)));
}

// ---------------------------------------------------------------------------
// fp16 (binary16) helpers, round to nearest even.
uint16_t f2h(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exp = (x >> 23) & 0xffu;
    uint32_t mant = x & 0x7fffffu;
    if (exp == 0xffu) return static_cast<uint16_t>(sign | (mant ? 0x7e00u : 0x7c00u));
    int e = static_cast<int>(exp) - 127 + 15;
    if (e >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return static_cast<uint16_t>(sign);
        mant |= 0x800000u;
        const uint32_t shift = static_cast<uint32_t>(14 - e);
        uint32_t r = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return static_cast<uint16_t>(sign | r);
    }
    uint32_t r = mant >> 13;
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) {
        ++r;
        if (r == 0x400u) {
            r = 0;
            ++e;
            if (e >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
        }
    }
    return static_cast<uint16_t>(sign | (static_cast<uint32_t>(e) << 10) | r);
}

float h2f(uint16_t h) {
    const uint32_t sign = (static_cast<uint32_t>(h) & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            int e = -1;
            do { ++e; mant <<= 1; } while ((mant & 0x400u) == 0);
            mant &= 0x3ffu;
            bits = sign | (static_cast<uint32_t>(127 - 15 - e) << 23) | (mant << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

inline float round_half(float f) { return h2f(f2h(f)); }

// ---------------------------------------------------------------------------
// int8 dot product; exact in int32 for |K| <= 2^31 / 127^2.
inline int32_t dot_i8(const int8_t* a, const int8_t* b, uint32_t k) {
    int32_t s = 0;
    for (uint32_t i = 0; i < k; ++i) s += static_cast<int32_t>(a[i]) * static_cast<int32_t>(b[i]);
    return s;
}

inline int32_t hsum_epi32(__m256i v) {
    __m128i x = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    x = _mm_add_epi32(x, _mm_shuffle_epi32(x, 0x4e));
    x = _mm_add_epi32(x, _mm_shuffle_epi32(x, 0xb1));
    return _mm_cvtsi128_si32(x);
}

// 2 rows of a x 4 rows of b over k: 32 bytes at a time, |a| as unsigned bytes
// times b carrying a's sign (_mm256_sign_epi8) in _mm256_maddubs_epi16 (pairs
// of products: |sum| <= 2 * 128 * 127 < 2^15 for operands in [-128, 127]
// that are not both -128; the quantizers only produce [-127, 127]), then
// widened by _mm256_madd_epi16 with ones into int32. Every sum is exact, so
// the order does not matter.
inline void dot_i8_2x4(const int8_t* a0, const int8_t* a1, const int8_t* const* bj, uint32_t k, int32_t out[2][4]) {
    const __m256i ones = _mm256_set1_epi16(1);
    __m256i acc[2][4];
    for (int r = 0; r < 2; ++r)
        for (int c = 0; c < 4; ++c) acc[r][c] = _mm256_setzero_si256();
    uint32_t kk = 0;
    for (; kk + 32 <= k; kk += 32) {
        const __m256i x0 = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(a0 + kk));
        const __m256i x1 = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(a1 + kk));
        const __m256i u0 = _mm256_abs_epi8(x0), u1 = _mm256_abs_epi8(x1);
        for (int c = 0; c < 4; ++c) {
            const __m256i y = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(bj[c] + kk));
            acc[0][c] = _mm256_add_epi32(acc[0][c],
                                         _mm256_madd_epi16(_mm256_maddubs_epi16(u0, _mm256_sign_epi8(y, x0)), ones));
            acc[1][c] = _mm256_add_epi32(acc[1][c],
                                         _mm256_madd_epi16(_mm256_maddubs_epi16(u1, _mm256_sign_epi8(y, x1)), ones));
        }
    }
    for (int c = 0; c < 4; ++c) {
        out[0][c] = hsum_epi32(acc[0][c]) + (kk < k ? dot_i8(a0 + kk, bj[c] + kk, k - kk) : 0);
        out[1][c] = hsum_epi32(acc[1][c]) + (kk < k ? dot_i8(a1 + kk, bj[c] + kk, k - kk) : 0);
    }
}

void gemm_i8_blocked(const int8_t* a, const int8_t* b, uint32_t m, uint32_t n,
                     uint32_t k, int32_t* acc) {
    constexpr uint32_t MB = 32, NB = 64;
    const uint32_t mblocks = (m + MB - 1) / MB, nblocks = (n + NB - 1) / NB;
    const int64_t tasks = static_cast<int64_t>(mblocks) * nblocks;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t t = 0; t < tasks; ++t) {
        const uint32_t mb = static_cast<uint32_t>(t / nblocks);
        const uint32_t nb = static_cast<uint32_t>(t % nblocks);
        const uint32_t m0 = mb * MB, m1 = std::min(m, m0 + MB);
        const uint32_t n0 = nb * NB, n1 = std::min(n, n0 + NB);
        uint32_t j = n0;
        for (; j + 4 <= n1; j += 4) {
            const int8_t* bj[4];
            for (int c = 0; c < 4; ++c) bj[c] = b + static_cast<size_t>(j + c) * k;
            uint32_t i = m0;
            for (; i + 2 <= m1; i += 2) {
                int32_t o[2][4];
                dot_i8_2x4(a + static_cast<size_t>(i) * k, a + static_cast<size_t>(i + 1) * k, bj, k, o);
                for (int r = 0; r < 2; ++r)
                    for (int c = 0; c < 4; ++c) acc[static_cast<size_t>(i + r) * n + j + c] = o[r][c];
            }
            for (; i < m1; ++i)
                for (int c = 0; c < 4; ++c)
                    acc[static_cast<size_t>(i) * n + j + c] = dot_i8(a + static_cast<size_t>(i) * k, bj[c], k);
        }
        for (; j < n1; ++j) {
            const int8_t* bj = b + static_cast<size_t>(j) * k;
            for (uint32_t i = m0; i < m1; ++i)
                acc[static_cast<size_t>(i) * n + j] = dot_i8(a + static_cast<size_t>(i) * k, bj, k);
        }
    }
}

// linear_int8_tiled.glsl:109-114: float(sum) * s_in[row] * s_w[col] + bias
inline float dequant(int32_t acc, float s_in, float s_w, float b) {
    float v = static_cast<float>(acc);
    v = v * s_in;
    v = v * s_w;
    return v + b;
}

// e^a: Cody-Waite reduction a = n ln2 + r (ln2 as a 16-bit head plus tail),
// degree-7 Taylor polynomial of e^r by Horner with fused multiply-adds,
// scaling by 2^n. Each step is one correctly rounded IEEE operation, the
// sequence the GPU kernels evaluate; results below e^-86 are zero.
float exp_cw(float a) {
    if (!(a > -86.0f)) return a != a ? a : 0.0f;
    if (a > 88.72f) return std::numeric_limits<float>::infinity();
    const float n = std::nearbyint(a * 1.44269504f);
    float r = std::fmaf(-n, 0.693145751953125f, a);
    r = std::fmaf(-n, 1.42860677e-6f, r);
    float p = 1.98412698e-4f;
    p = std::fmaf(p, r, 1.38888889e-3f);
    p = std::fmaf(p, r, 8.33333333e-3f);
    p = std::fmaf(p, r, 4.16666667e-2f);
    p = std::fmaf(p, r, 1.66666667e-1f);
    p = std::fmaf(p, r, 0.5f);
    p = std::fmaf(p, r, 1.0f);
    p = std::fmaf(p, r, 1.0f);
    return std::ldexp(p, static_cast<int>(n));
}

inline float gelu_value(float value) {
    // gelu.glsl:29-48: 0.5*x*(1+erf(x/sqrt2)), erf = 1 - erfc from the
    // Numerical Recipes fit (coefficients and Horner order of the shader),
    // its exp evaluated by exp_cw.
    const float x = value * 0.70710678118654752440f;
    const float magnitude = std::fabs(x);
    const float t = 1.0f / (1.0f + 0.5f * magnitude);
    float poly = t * 0.17087277f;
    poly = t * (-0.82215223f + poly);
    poly = t * (1.48851587f + poly);
    poly = t * (-1.13520398f + poly);
    poly = t * (0.27886807f + poly);
    poly = t * (-0.18628806f + poly);
    poly = t * (0.09678418f + poly);
    poly = t * (0.37409196f + poly);
    poly = t * (1.00002368f + poly);
    poly = -1.26551223f + poly;
    const float erfc_magnitude = t * exp_cw(-magnitude * magnitude + poly);
    const float erf_value = x >= 0.0f ? 1.0f - erfc_magnitude : erfc_magnitude - 1.0f;
    return 0.5f * value * (1.0f + erf_value);
}

// ---------------------------------------------------------------------------
// .dav2 reader (format: src/model.cpp:27-69, tools/export_model.py:21-38)
#pragma pack(push, 1)
struct Header {
    char magic[8];
    uint32_t version, endian, encoder, tensor_count;
    uint64_t directory_offset, directory_bytes, data_offset, file_bytes, reserved;
};
struct Record {
    char name[112];
    uint32_t dtype, rank;
    uint64_t dims[4];
    uint64_t data_offset, data_bytes, element_count;
    uint32_t crc32, flags;
    uint64_t reserved;
};
#pragma pack(pop)
static_assert(sizeof(Header) == 64, "header");
static_assert(sizeof(Record) == 192, "record");

uint32_t crc32_impl(const void* data, size_t bytes) {
    static uint32_t table[256];
    static bool init = false;
    if (!init) {
        for (uint32_t i = 0; i < 256; ++i) {
            uint32_t c = i;
            for (int b = 0; b < 8; ++b) c = (c & 1u) ? (0xedb88320u ^ (c >> 1)) : (c >> 1);
            table[i] = c;
        }
        init = true;
    }
    const auto* p = static_cast<const unsigned char*>(data);
    uint32_t c = 0xffffffffu;
    for (size_t i = 0; i < bytes; ++i) c = table[(c ^ p[i]) & 0xffu] ^ (c >> 8);
    return c ^ 0xffffffffu;
}

struct Tensor {
    std::vector<float> data;
    uint64_t dims[4] = {0, 0, 0, 0};
    uint32_t rank = 0;
    std::vector<int8_t> q;      // per-row int8 (reference weight quantizer rule)
    std::vector<float> qscale;  // per-row scale
};

}  // namespace

struct orc_model {
    int encoder = 0;
    uint32_t dim = 0, heads = 0, blocks = 0, features = 0;
    uint32_t capture[4] = {0, 0, 0, 0};
    uint32_t project[4] = {0, 0, 0, 0};
    std::unordered_map<std::string, Tensor> tensors;
    bool fp32 = false;  // graph precision of the current inference: fp32 mode,
    bool fp16 = false;  // fp16 mode, or (neither) int8

    const Tensor& t(const std::string& name) const {
        auto it = tensors.find(name);
        if (it == tensors.end()) throw std::runtime_error("oracle: missing tensor " + name);
        return it->second;
    }
};

extern "C" {

int orc_set_threads(int threads) {
    if (threads > 0) omp_set_num_threads(threads);
    return omp_get_max_threads();
}
int orc_get_threads(void) { return omp_get_max_threads(); }

uint16_t orc_float_to_half(float value) { return f2h(value); }
float orc_half_to_float(uint16_t value) { return h2f(value); }
uint32_t orc_crc32(const void* data, size_t bytes) { return crc32_impl(data, bytes); }
void orc_exp(const float* input, uint64_t count, float* out) {
    for (uint64_t i = 0; i < count; ++i) out[i] = exp_cw(input[i]);
}

void orc_quantize_rows(const float* input, uint32_t rows, uint32_t columns,
                       uint32_t input_offset, int8_t* q, float* scales) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* x = input + input_offset + static_cast<size_t>(r) * columns;
        float maximum = 0.0f;
        for (uint32_t c = 0; c < columns; ++c) maximum = std::max(maximum, std::fabs(x[c]));
        const float scale = std::max(maximum / 127.0f, 1.0e-8f);
        scales[r] = scale;
        int8_t* out = q + static_cast<size_t>(r) * columns;
        for (uint32_t c = 0; c < columns; ++c) out[c] = round_rne(clamp127(x[c] / scale));
    }
}

static inline float im2col_read(const float* input, uint32_t iw, uint32_t ih,
                                uint32_t ow, uint32_t kernel, uint32_t stride,
                                int32_t padding, uint32_t row, uint32_t column) {
    const uint32_t ox = row % ow, oy = row / ow;
    const uint32_t area = kernel * kernel;
    const uint32_t ic = column / area, kidx = column % area;
    const uint32_t kx = kidx % kernel, ky = kidx / kernel;
    const int32_t ix = static_cast<int32_t>(ox * stride + kx) - padding;
    const int32_t iy = static_cast<int32_t>(oy * stride + ky) - padding;
    if (ix < 0 || iy < 0 || ix >= static_cast<int32_t>(iw) || iy >= static_cast<int32_t>(ih)) return 0.0f;
    return input[(static_cast<size_t>(ic) * ih + static_cast<uint32_t>(iy)) * iw + static_cast<uint32_t>(ix)];
}

void orc_im2col_quantize(const float* input, uint32_t iw, uint32_t ih, uint32_t ic,
                         uint32_t ow, uint32_t oh, uint32_t kernel, uint32_t stride,
                         int32_t padding, int8_t* q, float* scales) {
    const uint32_t rows = ow * oh;
    const uint32_t columns = ic * kernel * kernel;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const uint32_t row = static_cast<uint32_t>(r);
        float maximum = 0.0f;
        for (uint32_t c = 0; c < columns; ++c)
            maximum = std::max(maximum, std::fabs(im2col_read(input, iw, ih, ow, kernel, stride, padding, row, c)));
        const float scale = std::max(maximum / 127.0f, 1.0e-8f);
        scales[r] = scale;
        const float inverse = 1.0f / scale;  // im2col_quantize_int8.glsl:68
        int8_t* out = q + static_cast<size_t>(r) * columns;
        for (uint32_t c = 0; c < columns; ++c)
            out[c] = round_rne(clamp127(im2col_read(input, iw, ih, ow, kernel, stride, padding, row, c) * inverse));
    }
}

void orc_quantize_weight_rows(const float* weight, uint64_t rows, uint64_t columns,
                              int8_t* q, float* scales) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < static_cast<int64_t>(rows); ++r) {
        const float* w = weight + static_cast<size_t>(r) * columns;
        float maximum = 0.0f;
        for (uint64_t c = 0; c < columns; ++c) maximum = std::max(maximum, std::abs(w[c]));
        const float scale = std::max(maximum / 127.0f, 1.0e-8f);
        scales[r] = scale;
        for (uint64_t c = 0; c < columns; ++c) {
            const float normalized = w[c] / scale;
            q[static_cast<size_t>(r) * columns + c] = static_cast<int8_t>(
                static_cast<int>(std::nearbyint(std::max(-127.0f, std::min(127.0f, normalized)))));
        }
    }
}

void orc_quantize_convT_weight(const float* weight, uint32_t in_channels,
                               uint32_t out_channels, uint32_t kernel, int8_t* q,
                               float* scales) {
    const uint32_t rows = kernel * kernel * out_channels;
    std::vector<float> reordered(static_cast<size_t>(rows) * in_channels);
    for (uint32_t row = 0; row < rows; ++row) {
        const uint32_t kidx = row / out_channels, oc = row % out_channels;
        const uint32_t ky = kidx / kernel, kx = kidx % kernel;
        for (uint32_t c = 0; c < in_channels; ++c)
            reordered[static_cast<size_t>(row) * in_channels + c] =
                weight[((static_cast<size_t>(c) * out_channels + oc) * kernel + ky) * kernel + kx];
    }
    orc_quantize_weight_rows(reordered.data(), rows, in_channels, q, scales);
}

void orc_gemm_i8(const int8_t* a, const int8_t* b, uint32_t m, uint32_t n, uint32_t k,
                 int32_t* acc) {
    gemm_i8_blocked(a, b, m, n, k, acc);
}

void orc_linear_epilogue(const int32_t* acc, const float* s_in, const float* s_w,
                         const float* bias, uint32_t rows, uint32_t columns,
                         uint32_t row_offset, uint32_t row_stride, int transposed,
                         float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        for (uint32_t c = 0; c < columns; ++c) {
            const float v = dequant(acc[static_cast<size_t>(r) * columns + c], s_in[r], s_w[c],
                                    bias ? bias[c] : 0.0f);
            const size_t dst_row = static_cast<size_t>(r) + row_offset;
            const size_t idx = transposed ? static_cast<size_t>(c) * row_stride + dst_row
                                          : dst_row * columns + c;
            out[idx] = v;
        }
    }
}

void orc_gelu(const float* input, uint64_t count, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < static_cast<int64_t>(count); ++i) out[i] = gelu_value(input[i]);
}

void orc_linear_int8(const float* input, const int8_t* w8, const float* w_scales,
                     const float* bias, uint32_t rows, uint32_t in_cols,
                     uint32_t out_cols, int gelu, float* out) {
    // operators.cpp:770-845: quantize_rows -> tiled int8 GEMM -> (gelu pass)
    std::vector<int8_t> q(static_cast<size_t>(rows) * in_cols);
    std::vector<float> s(rows);
    orc_quantize_rows(input, rows, in_cols, 0, q.data(), s.data());
    std::vector<int32_t> acc(static_cast<size_t>(rows) * out_cols);
    gemm_i8_blocked(q.data(), w8, rows, out_cols, in_cols, acc.data());
    orc_linear_epilogue(acc.data(), s.data(), w_scales, bias, rows, out_cols, 0, rows, 0, out);
    if (gelu) orc_gelu(out, static_cast<uint64_t>(rows) * out_cols, out);
}

void orc_layer_norm(const float* input, const float* weight, const float* bias,
                    uint32_t rows, uint32_t columns, float epsilon, float* out) {
    // layer_norm.glsl:27-68: 64 lanes, lane l sums columns l, l+64, ... in
    // order, then an LDS tree over widths 32..1.
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* x = input + static_cast<size_t>(r) * columns;
        float ps[64], pq[64];
        for (uint32_t lane = 0; lane < 64; ++lane) {
            float s = 0.0f, sq = 0.0f;
            for (uint32_t c = lane; c < columns; c += 64) {
                const float v = x[c];
                s = s + v;
                sq = sq + v * v;
            }
            ps[lane] = s;
            pq[lane] = sq;
        }
        for (uint32_t width = 32; width > 0; width >>= 1)
            for (uint32_t lane = 0; lane < width; ++lane) {
                ps[lane] = ps[lane] + ps[lane + width];
                pq[lane] = pq[lane] + pq[lane + width];
            }
        const float denom = std::max(static_cast<float>(columns), 1.0f);
        const float mean = ps[0] / denom;
        const float var = std::max(pq[0] / denom - mean * mean, 0.0f);
        const float inv = 1.0f / std::sqrt(var + epsilon);
        float* y = out + static_cast<size_t>(r) * columns;
        for (uint32_t c = 0; c < columns; ++c) y[c] = (x[c] - mean) * inv * weight[c] + bias[c];
    }
}

void orc_add_scaled(const float* residual, const float* addend, const float* scale,
                    uint64_t count, uint32_t columns, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < static_cast<int64_t>(count); ++i) {
        const float scaled = addend[i] * scale[static_cast<uint64_t>(i) % columns];
        out[i] = residual[i] + scaled;
    }
}

void orc_add(const float* left, const float* right, uint64_t count, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < static_cast<int64_t>(count); ++i) out[i] = left[i] + right[i];
}

void orc_relu(const float* input, uint64_t count, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < static_cast<int64_t>(count); ++i) out[i] = std::max(input[i], 0.0f);
}

static void softmax_row_fp32(const float* x, uint32_t columns, float* y) {
    // softmax_lastdim.glsl:19-69 (128 lanes; sum partition lane = column % 128)
    float maximum = -3.402823466e+38f;
    for (uint32_t c = 0; c < columns; ++c) maximum = std::max(maximum, x[c]);
    float partial[128];
    for (uint32_t lane = 0; lane < 128; ++lane) {
        float d = 0.0f;
        for (uint32_t c = lane; c < columns; c += 128) {
            const float e = exp_cw(x[c] - maximum);
            y[c] = e;
            d = d + e;
        }
        partial[lane] = d;
    }
    for (uint32_t stride = 64; stride > 0; stride >>= 1)
        for (uint32_t lane = 0; lane < stride; ++lane) partial[lane] = partial[lane] + partial[lane + stride];
    const float inverse = 1.0f / std::max(partial[0], 1.0e-20f);
    for (uint32_t c = 0; c < columns; ++c) y[c] = y[c] * inverse;
}

void orc_softmax_rows(const float* input, uint64_t rows, uint32_t columns, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < static_cast<int64_t>(rows); ++r)
        softmax_row_fp32(input + static_cast<size_t>(r) * columns, columns,
                         out + static_cast<size_t>(r) * columns);
}

namespace {

// 15-bit block floating point: x[i*stride] ~= X[i] * 2^exponent with
// |X| <= 16383. a = max|x| = m * 2^e (frexp, m in [0.5, 1)), exponent = e - 14,
// X = clamp(rint(x * 2^(14 - e)), -16383, 16383); an all-zero vector gets
// X = 0, exponent 0.
void block_fixed15(const float* x, size_t n, size_t stride, int32_t* X, int* exponent) {
    float a = 0.0f;
    for (size_t i = 0; i < n; ++i) a = std::max(a, std::fabs(x[i * stride]));
    if (a == 0.0f) {
        for (size_t i = 0; i < n; ++i) X[i] = 0;
        *exponent = 0;
        return;
    }
    int e = 0;
    std::frexp(a, &e);
    for (size_t i = 0; i < n; ++i) {
        const float v = std::nearbyint(std::ldexp(x[i * stride], 14 - e));
        X[i] = static_cast<int32_t>(std::min(std::max(v, -16383.0f), 16383.0f));
    }
    *exponent = e - 14;
}

// 2^x scaled to 21 bits: E = rint(min(2^n P(x - n), 2^21 - 1)) with
// n = rint(max(x, -100)) and P = 2^21 p, p the degree-5 minimax polynomial
// of 2^f on [-1/2, 1/2] (relative error 7.5e-8; coefficients computed for
// this build by the Remez exchange on the relative error, rounded to float,
// each times 2^21, an exact scaling) evaluated by Horner with fused
// multiply-adds.
float numerator21(float x) {
    constexpr float k21 = 2097152.0f;
    const float xc = std::fmax(x, -100.0f);
    const float n = std::nearbyint(xc);
    const float f = xc - n;
    float p = 1.327647245e-3f * k21;
    p = std::fmaf(p, f, 9.675540961e-3f * k21);
    p = std::fmaf(p, f, 5.550713092e-2f * k21);
    p = std::fmaf(p, f, 2.402212024e-1f * k21);
    p = std::fmaf(p, f, 6.931469440e-1f * k21);
    p = std::fmaf(p, f, 1.000000119e+0f * k21);
    const float v = std::fmin(std::ldexp(p, static_cast<int>(n)), 2097151.0f);
    return std::nearbyint(v);
}

// numerator21 of eight values at once, the same operations: round to nearest
// even (vroundps), fused multiply-adds (vfmadd), and ldexp(p, n) for n in
// [-100, 0] as the product with 2^n, exact because p * 2^n stays a normal
// float (p is near 2^21). Pinned against numerator21 in the oracle tests.
inline __m256 numerator21_x8(__m256 x) {
    constexpr float k21 = 2097152.0f;
    const __m256 xc = _mm256_max_ps(x, _mm256_set1_ps(-100.0f));
    const __m256 n = _mm256_round_ps(xc, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    const __m256 f = _mm256_sub_ps(xc, n);
    __m256 p = _mm256_set1_ps(1.327647245e-3f * k21);
    p = _mm256_fmadd_ps(p, f, _mm256_set1_ps(9.675540961e-3f * k21));
    p = _mm256_fmadd_ps(p, f, _mm256_set1_ps(5.550713092e-2f * k21));
    p = _mm256_fmadd_ps(p, f, _mm256_set1_ps(2.402212024e-1f * k21));
    p = _mm256_fmadd_ps(p, f, _mm256_set1_ps(6.931469440e-1f * k21));
    p = _mm256_fmadd_ps(p, f, _mm256_set1_ps(1.000000119e+0f * k21));
    const __m256i e = _mm256_slli_epi32(_mm256_add_epi32(_mm256_cvtps_epi32(n), _mm256_set1_epi32(127)), 23);
    const __m256 v = _mm256_min_ps(_mm256_mul_ps(p, _mm256_castsi256_ps(e)), _mm256_set1_ps(2097151.0f));
    return _mm256_round_ps(v, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
}

// Integer-exact attention (the int8-mode kernel): q*0.125 in 15-bit block
// floating point per token row, k per head (one exponent over all tokens),
// v per feature column over the tokens; X = 128 d1 + d0 (d1 in [-128, 127],
// d0 in [0, 127]).
//   H_ij = sum_f d1(Q_if) d1(K_jf),  R_ij = Q_i . K_j - 2^14 H_ij  (exact)
//   u_ij = fmaf(fp32(H), 2^14, fp32(R))      (score = u_ij * 2^(eq_i + ek))
//   c_i = ldexp(log2(e), eq_i + ek),  x_ij = fmaf(u_ij, c_i, -(max_j u_ij * c_i))
//   E_ij = numerator21(x_ij)
//   o_if = ldexp(fp32(sum_j E_ij V_jf) / fp32(sum_j E_ij), ev_f)
// Every sum is an exact integer, so no result depends on summation order.
void attention_exact(const float* qkv, uint32_t tokens, uint32_t heads, float* out,
                     float* probabilities) {
    const size_t D = static_cast<size_t>(heads) * 64;
    const size_t T = tokens;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t h = 0; h < heads; ++h) {
        std::vector<double> qd(T * 64), kd(T * 64), vd(T * 64), qh(T * 64), kh(T * 64);
        std::vector<int> qe(T), ve(64);
        int ke = 0;
        std::vector<int32_t> X(std::max<size_t>(T * 64, 64));
        std::vector<float> row(64), kall(T * 64);
        for (size_t t = 0; t < T; ++t) {
            const float* q = qkv + t * D * 3 + h * 64;
            for (int f = 0; f < 64; ++f) row[f] = q[f] * 0.125f;
            block_fixed15(row.data(), 64, 1, X.data(), &qe[t]);
            for (int f = 0; f < 64; ++f) {
                qd[t * 64 + f] = X[f];
                qh[t * 64 + f] = X[f] >> 7;  // high digit (arithmetic shift)
            }
            for (int f = 0; f < 64; ++f) kall[t * 64 + f] = q[D + f];
        }
        block_fixed15(kall.data(), T * 64, 1, X.data(), &ke);
        for (size_t i = 0; i < T * 64; ++i) {
            kd[i] = X[i];
            kh[i] = X[i] >> 7;
        }
        for (int f = 0; f < 64; ++f) {
            block_fixed15(qkv + 2 * D + h * 64 + f, T, D * 3, X.data(), &ve[f]);
            for (size_t t = 0; t < T; ++t) vd[t * 64 + f] = X[t];
        }
        // Blocks of QB query rows: each key and value row is loaded once per
        // block. Every sum below is an exact integer in double (products <
        // 2^28, score sums < 2^34, value sums < 2^52), so the order of the
        // additions does not change any result.
        constexpr size_t QB = 4;
        std::vector<float> u(QB * T);
        std::vector<double> E(QB * T);
        for (size_t i0 = 0; i0 < T; i0 += QB) {
            const size_t nb = std::min(QB, T - i0);
            float maximum[QB];
            for (size_t b = 0; b < QB; ++b) maximum[b] = -std::numeric_limits<float>::infinity();
            // rows past T repeat the last row (computed, never stored)
            const double* qi[QB];
            const double* qhi[QB];
            for (size_t b = 0; b < QB; ++b) {
                const size_t i = i0 + std::min(b, nb - 1);
                qi[b] = &qd[i * 64];
                qhi[b] = &qh[i * 64];
            }
            for (size_t j = 0; j < T; ++j) {
                const double* kj = &kd[j * 64];
                const double* khj = &kh[j * 64];
                __m256d acc[QB], acch[QB];
                for (size_t b = 0; b < QB; ++b) acc[b] = acch[b] = _mm256_setzero_pd();
                for (int f = 0; f < 64; f += 4) {
                    const __m256d kv = _mm256_loadu_pd(kj + f), khv = _mm256_loadu_pd(khj + f);
                    for (size_t b = 0; b < QB; ++b) {
                        acc[b] = _mm256_fmadd_pd(_mm256_loadu_pd(qi[b] + f), kv, acc[b]);
                        acch[b] = _mm256_fmadd_pd(_mm256_loadu_pd(qhi[b] + f), khv, acch[b]);
                    }
                }
                for (size_t b = 0; b < QB; ++b) {
                    alignas(32) double lanes[4], lanesh[4];
                    _mm256_store_pd(lanes, acc[b]);
                    _mm256_store_pd(lanesh, acch[b]);
                    const double dot = (lanes[0] + lanes[1]) + (lanes[2] + lanes[3]);
                    const double hi = (lanesh[0] + lanesh[1]) + (lanesh[2] + lanesh[3]);
                    const int32_t rest = static_cast<int32_t>(dot - hi * 16384.0);
                    const float uj = std::fmaf(static_cast<float>(hi), 16384.0f, static_cast<float>(rest));
                    u[b * T + j] = uj;
                    maximum[b] = std::max(maximum[b], uj);
                }
            }
            double L[QB];
            for (size_t b = 0; b < nb; ++b) {
                const size_t i = i0 + b;
                const float row_scale = std::ldexp(1.44269504f, qe[i] + ke);
                const float neg_ms = -(maximum[b] * row_scale);
                const float* ub = &u[b * T];
                double* Eb = &E[b * T];
                double Lb = 0.0;
                size_t j8 = 0;
                for (; j8 + 8 <= T; j8 += 8) {
                    alignas(32) float e8[8];
                    _mm256_store_ps(e8, numerator21_x8(_mm256_fmadd_ps(_mm256_loadu_ps(ub + j8),
                                                                       _mm256_set1_ps(row_scale),
                                                                       _mm256_set1_ps(neg_ms))));
                    for (int l = 0; l < 8; ++l) {
                        Eb[j8 + l] = e8[l];
                        Lb += e8[l];
                    }
                }
                for (size_t j = j8; j < T; ++j) {
                    Eb[j] = numerator21(std::fmaf(ub[j], row_scale, neg_ms));
                    Lb += Eb[j];
                }
                L[b] = Lb;
            }
            for (size_t b = nb; b < QB; ++b)
                std::fill(E.begin() + static_cast<ptrdiff_t>(b * T), E.begin() + static_cast<ptrdiff_t>((b + 1) * T),
                          0.0);
            // values, eight features at a time for the block's rows
            alignas(32) double ov[QB][64];
            for (int f0 = 0; f0 < 64; f0 += 8) {
                __m256d o[QB][2];
                for (size_t b = 0; b < QB; ++b) o[b][0] = o[b][1] = _mm256_setzero_pd();
                for (size_t j = 0; j < T; ++j) {
                    const double* vj = &vd[j * 64 + f0];
                    const __m256d v0 = _mm256_loadu_pd(vj), v1 = _mm256_loadu_pd(vj + 4);
                    for (size_t b = 0; b < QB; ++b) {
                        const __m256d e = _mm256_set1_pd(E[b * T + j]);
                        o[b][0] = _mm256_fmadd_pd(e, v0, o[b][0]);
                        o[b][1] = _mm256_fmadd_pd(e, v1, o[b][1]);
                    }
                }
                for (size_t b = 0; b < QB; ++b) {
                    _mm256_store_pd(&ov[b][f0], o[b][0]);
                    _mm256_store_pd(&ov[b][f0 + 4], o[b][1]);
                }
            }
            for (size_t b = 0; b < nb; ++b) {
                const size_t i = i0 + b;
                const float Lf = static_cast<float>(L[b]);
                float* dst = out + i * D + h * 64;
                for (int f = 0; f < 64; ++f) dst[f] = std::ldexp(static_cast<float>(ov[b][f]) / Lf, ve[f]);
                if (probabilities)
                    for (size_t j = 0; j < T; ++j)
                        probabilities[(h * T + i) * T + j] = static_cast<float>(E[b * T + j]) / Lf;
            }
        }
    }
}

}  // namespace

void orc_numerator21(const float* x, uint64_t count, float* out) {
    for (uint64_t i = 0; i < count; ++i) out[i] = numerator21(x[i]);
}

void orc_numerator21_x8(const float* x, uint64_t count, float* out) {
    uint64_t i = 0;
    for (; i + 8 <= count; i += 8) _mm256_storeu_ps(out + i, numerator21_x8(_mm256_loadu_ps(x + i)));
    for (; i < count; ++i) out[i] = numerator21(x[i]);
}

// Binary16 attention, the reference's int8-mode default (encoder.cpp:389-396
// -> operators.cpp:1132-1167 without the cooperative-matrix shader), as the
// three shaders state it:
//  * bmm_score_fp16.glsl:24-70: operands q16 = fp16(q * 0.125) and
//    k16 = fp16(k); each product q16 * k16 is a binary16 multiplication
//    (rounded to binary16), converted to float and added to an fp32 sum in
//    feature order 0..63; the sum is stored as binary16 (packHalf2x16).
//  * softmax_lastdim_half.glsl:19-65: the row maximum; per word w = (2w, 2w+1)
//    e = exp(score - max) in fp32, stored as binary16, while lane w % 128
//    adds (e.x + e.y) of its words in order to an fp32 partial; the 128
//    partials are added by the halving tree (stride 64, 32, ..., 1);
//    p = fp16(float(fp16(e)) * (1 / max(sum, 1e-20))).
//  * bmm_value_fp16.glsl:23-79: v16 = fp16(v); out = sum over source tokens
//    0..T-1 in order of float(fp16(p16 * v16)) in fp32.
// Pinned build choices where GLSL leaves latitude: binary16 rounding is to
// nearest even with subnormals, no multiply-add contraction, exp is exp_cw,
// the division is IEEE.
namespace {

// fp16(a * b) for binary16 values a, b held in floats: the fp32 product is
// exact (11 x 11 significant bits), so one rounding to binary16 is the
// binary16 multiplication. Eight lanes: F16C round-to-nearest-even.
inline __m256 mul_round_half8(__m256 a, __m256 b) {
    return _mm256_cvtph_ps(_mm256_cvtps_ph(_mm256_mul_ps(a, b), _MM_FROUND_TO_NEAREST_INT));
}

// Keys of head h feature-major [64][T8] (T8 = T rounded up to 8, zero
// padding), rounded to binary16.
std::vector<float> binary16_keys(const float* qkv, size_t T, size_t D, size_t h) {
    const size_t T8 = (T + 7) & ~size_t(7);
    std::vector<float> kt(64 * T8, 0.0f);
    for (size_t j = 0; j < T; ++j)
        for (int f = 0; f < 64; ++f) kt[f * T8 + j] = round_half(qkv[j * D * 3 + D + h * 64 + f]);
    return kt;
}

// One row of bmm_score_fp16.glsl: for every key j, features 0..63 in order,
// s = s + float(fp16(q16[f] * k16[j][f])); stored as binary16. Eight keys per
// vector.
void binary16_score_row(const float* q16, const std::vector<float>& kt, size_t T, uint16_t* hrow) {
    const size_t T8 = (T + 7) & ~size_t(7);
    for (size_t j = 0; j < T; j += 8) {
        __m256 s = _mm256_setzero_ps();
        for (int f = 0; f < 64; ++f)
            s = _mm256_add_ps(s, mul_round_half8(_mm256_set1_ps(q16[f]), _mm256_loadu_ps(&kt[f * T8 + j])));
        alignas(32) float lanes[8];
        _mm256_store_ps(lanes, s);
        for (size_t l = 0; l < 8 && j + l < T; ++l) hrow[j + l] = f2h(lanes[l]);
    }
}

// One row of bmm_score_coop_fp16.glsl:12-33: s = sum over features 0..63 of
// q16[f] * k16[j][f], every product exact, summed in double in feature order,
// rounded to fp32 (the accumulator's type), then stored as binary16
// (packHalf2x16). Four keys per vector.
void coop_score_row(const float* q16, const std::vector<float>& kt, size_t T, uint16_t* hrow) {
    const size_t T8 = (T + 7) & ~size_t(7);
    for (size_t j = 0; j < T; j += 4) {
        __m256d s = _mm256_setzero_pd();
        for (int f = 0; f < 64; ++f)
            s = _mm256_add_pd(s, _mm256_mul_pd(_mm256_set1_pd(q16[f]), _mm256_cvtps_pd(_mm_loadu_ps(&kt[f * T8 + j]))));
        alignas(16) float lanes[4];
        _mm_store_ps(lanes, _mm256_cvtpd_ps(s));
        for (size_t l = 0; l < 4 && j + l < T; ++l) hrow[j + l] = f2h(lanes[l]);
    }
}

void attention_binary16(const float* qkv, uint32_t tokens, uint32_t heads, float* out, float* probabilities,
                        bool coop) {
    const size_t D = static_cast<size_t>(heads) * 64;
    const size_t T = tokens;
    // Per head: keys feature-major and values token-major [T][64], rounded to
    // binary16 once.
    std::vector<std::vector<float>> keys_t(heads), values(heads);
#pragma omp parallel for schedule(static)
    for (int64_t h = 0; h < heads; ++h) {
        keys_t[h] = binary16_keys(qkv, T, D, h);
        values[h].resize(T * 64);
        for (size_t j = 0; j < T; ++j)
            for (int f = 0; f < 64; ++f) values[h][j * 64 + f] = round_half(qkv[j * D * 3 + 2 * D + h * 64 + f]);
    }
#pragma omp parallel
    {
        std::vector<uint16_t> hrow(T + 1);
        std::vector<float> p(T);
#pragma omp for schedule(dynamic, 4) collapse(2)
        for (int64_t h = 0; h < heads; ++h) {
            for (int64_t i = 0; i < static_cast<int64_t>(T); ++i) {
                const float* q = qkv + static_cast<size_t>(i) * D * 3 + h * 64;
                float q16[64];
                for (int f = 0; f < 64; ++f) q16[f] = round_half(q[f] * 0.125f);
                if (coop)
                    coop_score_row(q16, keys_t[h], T, hrow.data());
                else
                    binary16_score_row(q16, keys_t[h], T, hrow.data());
                // softmax over the packed row
                float maximum = -3.402823466e+38f;
                for (size_t j = 0; j < T; ++j) maximum = std::max(maximum, h2f(hrow[j]));
                const size_t words = (T + 1) / 2;
                float partial[128];
                for (uint32_t lane = 0; lane < 128; ++lane) {
                    float d = 0.0f;
                    for (size_t w = lane; w < words; w += 128) {
                        const size_t j0 = 2 * w, j1 = 2 * w + 1;
                        const float ex = exp_cw(h2f(hrow[j0]) - maximum);
                        const float ey = j1 < T ? exp_cw(h2f(hrow[j1]) - maximum) : 0.0f;
                        hrow[j0] = f2h(ex);
                        if (j1 < T) hrow[j1] = f2h(ey);
                        d = d + (ex + ey);
                    }
                    partial[lane] = d;
                }
                for (uint32_t stride = 64; stride > 0; stride >>= 1)
                    for (uint32_t lane = 0; lane < stride; ++lane) partial[lane] = partial[lane] + partial[lane + stride];
                const float inverse = 1.0f / std::max(partial[0], 1.0e-20f);
                for (size_t j = 0; j < T; ++j) p[j] = round_half(h2f(hrow[j]) * inverse);
                // values: eight features per vector, source tokens in order
                const std::vector<float>& vr = values[h];
                float* o = out + static_cast<size_t>(i) * D + h * 64;
                for (int f0 = 0; f0 < 64; f0 += 8) {
                    __m256 s = _mm256_setzero_ps();
                    for (size_t j = 0; j < T; ++j)
                        s = _mm256_add_ps(s, mul_round_half8(_mm256_set1_ps(p[j]), _mm256_loadu_ps(&vr[j * 64 + f0])));
                    _mm256_storeu_ps(o + f0, s);
                }
                if (probabilities) std::memcpy(probabilities + (h * T + i) * T, p.data(), T * sizeof(float));
            }
        }
    }
}

}  // namespace

void orc_attention_scores_binary16(const float* qkv, uint32_t tokens, uint32_t heads, uint16_t* scores) {
    const size_t D = static_cast<size_t>(heads) * 64, T = tokens;
    for (size_t h = 0; h < heads; ++h) {
        const std::vector<float> kt = binary16_keys(qkv, T, D, h);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < static_cast<int64_t>(T); ++i) {
            float q16[64];
            for (int f = 0; f < 64; ++f) q16[f] = round_half(qkv[i * D * 3 + h * 64 + f] * 0.125f);
            binary16_score_row(q16, kt, T, scores + (h * T + i) * T);
        }
    }
}

void orc_attention_scores_coop(const float* qkv, uint32_t tokens, uint32_t heads, uint16_t* scores) {
    const size_t D = static_cast<size_t>(heads) * 64, T = tokens;
    for (size_t h = 0; h < heads; ++h) {
        const std::vector<float> kt = binary16_keys(qkv, T, D, h);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < static_cast<int64_t>(T); ++i) {
            float q16[64];
            for (int f = 0; f < 64; ++f) q16[f] = round_half(qkv[i * D * 3 + h * 64 + f] * 0.125f);
            coop_score_row(q16, kt, T, scores + (h * T + i) * T);
        }
    }
}

void orc_round_half_product(const float* a, const float* b, uint64_t count, float* out) {
    uint64_t i = 0;
    for (; i + 8 <= count; i += 8)
        _mm256_storeu_ps(out + i, mul_round_half8(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i)));
    for (; i < count; ++i) out[i] = round_half(a[i] * b[i]);
}

void orc_attention_head64(const float* qkv, uint32_t tokens, uint32_t heads, int mode,
                          float* out, float* probabilities) {
    if (mode == 2) {
        attention_exact(qkv, tokens, heads, out, probabilities);
        return;
    }
    const size_t D = static_cast<size_t>(heads) * 64;
    const size_t T = tokens;
    if (mode == 1 || mode == 3) {
        attention_binary16(qkv, tokens, heads, out, probabilities, mode == 3);
        return;
    }
#pragma omp parallel
    {
        std::vector<float> row(T), p(T);
#pragma omp for schedule(dynamic, 4) collapse(2)
        for (int64_t h = 0; h < heads; ++h) {
            for (int64_t i = 0; i < static_cast<int64_t>(T); ++i) {
                const float* q = qkv + static_cast<size_t>(i) * D * 3 + h * 64;
                // bmm.glsl with input_qkv_query=1, weight_qkv_kind=1: sequential
                // accumulation over the 64 features of (q*0.125)*k.
                for (size_t j = 0; j < T; ++j) {
                    const float* k = qkv + j * D * 3 + D + h * 64;
                    float s = 0.0f;
                    for (int f = 0; f < 64; ++f) {
                        const float sq = q[f] * 0.125f;
                        s = s + sq * k[f];
                    }
                    row[j] = s;
                }
                softmax_row_fp32(row.data(), tokens, p.data());
                // bmm.glsl value pass: sequential over source tokens j.
                float* o = out + static_cast<size_t>(i) * D + h * 64;
                for (int f = 0; f < 64; ++f) {
                    float s = 0.0f;
                    for (size_t j = 0; j < T; ++j) s = s + p[j] * qkv[j * D * 3 + 2 * D + h * 64 + f];
                    o[f] = s;
                }
                if (probabilities) std::memcpy(probabilities + (h * T + i) * T, p.data(), T * sizeof(float));
            }
        }
    }
}

void orc_bilinear_align_true(const float* input, uint32_t iw, uint32_t ih, uint32_t ow,
                             uint32_t oh, uint32_t channels, float* out) {
    // bilinear_align_true.glsl:27-63
#pragma omp parallel for schedule(static) collapse(2)
    for (int64_t c = 0; c < channels; ++c) {
        for (int64_t oy = 0; oy < oh; ++oy) {
            const float sy = oh > 1 ? static_cast<float>(oy) * static_cast<float>(ih - 1) / static_cast<float>(oh - 1) : 0.0f;
            const uint32_t y0 = static_cast<uint32_t>(std::floor(sy));
            const uint32_t y1 = std::min(y0 + 1, ih - 1);
            const float fy = sy - static_cast<float>(y0);
            const float* src = input + static_cast<size_t>(c) * ih * iw;
            for (uint32_t ox = 0; ox < ow; ++ox) {
                const float sx = ow > 1 ? static_cast<float>(ox) * static_cast<float>(iw - 1) / static_cast<float>(ow - 1) : 0.0f;
                const uint32_t x0 = static_cast<uint32_t>(std::floor(sx));
                const uint32_t x1 = std::min(x0 + 1, iw - 1);
                const float fx = sx - static_cast<float>(x0);
                const float top = src[y0 * iw + x0] * (1.0f - fx) + src[y0 * iw + x1] * fx;
                const float bottom = src[y1 * iw + x0] * (1.0f - fx) + src[y1 * iw + x1] * fx;
                out[(static_cast<size_t>(c) * oh + oy) * ow + ox] = top * (1.0f - fy) + bottom * fy;
            }
        }
    }
}

void orc_reduce_minmax(const float* input, uint64_t count, float* range) {
    float mn = std::numeric_limits<float>::infinity();
    float mx = -std::numeric_limits<float>::infinity();
    for (uint64_t i = 0; i < count; ++i) {
        mn = std::min(mn, input[i]);
        mx = std::max(mx, input[i]);
    }
    range[0] = mn;
    range[1] = mx;
}

void orc_normalize_relative(float* depth, const float* range, uint64_t count) {
    const float minimum = range[0];
    const float span = range[1] - minimum;
    for (uint64_t i = 0; i < count; ++i)
        depth[i] = span > 1.0e-12f ? std::min(std::max((depth[i] - minimum) / span, 0.0f), 1.0f) : 0.0f;
}

int orc_network_shape(int width, int height, int input_size, int* out_width, int* out_height) {
    // image.cpp:138-161: scale the shorter side up to input_size, round each
    // side to a multiple of 14 with ties to even (numpy.round), keep at least
    // input_size, then round up to a multiple of 14.
    if (width <= 0 || height <= 0 || input_size <= 0) return 1;
    const double scale = std::max(static_cast<double>(input_size) / height, static_cast<double>(input_size) / width);
    auto to14 = [](double v) { return static_cast<int>(std::nearbyint(v / 14)) * 14; };
    int h = std::max(to14(scale * height), input_size);
    int w = std::max(to14(scale * width), input_size);
    h = (h + 13) / 14 * 14;
    w = (w + 13) / 14 * 14;
    *out_width = w;
    *out_height = h;
    return 0;
}

namespace {
// image.cpp:20-39: OpenCV's interpolateCubic (A = -0.75) in float32, in the
// shader-independent order written there; c[3] closes the partition of unity.
void opencv_cubic(float x, float c[4]) {
    const float a = -0.75f;
    const float x1 = x + 1.0f, o = 1.0f - x;
    c[0] = ((a * x1 - 5.0f * a) * x1 + 8.0f * a) * x1 - 4.0f * a;
    c[1] = ((a + 2.0f) * x - (a + 3.0f)) * x * x + 1.0f;
    c[2] = ((a + 2.0f) * o - (a + 3.0f)) * o * o + 1.0f;
    c[3] = 1.0f - c[0] - c[1] - c[2];
}

// Source sample position of destination index d (half-pixel centres,
// image.cpp:187-196 / :238-241): float32 coordinate, floor index, weights.
void cubic_tap(int d, double scale, int* base, float c[4]) {
    const float coord = static_cast<float>((d + 0.5) * scale - 0.5);
    *base = static_cast<int>(std::floor(coord));
    opencv_cubic(coord - static_cast<float>(*base), c);
}
}  // namespace

void orc_preprocess_bgr8(const uint8_t* bgr, int width, int height, int64_t stride, int dst_width, int dst_height,
                         float* out) {
    // image.cpp:163-270. Horizontal pass per source row into float64
    // [height][dst_width][3] (RGB order; tap sum from 0.0 in tap order), then
    // the vertical pass ((h0 b0 + h1 b1) + h2 b2) + h3 b3 and
    // float((v - mean) / std) in float64. Taps clamp to the image edge.
    const double sx = static_cast<double>(width) / dst_width, sy = static_cast<double>(height) / dst_height;
    std::vector<double> rows(static_cast<size_t>(height) * dst_width * 3);
    const double mean[3] = {0.485, 0.456, 0.406}, stddev[3] = {0.229, 0.224, 0.225};
#pragma omp parallel for schedule(static)
    for (int64_t y = 0; y < height; ++y) {
        const uint8_t* src = bgr + y * stride;
        for (int dx = 0; dx < dst_width; ++dx) {
            int base;
            float c[4];
            cubic_tap(dx, sx, &base, c);
            for (int ch = 0; ch < 3; ++ch) {
                double acc = 0.0;
                for (int t = 0; t < 4; ++t) {
                    const int x = std::min(std::max(base - 1 + t, 0), width - 1);
                    acc += static_cast<double>(src[3 * x + (2 - ch)]) / 255.0 * c[t];
                }
                rows[(static_cast<size_t>(y) * dst_width + dx) * 3 + ch] = acc;
            }
        }
    }
    const size_t plane = static_cast<size_t>(dst_width) * dst_height;
#pragma omp parallel for schedule(static)
    for (int64_t dy = 0; dy < dst_height; ++dy) {
        int base;
        float c[4];
        cubic_tap(static_cast<int>(dy), sy, &base, c);
        int ys[4];
        for (int t = 0; t < 4; ++t) ys[t] = std::min(std::max(base - 1 + t, 0), height - 1);
        for (int dx = 0; dx < dst_width; ++dx)
            for (int ch = 0; ch < 3; ++ch) {
                auto h = [&](int t) { return rows[(static_cast<size_t>(ys[t]) * dst_width + dx) * 3 + ch]; };
                const double v = h(0) * c[0] + h(1) * c[1] + h(2) * c[2] + h(3) * c[3];
                out[ch * plane + static_cast<size_t>(dy) * dst_width + dx] =
                    static_cast<float>((v - mean[ch]) / stddev[ch]);
            }
    }
}

void orc_preprocess_bgra8_nearest(const uint8_t* bgra, int width, int height, int64_t stride, int dst_width,
                                  int dst_height, float* out) {
    // image.cpp:289-339: float32 scale, floor(d * scale) clamped to the
    // last pixel, byte c of the pixel is model channel c (B, G, R).
    const float sx = static_cast<float>(width) / dst_width, sy = static_cast<float>(height) / dst_height;
    const float mean[3] = {0.485f, 0.456f, 0.406f}, stddev[3] = {0.229f, 0.224f, 0.225f};
    const size_t plane = static_cast<size_t>(dst_width) * dst_height;
    for (int dy = 0; dy < dst_height; ++dy) {
        const int y = std::min(static_cast<int>(std::floor(dy * sy)), height - 1);
        for (int dx = 0; dx < dst_width; ++dx) {
            const int x = std::min(static_cast<int>(std::floor(dx * sx)), width - 1);
            const uint8_t* px = bgra + y * stride + 4 * static_cast<int64_t>(x);
            for (int ch = 0; ch < 3; ++ch)
                out[ch * plane + static_cast<size_t>(dy) * dst_width + dx] =
                    (static_cast<float>(px[ch]) / 255.0f - mean[ch]) / stddev[ch];
        }
    }
}

namespace {
// preprocess_rgba.glsl:19-35 in float32
float rgba_cubic1(float v) { return ((1.25f * v - 2.25f) * v) * v + 1.0f; }
float rgba_cubic2(float v) {
    const float a = -0.75f;
    return ((a * v - 5.0f * a) * v + 8.0f * a) * v - 4.0f * a;
}
}  // namespace

void orc_preprocess_rgba8(const uint32_t* pixels, int width, int height, int64_t stride_pixels, int dst_width,
                          int dst_height, int rgba_order, float* out) {
    // preprocess_rgba.glsl:50-101 (src/gpu_preprocess.cpp:41-104)
    const float mean[3] = {0.485f, 0.456f, 0.406f}, dev[3] = {0.229f, 0.224f, 0.225f};
    const size_t plane = static_cast<size_t>(dst_width) * dst_height;
    auto taps = [](int d, int src, int dst, int idx[4], float c[4]) {
        const float coord = (static_cast<float>(d) + 0.5f) * static_cast<float>(src) / static_cast<float>(dst) - 0.5f;
        const int base = static_cast<int>(std::floor(coord));
        const float f = coord - static_cast<float>(base);
        c[0] = rgba_cubic2(f + 1.0f);
        c[1] = rgba_cubic1(f);
        c[2] = rgba_cubic1(1.0f - f);
        c[3] = rgba_cubic2(2.0f - f);
        for (int t = 0; t < 4; ++t) idx[t] = std::min(std::max(base - 1 + t, 0), src - 1);
    };
    for (int dy = 0; dy < dst_height; ++dy) {
        int ys[4];
        float cy[4];
        taps(dy, height, dst_height, ys, cy);
        for (int dx = 0; dx < dst_width; ++dx) {
            int xs[4];
            float cx[4];
            taps(dx, width, dst_width, xs, cx);
            for (int ch = 0; ch < 3; ++ch) {
                const int shift = ch == 1 ? 8 : ((ch == 0) == (rgba_order != 0) ? 0 : 16);
                float resized = 0.0f;
                for (int t = 0; t < 4; ++t) {
                    float row = 0.0f;
                    for (int k = 0; k < 4; ++k) {
                        const uint32_t p = pixels[ys[t] * stride_pixels + xs[k]];
                        row = row + static_cast<float>((p >> shift) & 255u) / 255.0f * cx[k];
                    }
                    resized = resized + row * cy[t];
                }
                out[ch * plane + static_cast<size_t>(dy) * dst_width + dx] = (resized - mean[ch]) / dev[ch];
            }
        }
    }
}

void orc_normalize_span(const float* depth, uint64_t count, float* out) {
    // dav2.cpp:787-800 (relative models): min and max over the map.
    if (count == 0) return;
    float mn = depth[0], mx = depth[0];
    for (uint64_t i = 1; i < count; ++i) {
        mn = std::min(mn, depth[i]);
        mx = std::max(mx, depth[i]);
    }
    const float span = mx - mn;
    for (uint64_t i = 0; i < count; ++i) out[i] = span > 0.0f ? (depth[i] - mn) / span : 0.0f;
}

static inline void cubic_coeffs(float t, float c[4]) {
    // position_bicubic.glsl:39-56 (A = -0.75)
    const float a = -0.75f;
    auto cc1 = [a](float x) { return ((a + 2.0f) * x - (a + 3.0f)) * x * x + 1.0f; };
    auto cc2 = [a](float x) { return ((a * x - 5.0f * a) * x + 8.0f * a) * x - 4.0f * a; };
    c[0] = cc2(t + 1.0f);
    c[1] = cc1(t);
    c[2] = cc1(1.0f - t);
    c[3] = cc2((1.0f - t) + 1.0f);
}

static inline float cubic_interp(float x0, float x1, float x2, float x3, float t) {
    float c[4];
    cubic_coeffs(t, c);
    return x0 * c[0] + x1 * c[1] + x2 * c[2] + x3 * c[3];
}

void orc_position_bicubic(const float* position, uint32_t pw, uint32_t ph, uint32_t D,
                          float* out) {
    const bool identity = pw == 37 && ph == 37;
    const float scale_x = identity ? 1.0f : static_cast<float>(1.0 / ((static_cast<double>(pw) + 0.1) / 37.0));
    const float scale_y = identity ? 1.0f : static_cast<float>(1.0 / ((static_cast<double>(ph) + 0.1) / 37.0));
    const size_t spatial = static_cast<size_t>(pw) * ph;
#pragma omp parallel for schedule(static)
    for (int64_t d = 0; d < D; ++d) {
        for (uint32_t y = 0; y < ph; ++y) {
            for (uint32_t x = 0; x < pw; ++x) {
                const float srcx = (static_cast<float>(x) + 0.5f) * scale_x - 0.5f;
                const float srcy = (static_cast<float>(y) + 0.5f) * scale_y - 0.5f;
                const int bx = static_cast<int>(std::floor(srcx));
                const int by = static_cast<int>(std::floor(srcy));
                const float tx = srcx - static_cast<float>(bx);
                const float ty = srcy - static_cast<float>(by);
                auto fetch = [&](int xx, int yy) {
                    xx = std::min(std::max(xx, 0), 36);
                    yy = std::min(std::max(yy, 0), 36);
                    // physical strides {D, 37*D, 1, 1370*D} + offset D (skip CLS)
                    return position[static_cast<size_t>(xx) * D + static_cast<size_t>(yy) * 37 * D + d + D];
                };
                float rows[4];
                for (int k = 0; k < 4; ++k) {
                    const int yy = by - 1 + k;
                    rows[k] = cubic_interp(fetch(bx - 1, yy), fetch(bx, yy), fetch(bx + 1, yy), fetch(bx + 2, yy), tx);
                }
                out[static_cast<size_t>(d) * spatial + static_cast<size_t>(y) * pw + x] =
                    cubic_interp(rows[0], rows[1], rows[2], rows[3], ty);
            }
        }
    }
}

void orc_prepare_tokens_int8(const float* image, const int8_t* w8, const float* w_scales,
                             const float* bias, const float* class_token,
                             const float* position, uint32_t width, uint32_t height,
                             uint32_t D, float* tokens) {
    // operators.cpp:1270-1308 (int8 branch) then :1323-1405 (position)
    const uint32_t pw = width / 14, ph = height / 14, spatial = pw * ph;
    constexpr uint32_t K = 3 * 14 * 14;
    std::vector<int8_t> q(static_cast<size_t>(spatial) * K);
    std::vector<float> s(spatial);
    orc_im2col_quantize(image, width, height, 3, pw, ph, 14, 14, 0, q.data(), s.data());
    std::memcpy(tokens, class_token, D * sizeof(float));
    std::vector<int32_t> acc(static_cast<size_t>(spatial) * D);
    gemm_i8_blocked(q.data(), w8, spatial, D, K, acc.data());
    orc_linear_epilogue(acc.data(), s.data(), w_scales, bias, spatial, D, 1, spatial + 1, 0, tokens);
    std::vector<float> interp(static_cast<size_t>(spatial) * D);
    orc_position_bicubic(position, pw, ph, D, interp.data());
    // add_position.glsl:25-41
    const size_t count = static_cast<size_t>(spatial + 1) * D;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < static_cast<int64_t>(count); ++i) {
        const size_t token = static_cast<size_t>(i) / D, feature = static_cast<size_t>(i) % D;
        const float p = token == 0 ? position[feature] : interp[feature * spatial + (token - 1)];
        tokens[i] = tokens[i] + p;
    }
}

void orc_project_tokens_int8(const float* tokens, const int8_t* w8, const float* w_scales,
                             const float* bias, uint32_t width, uint32_t height, uint32_t D,
                             uint32_t C, float* out) {
    // operators.cpp:1483-1526: skip CLS, GEMM, channel-major output
    const uint32_t spatial = width * height;
    std::vector<int8_t> q(static_cast<size_t>(spatial) * D);
    std::vector<float> s(spatial);
    orc_quantize_rows(tokens, spatial, D, D, q.data(), s.data());
    std::vector<int32_t> acc(static_cast<size_t>(spatial) * C);
    gemm_i8_blocked(q.data(), w8, spatial, C, D, acc.data());
    orc_linear_epilogue(acc.data(), s.data(), w_scales, bias, spatial, C, 0, spatial, 1, out);
}

void orc_conv2d_int8(const float* input, const int8_t* w8, const float* w_scales,
                     const float* bias, uint32_t width, uint32_t height, uint32_t ic,
                     uint32_t oc, uint32_t kernel, uint32_t stride, uint32_t padding,
                     int has_bias, float* out) {
    // operators.cpp:1735-1805
    const uint32_t ow = (width + 2 * padding - kernel) / stride + 1;
    const uint32_t oh = (height + 2 * padding - kernel) / stride + 1;
    const uint32_t rows = ow * oh, K = ic * kernel * kernel;
    std::vector<int8_t> q(static_cast<size_t>(rows) * K);
    std::vector<float> s(rows);
    orc_im2col_quantize(input, width, height, ic, ow, oh, kernel, stride,
                        static_cast<int32_t>(padding), q.data(), s.data());
    std::vector<int32_t> acc(static_cast<size_t>(rows) * oc);
    gemm_i8_blocked(q.data(), w8, rows, oc, K, acc.data());
    orc_linear_epilogue(acc.data(), s.data(), w_scales, has_bias ? bias : nullptr, rows, oc, 0,
                        rows, 1, out);
}

void orc_conv_transpose_int8(const float* input, const int8_t* w8, const float* w_scales,
                             const float* bias, uint32_t width, uint32_t height,
                             uint32_t ic, uint32_t oc, uint32_t kernel, float* out) {
    // operators.cpp:1908-1976 + conv_transpose_int8.glsl:31-58
    const uint32_t rows = width * height;
    std::vector<int8_t> q(static_cast<size_t>(rows) * ic);
    std::vector<float> s(rows);
    orc_im2col_quantize(input, width, height, ic, width, height, 1, 1, 0, q.data(), s.data());
    const uint32_t wrows = kernel * kernel * oc;
    std::vector<int32_t> acc(static_cast<size_t>(rows) * wrows);
    gemm_i8_blocked(q.data(), w8, rows, wrows, ic, acc.data());
    const uint32_t ow = width * kernel, oh = height * kernel;
#pragma omp parallel for schedule(static) collapse(2)
    for (int64_t c = 0; c < oc; ++c) {
        for (int64_t oy = 0; oy < oh; ++oy) {
            for (uint32_t ox = 0; ox < ow; ++ox) {
                const uint32_t ix = ox / kernel, iy = static_cast<uint32_t>(oy) / kernel;
                const uint32_t kx = ox % kernel, ky = static_cast<uint32_t>(oy) % kernel;
                const uint32_t row = iy * width + ix;
                const uint32_t wrow = (ky * kernel + kx) * oc + static_cast<uint32_t>(c);
                out[(static_cast<size_t>(c) * oh + oy) * ow + ox] =
                    dequant(acc[static_cast<size_t>(row) * wrows + wrow], s[row], w_scales[wrow], bias[c]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// fp32 precision mode (DAV2_CREATE_FORCE_FP32): the same operators with fp32
// weights and no quantization. Each dot product is a float32 sum in k order.

namespace {
// acc[i][j] = sum_k a[i][k] * w[j][k], float32, k ascending.
void gemm_f32(const float* a, uint64_t lda, const float* w, uint32_t m, uint32_t n, uint32_t k, float* acc) {
    std::vector<float> wt(static_cast<size_t>(k) * n);
    for (uint32_t j = 0; j < n; ++j)
        for (uint32_t kk = 0; kk < k; ++kk) wt[static_cast<size_t>(kk) * n + j] = w[static_cast<size_t>(j) * k + kk];
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < static_cast<int64_t>(m); ++i) {
        float* o = acc + static_cast<size_t>(i) * n;
        std::fill(o, o + n, 0.0f);
        const float* ai = a + static_cast<size_t>(i) * lda;
        for (uint32_t kk = 0; kk < k; ++kk) {
            const float av = ai[kk];
            const float* wr = wt.data() + static_cast<size_t>(kk) * n;
            for (uint32_t j = 0; j < n; ++j) o[j] = o[j] + av * wr[j];
        }
    }
}
}  // namespace

void orc_linear_f32(const float* input, const float* weight, const float* bias, uint32_t rows, uint32_t in_cols,
                    uint32_t out_cols, int gelu, float* out) {
    // operators.cpp:882-955: out = x W^T + b, then gelu.glsl when asked
    gemm_f32(input, in_cols, weight, rows, out_cols, in_cols, out);
    const size_t count = static_cast<size_t>(rows) * out_cols;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < static_cast<int64_t>(count); ++i) {
        const float v = out[i] + (bias ? bias[static_cast<size_t>(i) % out_cols] : 0.0f);
        out[i] = gelu ? gelu_value(v) : v;
    }
}

void orc_conv2d_f32(const float* input, const float* weight, const float* bias, uint32_t width, uint32_t height,
                    uint32_t ic, uint32_t oc, uint32_t kernel, uint32_t stride, uint32_t padding, int has_bias,
                    float* out) {
    // operators.cpp:1528-1676: weight [OC][IC][k][k], CHW in and out
    const uint32_t ow = (width + 2 * padding - kernel) / stride + 1;
    const uint32_t oh = (height + 2 * padding - kernel) / stride + 1;
    const uint32_t rows = ow * oh, K = ic * kernel * kernel;
    std::vector<float> cols(static_cast<size_t>(rows) * K);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < static_cast<int64_t>(rows); ++r)
        for (uint32_t c = 0; c < K; ++c)
            cols[static_cast<size_t>(r) * K + c] = im2col_read(input, width, height, ow, kernel, stride,
                                                               static_cast<int32_t>(padding),
                                                               static_cast<uint32_t>(r), c);
    std::vector<float> acc(static_cast<size_t>(rows) * oc);
    gemm_f32(cols.data(), K, weight, rows, oc, K, acc.data());
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < static_cast<int64_t>(oc); ++o)
        for (uint32_t p = 0; p < rows; ++p)
            out[static_cast<size_t>(o) * rows + p] =
                acc[static_cast<size_t>(p) * oc + o] + (has_bias ? bias[o] : 0.0f);
}

void orc_conv_transpose_f32(const float* input, const float* weight, const float* bias, uint32_t width,
                            uint32_t height, uint32_t ic, uint32_t oc, uint32_t kernel, float* out) {
    // operators.cpp:1807-1861, stride == kernel: every output pixel has one
    // source pixel; weight [IC][OC][k][k]
    const uint32_t ow = width * kernel, oh = height * kernel;
#pragma omp parallel for schedule(static) collapse(2)
    for (int64_t o = 0; o < oc; ++o)
        for (int64_t oy = 0; oy < oh; ++oy)
            for (uint32_t ox = 0; ox < ow; ++ox) {
                const uint32_t iy = static_cast<uint32_t>(oy) / kernel, ky = static_cast<uint32_t>(oy) % kernel;
                const uint32_t ix = ox / kernel, kx = ox % kernel;
                float sum = 0.0f;
                for (uint32_t c = 0; c < ic; ++c)
                    sum = sum + input[(static_cast<size_t>(c) * height + iy) * width + ix] *
                                    weight[((static_cast<size_t>(c) * oc + o) * kernel + ky) * kernel + kx];
                out[(static_cast<size_t>(o) * oh + oy) * ow + ox] = sum + bias[o];
            }
}

void orc_project_tokens_f32(const float* tokens, const float* weight, const float* bias, uint32_t width,
                            uint32_t height, uint32_t D, uint32_t C, float* out) {
    // operators.cpp:1408-1452: skip CLS, channel-major output
    const uint32_t spatial = width * height;
    std::vector<float> acc(static_cast<size_t>(spatial) * C);
    gemm_f32(tokens + D, D, weight, spatial, C, D, acc.data());
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < static_cast<int64_t>(C); ++c)
        for (uint32_t p = 0; p < spatial; ++p)
            out[static_cast<size_t>(c) * spatial + p] = acc[static_cast<size_t>(p) * C + c] + bias[c];
}

void orc_prepare_tokens_f32(const float* image, const float* weight, const float* bias, const float* class_token,
                            const float* position, uint32_t width, uint32_t height, uint32_t D, float* tokens) {
    // operators.cpp:1211-1406 (fp32 branch): patch conv (k = s = 14) into
    // rows 1.., the class token in row 0, then the position embedding
    const uint32_t pw = width / 14, ph = height / 14, spatial = pw * ph;
    std::vector<float> patches(static_cast<size_t>(D) * spatial);
    orc_conv2d_f32(image, weight, bias, width, height, 3, D, 14, 14, 0, 1, patches.data());
    std::memcpy(tokens, class_token, D * sizeof(float));
    for (uint32_t p = 0; p < spatial; ++p)
        for (uint32_t d = 0; d < D; ++d)
            tokens[static_cast<size_t>(p + 1) * D + d] = patches[static_cast<size_t>(d) * spatial + p];
    std::vector<float> interp(static_cast<size_t>(spatial) * D);
    orc_position_bicubic(position, pw, ph, D, interp.data());
    const size_t count = static_cast<size_t>(spatial + 1) * D;
    for (size_t i = 0; i < count; ++i) {
        const size_t token = i / D, feature = i % D;
        const float p = token == 0 ? position[feature] : interp[feature * spatial + (token - 1)];
        tokens[i] = tokens[i] + p;
    }
}

// ---------------------------------------------------------------------------
// fp16 precision mode (DAV2_CREATE_FORCE_FP16). Weights are the reference's
// half buffers: every use_half_weight tensor rounded to binary16
// (gpu_model.cpp:51-98, round to nearest even; f2h is that conversion).
// Two kinds of arithmetic, as in the reference:
// - cooperative-matrix linears (linear_coop_fp16.glsl, reached through
//   linear_fp16* when the device has fp16 cooperative matrices,
//   operators.cpp:540-768): operands rounded to binary16, exact products,
//   fp32 sums (here in k order; a matrix unit's order is its own);
// - native binary16 shaders (prepare_tokens_fp16.glsl:37-52,
//   project_tokens_common.glsl and conv_transpose_nonoverlap_common.glsl
//   with NATIVE_FP16): sum += float(x16 * w16) in k order, every product a
//   binary16 multiplication.

namespace {
// fp16(h(a) * h(b)) widened: the product of two binary16 values is exact in
// fp32, so rounding it once gives the binary16 multiplication.
inline float half_product(float a, float b) { return round_half(round_half(a) * round_half(b)); }

std::vector<float> rounded_half(const float* v, size_t count) {
    std::vector<float> out(count);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < static_cast<int64_t>(count); ++i) out[i] = round_half(v[i]);
    return out;
}
}  // namespace

void orc_gemm_h16_products(const float* a, uint64_t lda, const float* b, uint64_t ldb, uint32_t m, uint32_t n,
                           uint32_t k, float* out) {
    // out[i][j] = sum over kk ascending of float(h(a[i][kk]) * h(b[j][kk])), fp32
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < static_cast<int64_t>(m); ++i)
        for (uint32_t j = 0; j < n; ++j) {
            const float* ai = a + static_cast<size_t>(i) * lda;
            const float* bj = b + static_cast<size_t>(j) * ldb;
            float sum = 0.0f;
            for (uint32_t kk = 0; kk < k; ++kk) sum = sum + half_product(ai[kk], bj[kk]);
            out[static_cast<size_t>(i) * n + j] = sum;
        }
}

void orc_linear_f16(const float* input, const float* weight, const float* bias, uint32_t rows, uint32_t in_cols,
                    uint32_t out_cols, int gelu, int half_output, float* out) {
    // linear_coop_common.glsl: coopMatMulAdd of binary16 tiles into fp32,
    // + bias, exact_gelu when fused, float16_t output with HALF_OUTPUT
    const std::vector<float> x = rounded_half(input, static_cast<size_t>(rows) * in_cols);
    const std::vector<float> w = rounded_half(weight, static_cast<size_t>(out_cols) * in_cols);
    gemm_f32(x.data(), in_cols, w.data(), rows, out_cols, in_cols, out);
    const size_t count = static_cast<size_t>(rows) * out_cols;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < static_cast<int64_t>(count); ++i) {
        float v = out[i] + (bias ? bias[static_cast<size_t>(i) % out_cols] : 0.0f);
        if (gelu) v = gelu_value(v);
        out[i] = half_output ? round_half(v) : v;
    }
}

void orc_project_tokens_f16(const float* tokens, const float* weight, const float* bias, uint32_t width,
                            uint32_t height, uint32_t D, uint32_t C, float* out) {
    // project_tokens_common.glsl (NATIVE_FP16), operators.cpp:1453-1481: CLS
    // skipped, channel-major output, sums + bias
    const uint32_t spatial = width * height;
    std::vector<float> acc(static_cast<size_t>(spatial) * C);
    orc_gemm_h16_products(tokens + D, D, weight, D, spatial, C, D, acc.data());
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < static_cast<int64_t>(C); ++c)
        for (uint32_t p = 0; p < spatial; ++p)
            out[static_cast<size_t>(c) * spatial + p] = acc[static_cast<size_t>(p) * C + c] + bias[c];
}

void orc_conv_transpose_f16(const float* input, const float* weight, const float* bias, uint32_t width,
                            uint32_t height, uint32_t ic, uint32_t oc, uint32_t kernel, float* out) {
    // conv_transpose_nonoverlap_common.glsl (NATIVE_FP16), operators.cpp:1862-1906:
    // weight [IC][OC][k][k], one source pixel per output pixel, sum over the
    // input channels in order, + bias
    const uint32_t ow = width * kernel, oh = height * kernel;
#pragma omp parallel for schedule(static) collapse(2)
    for (int64_t o = 0; o < oc; ++o)
        for (int64_t oy = 0; oy < oh; ++oy)
            for (uint32_t ox = 0; ox < ow; ++ox) {
                const uint32_t iy = static_cast<uint32_t>(oy) / kernel, ky = static_cast<uint32_t>(oy) % kernel;
                const uint32_t ix = ox / kernel, kx = ox % kernel;
                float sum = 0.0f;
                for (uint32_t c = 0; c < ic; ++c)
                    sum = sum + half_product(input[(static_cast<size_t>(c) * height + iy) * width + ix],
                                             weight[((static_cast<size_t>(c) * oc + o) * kernel + ky) * kernel + kx]);
                out[(static_cast<size_t>(o) * oh + oy) * ow + ox] = sum + bias[o];
            }
}

void orc_prepare_tokens_f16(const float* image, const float* weight, const float* bias, const float* class_token,
                            const float* position, uint32_t width, uint32_t height, uint32_t D, float* tokens) {
    // prepare_tokens_fp16.glsl:37-52 (sum over channel, ky, kx of binary16
    // products, + bias; the class token in row 0), then the position
    // embedding as in the other precisions (operators.cpp:1322-1405)
    const uint32_t pw = width / 14, ph = height / 14, spatial = pw * ph;
    constexpr uint32_t K = 3 * 14 * 14;
    std::vector<float> cols(static_cast<size_t>(spatial) * K);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < static_cast<int64_t>(spatial); ++r)
        for (uint32_t c = 0; c < K; ++c)
            cols[static_cast<size_t>(r) * K + c] =
                im2col_read(image, width, height, pw, 14, 14, 0, static_cast<uint32_t>(r), c);
    std::vector<float> acc(static_cast<size_t>(spatial) * D);
    orc_gemm_h16_products(cols.data(), K, weight, K, spatial, D, K, acc.data());
    std::memcpy(tokens, class_token, D * sizeof(float));
    for (uint32_t p = 0; p < spatial; ++p)
        for (uint32_t d = 0; d < D; ++d)
            tokens[static_cast<size_t>(p + 1) * D + d] = acc[static_cast<size_t>(p) * D + d] + bias[d];
    std::vector<float> interp(static_cast<size_t>(spatial) * D);
    orc_position_bicubic(position, pw, ph, D, interp.data());
    const size_t count = static_cast<size_t>(spatial + 1) * D;
    for (size_t i = 0; i < count; ++i) {
        const size_t token = i / D, feature = i % D;
        const float p = token == 0 ? position[feature] : interp[feature * spatial + (token - 1)];
        tokens[i] = tokens[i] + p;
    }
}

// ---------------------------------------------------------------------------
// Model

static bool use_int8_weight(const std::string& name, const Tensor& t) {
    // gpu_model.cpp:16-44
    const std::string suffix = ".weight";
    if (name.size() < suffix.size() || name.compare(name.size() - suffix.size(), suffix.size(), suffix) != 0) return false;
    bool half = false;
    if (name == "pretrained.patch_embed.proj.weight" || name.rfind("depth_head.", 0) == 0) half = true;
    else if (name.rfind("pretrained.blocks.", 0) == 0)
        half = name.find(".attn.") != std::string::npos || name.find(".mlp.") != std::string::npos;
    if (!half || t.dims[0] == 0) return false;
    uint64_t elements = 1;
    for (uint32_t i = 0; i < t.rank; ++i) elements *= t.dims[i];
    if (t.rank == 2) return t.dims[1] % 4 == 0;
    if (t.rank != 4) return false;
    if (name == "depth_head.resize_layers.0.weight" || name == "depth_head.resize_layers.1.weight")
        return t.dims[0] % 4 == 0;
    return (elements / t.dims[0]) % 4 == 0;
}

orc_model* orc_model_load(const char* path, int encoder, char* error, size_t error_bytes) {
    auto fail = [&](const std::string& msg) -> orc_model* {
        if (error && error_bytes) std::snprintf(error, error_bytes, "%s", msg.c_str());
        return nullptr;
    };
    std::ifstream file(path, std::ios::binary);
    if (!file) return fail("cannot open model");
    std::vector<char> bytes((std::istreambuf_iterator<char>(file)), std::istreambuf_iterator<char>());
    if (bytes.size() < sizeof(Header)) return fail("truncated");
    Header h;
    std::memcpy(&h, bytes.data(), sizeof(h));
    if (std::memcmp(h.magic, "DAV2MOD\0", 8) != 0 || h.version != 1 || h.endian != 0x01020304u)
        return fail("bad header");
    if (h.encoder != static_cast<uint32_t>(encoder)) return fail("encoder mismatch");
    auto model = std::make_unique<orc_model>();
    model->encoder = encoder;
    switch (encoder) {
        case 0: model->dim = 384; model->heads = 6; model->blocks = 12; model->features = 64;
            model->capture[0] = 2; model->capture[1] = 5; model->capture[2] = 8; model->capture[3] = 11;
            model->project[0] = 48; model->project[1] = 96; model->project[2] = 192; model->project[3] = 384; break;
        case 1: model->dim = 768; model->heads = 12; model->blocks = 12; model->features = 128;
            model->capture[0] = 2; model->capture[1] = 5; model->capture[2] = 8; model->capture[3] = 11;
            model->project[0] = 96; model->project[1] = 192; model->project[2] = 384; model->project[3] = 768; break;
        case 2: model->dim = 1024; model->heads = 16; model->blocks = 24; model->features = 256;
            model->capture[0] = 4; model->capture[1] = 11; model->capture[2] = 17; model->capture[3] = 23;
            model->project[0] = 256; model->project[1] = 512; model->project[2] = 1024; model->project[3] = 1024; break;
        default: return fail("bad encoder");
    }
    if (h.directory_offset + static_cast<uint64_t>(h.tensor_count) * sizeof(Record) > bytes.size())
        return fail("bad directory");
    for (uint32_t i = 0; i < h.tensor_count; ++i) {
        Record r;
        std::memcpy(&r, bytes.data() + h.directory_offset + static_cast<size_t>(i) * sizeof(Record), sizeof(r));
        if (r.data_offset + r.data_bytes > bytes.size() || r.element_count * 4 != r.data_bytes)
            return fail("bad record");
        Tensor t;
        t.rank = r.rank;
        for (int d = 0; d < 4; ++d) t.dims[d] = r.dims[d];
        t.data.resize(r.element_count);
        std::memcpy(t.data.data(), bytes.data() + r.data_offset, r.data_bytes);
        if (crc32_impl(t.data.data(), r.data_bytes) != r.crc32) return fail("crc mismatch");
        const std::string name(r.name, strnlen(r.name, sizeof(r.name)));
        if (use_int8_weight(name, t)) {
            const bool convT = name == "depth_head.resize_layers.0.weight" || name == "depth_head.resize_layers.1.weight";
            if (convT) {
                const uint32_t ic = static_cast<uint32_t>(t.dims[0]), oc = static_cast<uint32_t>(t.dims[1]);
                const uint32_t k = static_cast<uint32_t>(t.dims[2]);
                t.q.resize(static_cast<size_t>(k) * k * oc * ic);
                t.qscale.resize(static_cast<size_t>(k) * k * oc);
                orc_quantize_convT_weight(t.data.data(), ic, oc, k, t.q.data(), t.qscale.data());
            } else {
                const uint64_t rows = t.dims[0], cols = r.element_count / rows;
                t.q.resize(r.element_count);
                t.qscale.resize(rows);
                orc_quantize_weight_rows(t.data.data(), rows, cols, t.q.data(), t.qscale.data());
            }
        }
        model->tensors.emplace(name, std::move(t));
    }
    return model.release();
}

void orc_model_free(orc_model* model) { delete model; }

namespace {

struct Map {
    std::vector<float> v;
    uint32_t w = 0, h = 0, c = 0;
};

std::string blk(uint32_t b, const char* s) { return "pretrained.blocks." + std::to_string(b) + s; }

void encoder_block(const orc_model& m, std::vector<float>& cur, uint32_t T, uint32_t b, int attention_mode) {
    const uint32_t D = m.dim;
    const size_t n = static_cast<size_t>(T) * D;
    std::vector<float> norm(n), qkv(n * 3), attn(n), tmp(n), next(n), hidden(n * 4);
    auto lin = [&](const std::vector<float>& in, const std::string& w, const std::string& bias,
                   uint32_t ic, uint32_t oc, bool gelu, std::vector<float>& out) {
        const Tensor& wt = m.t(w);
        if (m.fp16)
            // encoder.cpp:428-546: layer_norm_fp16 / pack_fp16 inputs (the
            // rounding is the operand rounding), fc1 with a half output
            orc_linear_f16(in.data(), wt.data.data(), m.t(bias).data.data(), T, ic, oc, gelu, gelu ? 1 : 0,
                           out.data());
        else if (m.fp32)
            orc_linear_f32(in.data(), wt.data.data(), m.t(bias).data.data(), T, ic, oc, gelu, out.data());
        else
            orc_linear_int8(in.data(), wt.q.data(), wt.qscale.data(), m.t(bias).data.data(), T, ic, oc, gelu,
                            out.data());
    };
    orc_layer_norm(cur.data(), m.t(blk(b, ".norm1.weight")).data.data(), m.t(blk(b, ".norm1.bias")).data.data(),
                   T, D, 1.0e-6f, norm.data());
    lin(norm, blk(b, ".attn.qkv.weight"), blk(b, ".attn.qkv.bias"), D, 3 * D, false, qkv);
    // attention_mode as orc_attention_head64: 0 fp32 scores, 1 the reference's
    // binary16 pipeline, 2 integer-exact (this build's int8-mode default), 3
    // the binary16 pipeline with cooperative-matrix scores
    orc_attention_head64(qkv.data(), T, m.heads, attention_mode, attn.data(), nullptr);
    lin(attn, blk(b, ".attn.proj.weight"), blk(b, ".attn.proj.bias"), D, D, false, tmp);
    orc_add_scaled(cur.data(), tmp.data(), m.t(blk(b, ".ls1.gamma")).data.data(), n, D, next.data());
    cur.swap(next);
    orc_layer_norm(cur.data(), m.t(blk(b, ".norm2.weight")).data.data(), m.t(blk(b, ".norm2.bias")).data.data(),
                   T, D, 1.0e-6f, norm.data());
    lin(norm, blk(b, ".mlp.fc1.weight"), blk(b, ".mlp.fc1.bias"), D, 4 * D, true, hidden);
    lin(hidden, blk(b, ".mlp.fc2.weight"), blk(b, ".mlp.fc2.bias"), 4 * D, D, false, tmp);
    orc_add_scaled(cur.data(), tmp.data(), m.t(blk(b, ".ls2.gamma")).data.data(), n, D, next.data());
    cur.swap(next);
}

Map conv(const orc_model& m, const Map& in, const std::string& w, const std::string& b,
         uint32_t oc, uint32_t k, uint32_t stride, uint32_t pad, bool has_bias) {
    // dpt.cpp:479-535 with every conv routed to conv2d_int8
    Map out;
    out.w = (in.w + 2 * pad - k) / stride + 1;
    out.h = (in.h + 2 * pad - k) / stride + 1;
    out.c = oc;
    out.v.resize(static_cast<size_t>(out.w) * out.h * oc);
    const Tensor& wt = m.t(w);
    if (m.fp32) {
        orc_conv2d_f32(in.v.data(), wt.data.data(), has_bias ? m.t(b).data.data() : nullptr, in.w, in.h, in.c, oc, k,
                       stride, pad, has_bias ? 1 : 0, out.v.data());
        return out;
    }
    if (m.fp16) {
        // dpt.cpp:507-517, the conv2d route with the half weights: fp32
        // input, products and sums (conv2d_common.glsl without NATIVE_FP16)
        const std::vector<float> w16 = rounded_half(wt.data.data(), wt.data.size());
        orc_conv2d_f32(in.v.data(), w16.data(), has_bias ? m.t(b).data.data() : nullptr, in.w, in.h, in.c, oc, k,
                       stride, pad, has_bias ? 1 : 0, out.v.data());
        return out;
    }
    if (wt.q.empty()) throw std::runtime_error("oracle: conv weight not int8: " + w);
    orc_conv2d_int8(in.v.data(), wt.q.data(), wt.qscale.data(), has_bias ? m.t(b).data.data() : nullptr,
                    in.w, in.h, in.c, oc, k, stride, pad, has_bias ? 1 : 0, out.v.data());
    return out;
}

Map residual_unit(const orc_model& m, const Map& in, const std::string& prefix) {
    // dpt.cpp:537-572
    Map act = in;
    orc_relu(in.v.data(), in.v.size(), act.v.data());
    Map first = conv(m, act, prefix + ".conv1.weight", prefix + ".conv1.bias", in.c, 3, 1, 1, true);
    orc_relu(first.v.data(), first.v.size(), first.v.data());
    Map second = conv(m, first, prefix + ".conv2.weight", prefix + ".conv2.bias", in.c, 3, 1, 1, true);
    orc_add(second.v.data(), in.v.data(), second.v.size(), second.v.data());
    return second;
}

Map fusion(const orc_model& m, Map path, const Map* skip, const std::string& prefix, uint32_t ow, uint32_t oh) {
    // dpt.cpp:574-615
    if (skip) {
        Map processed = residual_unit(m, *skip, prefix + ".resConfUnit1");
        orc_add(path.v.data(), processed.v.data(), path.v.size(), path.v.data());
    }
    path = residual_unit(m, path, prefix + ".resConfUnit2");
    Map resized;
    resized.w = ow; resized.h = oh; resized.c = m.features;
    resized.v.resize(static_cast<size_t>(ow) * oh * m.features);
    orc_bilinear_align_true(path.v.data(), path.w, path.h, ow, oh, m.features, resized.v.data());
    return conv(m, resized, prefix + ".out_conv.weight", prefix + ".out_conv.bias", m.features, 1, 1, 0, true);
}

}  // namespace

int orc_model_encoder_blocks(orc_model* model, float* tokens, uint32_t T, uint32_t first,
                             uint32_t last, int attention_mode) {
    try {
        std::vector<float> cur(tokens, tokens + static_cast<size_t>(T) * model->dim);
        for (uint32_t b = first; b < last && b < model->blocks; ++b) encoder_block(*model, cur, T, b, attention_mode);
        std::memcpy(tokens, cur.data(), cur.size() * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "oracle: %s\n", e.what());
        return 1;
    }
}

int orc_model_infer_fp32(orc_model* model, const float* chw, uint32_t width, uint32_t height, float* depth,
                         float* pre_relu, float* features) {
    // FORCE_FP32: fp32 weights everywhere, fp32 attention (encoder.cpp:389-396)
    model->fp32 = true;
    const int rc = orc_model_infer(model, chw, width, height, 0, depth, pre_relu, features);
    model->fp32 = false;
    return rc;
}

int orc_model_infer_fp16(orc_model* model, const float* chw, uint32_t width, uint32_t height, int attention_mode,
                         float* depth, float* pre_relu, float* features) {
    // FORCE_FP16: half weights, binary16 attention (encoder.cpp:389-403;
    // attention_mode 0 with FORCE_FP32_ATTENTION)
    model->fp16 = true;
    const int rc = orc_model_infer(model, chw, width, height, attention_mode, depth, pre_relu, features);
    model->fp16 = false;
    return rc;
}

int orc_model_infer(orc_model* model, const float* chw, uint32_t width, uint32_t height,
                    int attention_mode, float* depth, float* pre_relu, float* features) {
    try {
        const orc_model& m = *model;
        const uint32_t D = m.dim, pw = width / 14, ph = height / 14, T = pw * ph + 1;
        const size_t n = static_cast<size_t>(T) * D;
        std::vector<float> cur(n);
        const Tensor& pe = m.t("pretrained.patch_embed.proj.weight");
        if (m.fp16)
            orc_prepare_tokens_f16(chw, pe.data.data(), m.t("pretrained.patch_embed.proj.bias").data.data(),
                                   m.t("pretrained.cls_token").data.data(), m.t("pretrained.pos_embed").data.data(),
                                   width, height, D, cur.data());
        else if (m.fp32)
            orc_prepare_tokens_f32(chw, pe.data.data(), m.t("pretrained.patch_embed.proj.bias").data.data(),
                                   m.t("pretrained.cls_token").data.data(), m.t("pretrained.pos_embed").data.data(),
                                   width, height, D, cur.data());
        else
            orc_prepare_tokens_int8(chw, pe.q.data(), pe.qscale.data(),
                                    m.t("pretrained.patch_embed.proj.bias").data.data(),
                                    m.t("pretrained.cls_token").data.data(), m.t("pretrained.pos_embed").data.data(),
                                    width, height, D, cur.data());
        std::vector<std::vector<float>> feats;
        uint32_t ci = 0;
        for (uint32_t b = 0; b < m.blocks; ++b) {
            encoder_block(m, cur, T, b, attention_mode);
            if (ci < 4 && b == m.capture[ci]) {
                std::vector<float> f(n);
                orc_layer_norm(cur.data(), m.t("pretrained.norm.weight").data.data(),
                               m.t("pretrained.norm.bias").data.data(), T, D, 1.0e-6f, f.data());
                if (features) std::memcpy(features + ci * n, f.data(), n * sizeof(float));
                feats.push_back(std::move(f));
                ++ci;
            }
        }
        // dpt.cpp:635-736
        Map layers[4];
        for (uint32_t i = 0; i < 4; ++i) {
            const std::string prefix = "depth_head.projects." + std::to_string(i);
            Map proj;
            proj.w = pw; proj.h = ph; proj.c = m.project[i];
            proj.v.resize(static_cast<size_t>(pw) * ph * proj.c);
            const Tensor& wt = m.t(prefix + ".weight");
            if (m.fp16)
                orc_project_tokens_f16(feats[i].data(), wt.data.data(), m.t(prefix + ".bias").data.data(), pw, ph, D,
                                       proj.c, proj.v.data());
            else if (m.fp32)
                orc_project_tokens_f32(feats[i].data(), wt.data.data(), m.t(prefix + ".bias").data.data(), pw, ph, D,
                                       proj.c, proj.v.data());
            else
                orc_project_tokens_int8(feats[i].data(), wt.q.data(), wt.qscale.data(),
                                        m.t(prefix + ".bias").data.data(), pw, ph, D, proj.c, proj.v.data());
            if (i < 2) {
                const uint32_t k = i == 0 ? 4 : 2;
                const std::string r = "depth_head.resize_layers." + std::to_string(i);
                Map res;
                res.w = pw * k; res.h = ph * k; res.c = proj.c;
                res.v.resize(static_cast<size_t>(res.w) * res.h * res.c);
                const Tensor& rw = m.t(r + ".weight");
                if (m.fp16)
                    orc_conv_transpose_f16(proj.v.data(), rw.data.data(), m.t(r + ".bias").data.data(), pw, ph,
                                           proj.c, proj.c, k, res.v.data());
                else if (m.fp32)
                    orc_conv_transpose_f32(proj.v.data(), rw.data.data(), m.t(r + ".bias").data.data(), pw, ph,
                                           proj.c, proj.c, k, res.v.data());
                else
                    orc_conv_transpose_int8(proj.v.data(), rw.q.data(), rw.qscale.data(),
                                            m.t(r + ".bias").data.data(), pw, ph, proj.c, proj.c, k, res.v.data());
                layers[i] = std::move(res);
            } else if (i == 2) {
                layers[i] = std::move(proj);
            } else {
                layers[i] = conv(m, proj, "depth_head.resize_layers.3.weight", "depth_head.resize_layers.3.bias",
                                 m.project[3], 3, 2, 1, true);
            }
        }
        Map refined[4];
        for (uint32_t i = 0; i < 4; ++i)
            refined[i] = conv(m, layers[i], "depth_head.scratch.layer" + std::to_string(i + 1) + "_rn.weight", "",
                              m.features, 3, 1, 1, false);
        Map path = fusion(m, refined[3], nullptr, "depth_head.scratch.refinenet4", refined[2].w, refined[2].h);
        path = fusion(m, path, &refined[2], "depth_head.scratch.refinenet3", refined[1].w, refined[1].h);
        path = fusion(m, path, &refined[1], "depth_head.scratch.refinenet2", refined[0].w, refined[0].h);
        path = fusion(m, path, &refined[0], "depth_head.scratch.refinenet1", refined[0].w * 2, refined[0].h * 2);
        path = conv(m, path, "depth_head.scratch.output_conv1.weight", "depth_head.scratch.output_conv1.bias",
                    m.features / 2, 3, 1, 1, true);
        Map full;
        full.w = pw * 14; full.h = ph * 14; full.c = m.features / 2;
        full.v.resize(static_cast<size_t>(full.w) * full.h * full.c);
        orc_bilinear_align_true(path.v.data(), path.w, path.h, full.w, full.h, full.c, full.v.data());
        full = conv(m, full, "depth_head.scratch.output_conv2.0.weight", "depth_head.scratch.output_conv2.0.bias",
                    32, 3, 1, 1, true);
        orc_relu(full.v.data(), full.v.size(), full.v.data());
        Map out = conv(m, full, "depth_head.scratch.output_conv2.2.weight", "depth_head.scratch.output_conv2.2.bias",
                       1, 1, 1, 0, true);
        if (pre_relu) std::memcpy(pre_relu, out.v.data(), out.v.size() * sizeof(float));
        orc_relu(out.v.data(), out.v.size(), depth);
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "oracle: %s\n", e.what());
        return 1;
    }
}

}  // extern "C"
