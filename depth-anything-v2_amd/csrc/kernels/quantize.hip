// Per-token dynamic int8 quantization, im2col + quantization, LayerNorm and
// fused LayerNorm + quantization for gfx950.
//
// Output int8 matrices are row-major [rows][ldq] bytes with ldq a multiple of
// 64 and bytes [K, ldq) zeroed, so the MFMA GEMM can stream whole 64-byte K
// steps. The first K bytes of each row are exactly the reference's packed
// 4x int8 words (little-endian byte c%4 of word c/4 = column c).

#include <algorithm>

#include "common.h"
#include "dav2_hip.h"

using namespace dav2k;

namespace {

// Rows are handled one wave each; kRowsPerBlock waves per workgroup.
constexpr int kRowsPerBlock = 4;

// ---------------------------------------------------------------------------
// Per-row quantization, quantize_rows_int8_fused.glsl:20-55. q = rne(clamp(x / s))
// (the IEEE quotient, through quantize_div).
// WPR waves share a row (kRowsPerBlock / WPR rows per workgroup): wave part
// p owns float4 chunks p*64*CH + lane + 64j (j < CH) kept in VGPRs; the row
// maximum is the maximum of the parts' maxima (exact, order-free). EXACT:
// columns == 256 * CH * WPR (every chunk in the row). The products x * (1/s)
// come first; a lane with a value near a half-integer redoes its chunks
// with the guarded quotient (quantize_div). GELU: the row is gelu(x)
// (gelu.glsl:16-49, gelu_erfcc) of the loaded values, as if a GELU pass had
// written it first.
template <int CH, int WPR, bool EXACT, bool GELU = false>
__global__ __launch_bounds__(64 * kRowsPerBlock) void quantize_rows_kernel(
    const float* __restrict__ input, uint64_t input_offset, uint32_t rows,
    uint32_t columns, int8_t* __restrict__ q, uint32_t ldq,
    float* __restrict__ scales) {
    static_assert(kRowsPerBlock % WPR == 0, "waves per row");
    __shared__ float part_max[kRowsPerBlock];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t row = blockIdx.x * (kRowsPerBlock / WPR) + wave / WPR, part = wave % WPR;
    const bool live = row < rows;
    const float* x = input + input_offset + static_cast<uint64_t>(live ? row : 0u) * columns;
    const uint32_t words = columns >> 2, w0 = part * 64u * CH;
    float4 v[CH];
    float absmax = 0.0f;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
        const uint32_t w = w0 + lane + 64u * j;
        v[j] = live && (EXACT || w < words) ? *reinterpret_cast<const float4*>(x + 4u * w)
                                            : make_float4(0.f, 0.f, 0.f, 0.f);
        if (GELU)  // gelu(0) == 0, so the zero padding stays out of the maximum
            v[j] = make_float4(gelu_erfcc(v[j].x), gelu_erfcc(v[j].y), gelu_erfcc(v[j].z), gelu_erfcc(v[j].w));
        absmax = fmaxf(absmax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
    }
    absmax = wave_max(absmax);
    if (WPR > 1) {
        if (lane == 0) part_max[wave] = absmax;
        __syncthreads();
        const uint32_t first = wave - part;
#pragma unroll
        for (int i = 0; i < WPR; ++i) absmax = fmaxf(absmax, part_max[first + i]);
    }
    if (!live) return;
    const float s = row_scale(absmax), inv = div_rn(1.0f, s);
    if (lane == 0 && part == 0) scales[row] = s;
    uint32_t* out = reinterpret_cast<uint32_t*>(q + static_cast<uint64_t>(row) * ldq);
    int b[CH][4];
    bool near_tie = false;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
        near_tie |= quantize_product(v[j].x, inv, b[j][0]);
        near_tie |= quantize_product(v[j].y, inv, b[j][1]);
        near_tie |= quantize_product(v[j].z, inv, b[j][2]);
        near_tie |= quantize_product(v[j].w, inv, b[j][3]);
    }
    if (__builtin_expect(near_tie, 0)) {
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            b[j][0] = quantize_div(v[j].x, s, inv);
            b[j][1] = quantize_div(v[j].y, s, inv);
            b[j][2] = quantize_div(v[j].z, s, inv);
            b[j][3] = quantize_div(v[j].w, s, inv);
        }
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) {
        const uint32_t w = w0 + lane + 64u * j;
        if (EXACT || w < words) out[w] = pack4(b[j][0], b[j][1], b[j][2], b[j][3]);
    }
    if (part == 0)
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
    const float s = row_scale(absmax), inv = div_rn(1.0f, s);
    if (lane == 0) scales[row] = s;
    uint32_t* out = reinterpret_cast<uint32_t*>(q + static_cast<uint64_t>(row) * ldq);
    for (uint32_t w = lane; w < words; w += 64u) {
        const float4 v = *reinterpret_cast<const float4*>(x + 4u * w);
        out[w] = pack4(quantize_div(v.x, s, inv), quantize_div(v.y, s, inv), quantize_div(v.z, s, inv),
                       quantize_div(v.w, s, inv));
    }
    for (uint32_t w = words + lane; w < (ldq >> 2); w += 64u) out[w] = 0u;
}

// ---------------------------------------------------------------------------
// im2col + quantization, im2col_quantize_int8.glsl:26-83. Column c of output row r reads
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

// Small maps: one output pixel per WPR waves with its im2col row held in
// registers, so the window absmax, the scale and the quantized bytes come
// from one pass over the input and no channel-group maxima are needed (the
// tiled paths below are built for many output pixels). Same bytes as the
// other paths: the row absmax (of max(x, 0) with RELU), s = row_scale,
// 1 / s, rne(clamp(x * (1 / s))). Wave part p of a row owns the words
// p * 64 * kRowWords + lane + 64 j (four columns each), so a wave's stores
// cover 256 contiguous bytes. The values come through raw buffer loads,
// all issued before the first use; a column in the zero padding (or past
// the row) loads from an offset beyond the buffer, which reads 0.
constexpr int kRowWords = 9;            // words per lane and wave part
constexpr uint32_t kSmallMapRows = 8192;  // output pixels up to which this path runs

// Column c of an im2col row -> (input channel, ky, kx); KS = 3 divides by
// constants (exact for c < 2^14: c * 58255 >> 19 = c / 9, t * 11 >> 5 = t / 3
// for t < 9), KS = 0 by the geometry's reciprocals.
template <int KS>
DAV2_DEV void im2col_column(const Im2colGeometry& g, uint32_t c, uint32_t& ic, uint32_t& ky, uint32_t& kx) {
    if (KS == 3) {
        ic = __umul24(c, 58255u) >> 19;
        const uint32_t t = c - __umul24(ic, 9u);
        ky = __umul24(t, 11u) >> 5;
        kx = t - __umul24(ky, 3u);
    } else {
        ic = g.div_area.div(c);
        const uint32_t kidx = c - ic * g.div_area.d;
        ky = g.div_k.div(kidx);
        kx = kidx - ky * g.k;
    }
}

template <int WPR, bool RELU, int KS>
__global__ __launch_bounds__(256) void im2col_rows_kernel(Im2colGeometry g, uint32_t rows, uint32_t ldq,
                                                          float* __restrict__ scales, int8_t* __restrict__ q) {
    static_assert(4 % WPR == 0, "wave parts per row");
    __shared__ float part_max[4];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t row = blockIdx.x * (4u / WPR) + wave / WPR, part = wave % WPR;
    const bool live = row < rows;
    // a row past the end (whole waves) reads the last row's window, stores nothing
    const uint32_t r = min(row, rows - 1u);
    const uint32_t oy = g.div_ow.div(r), ox = r - oy * g.ow;
    const int32_t bx = static_cast<int32_t>(ox * g.stride) - g.pad, by = static_cast<int32_t>(oy * g.stride) - g.pad;
    const uint32_t plane = static_cast<uint32_t>(g.plane);
    const uint32_t words = ldq >> 2, w0 = part * 64u * kRowWords + lane;
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(g.input), static_cast<short>(0),
                                                      static_cast<int>(g.columns / (g.k * g.k) * plane * 4u),
                                                      0x00020000);
    float v[kRowWords][4];
#pragma unroll
    for (int j = 0; j < kRowWords; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t c = 4u * (w0 + 64u * j) + i;
            uint32_t ic, ky, kx;
            im2col_column<KS>(g, c, ic, ky, kx);
            const uint32_t ix = static_cast<uint32_t>(bx + static_cast<int32_t>(kx));
            const uint32_t iy = static_cast<uint32_t>(by + static_cast<int32_t>(ky));
            // (negative coordinates wrap to large unsigned values)
            const bool in = (c < g.columns) & (ix < g.iw) & (iy < g.ih);
            // small maps: every index of the input fits 24 x 24 -> 32-bit
            // products (checked by the launcher)
            const uint32_t at = (__umul24(ic, plane) + __umul24(iy, g.iw) + ix) * 4u;
            v[j][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, in ? at : 0x80000000u, 0, 0));
        }
    float absmax = 0.0f;
#pragma unroll
    for (int j = 0; j < kRowWords; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (RELU) v[j][i] = fmaxf(v[j][i], 0.0f);
            absmax = fmaxf(absmax, fabsf(v[j][i]));
        }
    absmax = wave_max(absmax);
    if (WPR > 1) {
        if (lane == 0) part_max[wave] = absmax;
        __syncthreads();
        const uint32_t first = wave - part;
#pragma unroll
        for (int i = 0; i < WPR; ++i) absmax = fmaxf(absmax, part_max[first + i]);
    }
    if (!live) return;
    const float s = row_scale(absmax);
    const float inverse = 1.0f / s;
    if (lane == 0 && part == 0) scales[row] = s;
    uint32_t* out = reinterpret_cast<uint32_t*>(q + static_cast<uint64_t>(row) * ldq);
#pragma unroll
    for (int j = 0; j < kRowWords; ++j) {
        const uint32_t w = w0 + 64u * j;
        if (w < words)
            out[w] = pack4(quantize_rne(v[j][0] * inverse), quantize_rne(v[j][1] * inverse),
                           quantize_rne(v[j][2] * inverse), quantize_rne(v[j][3] * inverse));
    }
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
// Fast im2col paths for the DPT shapes (same bytes as the generic kernels).
//
// 3x3, stride 1, pad 1 (C % 16 == 0): a workgroup owns 64 consecutive output
// pixels of one row and a range of 16-channel chunks. Pass 1 folds the
// per-channel-group |x| maxima (channel_group_absmax_kernel) of the 3 x 66
// input window; the 3x3 window maximum of that map is the im2col row's absmax
// (zero padding never raises it, and max is order-free, so the scale is
// bit-identical to the generic kernel's). Pass 2 stages each chunk's 16 x 3 x 66
// window in LDS and writes the chunk's 144 bytes of every row with consecutive
// lanes on consecutive words, i.e. one 144-byte segment per output row.
constexpr int kTile = 64;     // output pixels per workgroup
constexpr int kChunk = 16;    // input channels per chunk (16 * 9 = 144 bytes)
constexpr int kHalo = kTile + 2;

// Per-pixel maxima of |x| over channel groups of kGroupChannels:
// partial[g][p] = max over c in group g of |x[c][p]|.
// RELU: maxima of |max(x, 0)| = max(x, 0), for a map that a consumer reads
// through a ReLU.
template <bool RELU>
__global__ __launch_bounds__(256) void channel_group_absmax_kernel(const float* __restrict__ x, uint32_t C,
                                                                   uint64_t plane, float* __restrict__ partial) {
    const uint64_t p = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    if (p >= plane) return;
    const uint32_t c0 = blockIdx.y * kGroupChannels;
    const uint32_t c1 = min(C, c0 + kGroupChannels);
    const float* src = x + c0 * plane + p;
    auto mag = [](float v) { return RELU ? fmaxf(v, 0.0f) : fabsf(v); };
    if (c1 - c0 == kGroupChannels) {
        // a full group: all 32 loads in flight at once
        float v[kGroupChannels];
#pragma unroll
        for (uint32_t k = 0; k < kGroupChannels; ++k) v[k] = mag(src[k * plane]);
#pragma unroll
        for (uint32_t w = kGroupChannels / 2; w > 0; w >>= 1)
#pragma unroll
            for (uint32_t k = 0; k < w; ++k) v[k] = fmaxf(v[k], v[k + w]);
        partial[blockIdx.y * plane + p] = fmaxf(v[0], 0.0f);  // max is exact: same value as the loop below
        return;
    }
    float m0 = 0.0f, m1 = 0.0f, m2 = 0.0f, m3 = 0.0f;
    uint32_t c = c0;
    for (; c + 4 <= c1; c += 4, src += 4 * plane) {
        m0 = fmaxf(m0, mag(src[0]));
        m1 = fmaxf(m1, mag(src[plane]));
        m2 = fmaxf(m2, mag(src[2 * plane]));
        m3 = fmaxf(m3, mag(src[3 * plane]));
    }
    for (; c < c1; ++c, src += plane) m0 = fmaxf(m0, mag(src[0]));
    partial[blockIdx.y * plane + p] = fmaxf(fmaxf(m0, m1), fmaxf(m2, m3));
}

// Row scales of any im2col geometry from the channel-group maxima: the
// maximum over the k x k input positions of output pixel r (positions in the
// zero padding contribute nothing) is the absmax of im2col row r. One wave per
// row; lanes stride over the (position, group) pairs, then a wave maximum.
__global__ __launch_bounds__(64 * kRowsPerBlock) void window_scale_kernel(
    const float* __restrict__ partial, uint32_t groups, uint64_t plane, uint32_t iw, uint32_t ih, uint32_t ow,
    uint32_t rows, uint32_t k, uint32_t stride, int32_t pad, float* __restrict__ scales) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t r = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (r >= rows) return;
    const uint32_t oy = r / ow, ox = r - oy * ow;
    const uint32_t taps = k * k, total = taps * groups;
    float m = 0.0f;
    for (uint32_t e = lane; e < total; e += 64u) {
        const uint32_t g = e / taps, t = e - g * taps, ky = t / k, kx = t - ky * k;
        const int32_t iy = static_cast<int32_t>(oy * stride + ky) - pad;
        const int32_t ix = static_cast<int32_t>(ox * stride + kx) - pad;
        if (iy >= 0 && iy < static_cast<int32_t>(ih) && ix >= 0 && ix < static_cast<int32_t>(iw))
            m = fmaxf(m, partial[g * plane + static_cast<uint64_t>(iy) * iw + static_cast<uint32_t>(ix)]);
    }
    m = wave_max(m);
    if (lane == 0) scales[r] = row_scale(m);
}

// RELU: the rows are those of max(x, 0) (a ReLU ahead of the convolution).
template <bool RELU>
__global__ __launch_bounds__(256) void im2col3x3_kernel(const float* __restrict__ x, const float* __restrict__ partial,
                                                        uint32_t groups, uint32_t C, uint32_t H, uint32_t W,
                                                        uint32_t chunks_per_block, int8_t* __restrict__ q,
                                                        uint32_t ldq, float* __restrict__ scales) {
    __shared__ float amax[3 * kHalo];
    __shared__ float inv[kTile];
    __shared__ float tile[kChunk * 3 * kHalo];
    const uint32_t tid = threadIdx.x;
    const uint32_t x0 = blockIdx.x * kTile, y = blockIdx.y;
    const uint64_t plane = static_cast<uint64_t>(H) * W;

    // Pass 1: channel absmax of rows y-1..y+1, columns x0-1..x0+64, folded
    // from the per-channel-group maxima of channel_group_absmax_kernel.
    if (tid < 3 * kHalo) {
        const int r = static_cast<int>(tid) / kHalo, col = static_cast<int>(tid) % kHalo;
        const int gy = static_cast<int>(y) + r - 1, gx = static_cast<int>(x0) + col - 1;
        float m = 0.0f;
        if (gy >= 0 && gy < static_cast<int>(H) && gx >= 0 && gx < static_cast<int>(W)) {
            const float* src = partial + static_cast<uint64_t>(gy) * W + gx;
            for (uint32_t g = 0; g < groups; ++g) m = fmaxf(m, src[g * plane]);
        }
        amax[tid] = m;
    }
    __syncthreads();
    if (tid < kTile) {
        float m = 0.0f;
#pragma unroll
        for (int r = 0; r < 3; ++r)
#pragma unroll
            for (int dx = 0; dx < 3; ++dx) m = fmaxf(m, amax[r * kHalo + tid + dx]);
        const float s = row_scale(m);
        inv[tid] = 1.0f / s;
        if (blockIdx.z == 0 && x0 + tid < W) scales[static_cast<uint64_t>(y) * W + x0 + tid] = s;
    }

    const uint32_t chunks = C / kChunk;
    const uint32_t first = blockIdx.z * chunks_per_block;
    const uint32_t last = min(chunks, first + chunks_per_block);
    const uint32_t valid = min(static_cast<uint32_t>(kTile), W - x0);
    uint8_t* row_base = reinterpret_cast<uint8_t*>(q) + (static_cast<uint64_t>(y) * W + x0) * ldq;
    for (uint32_t chunk = first; chunk < last; ++chunk) {
        __syncthreads();  // previous chunk's readers are done with `tile`
        const uint32_t c0 = chunk * kChunk;
        for (uint32_t idx = tid; idx < kChunk * 3 * kHalo; idx += 256) {
            const uint32_t ch = idx / (3 * kHalo), rem = idx - ch * (3 * kHalo);
            const int r = static_cast<int>(rem) / kHalo, col = static_cast<int>(rem) % kHalo;
            const int gy = static_cast<int>(y) + r - 1, gx = static_cast<int>(x0) + col - 1;
            float v = 0.0f;
            if (gy >= 0 && gy < static_cast<int>(H) && gx >= 0 && gx < static_cast<int>(W))
                v = x[(c0 + ch) * plane + static_cast<uint64_t>(gy) * W + gx];
            tile[idx] = RELU ? fmaxf(v, 0.0f) : v;
        }
        __syncthreads();
        // 36 words (144 bytes) per pixel; word w of pixel p covers chunk
        // columns 4w..4w+3, column j -> channel j/9, tap j%9 = 3*ky + kx.
        for (uint32_t idx = tid; idx < valid * 36u; idx += 256) {
            const uint32_t p = idx / 36u, w = idx - p * 36u;
            const float sc = inv[p];
            int b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t j = 4u * w + i;
                const uint32_t ch = j / 9u, t = j - ch * 9u;
                const uint32_t ky = t / 3u, kx = t - ky * 3u;
                b[i] = quantize_rne(tile[ch * (3 * kHalo) + ky * kHalo + p + kx] * sc);
            }
            *reinterpret_cast<uint32_t*>(row_base + static_cast<uint64_t>(p) * ldq + c0 * 9u + 4u * w) =
                pack4(b[0], b[1], b[2], b[3]);
        }
    }
    // Zero the row padding [9C, ldq) once.
    if (blockIdx.z == 0) {
        const uint32_t pad_words = (ldq - 9u * C) / 4u;
        for (uint32_t idx = tid; idx < valid * pad_words; idx += 256) {
            const uint32_t p = idx / pad_words, w = idx - p * pad_words;
            *reinterpret_cast<uint32_t*>(row_base + static_cast<uint64_t>(p) * ldq + 9u * C + 4u * w) = 0u;
        }
    }
}

// 1x1 (rows = pixels, K = C): a workgroup owns 64 consecutive pixels of the
// flattened map and a range of 64-channel chunks; chunks are staged as
// [64 channels][64 pixels] (coalesced along pixels) and written back as one
// 64-byte segment per output row. Columns beyond C (the row padding) are zero.
constexpr int kChunk1 = 64;

template <bool RELU>
__global__ __launch_bounds__(256) void im2col1x1_kernel(const float* __restrict__ x, const float* __restrict__ partial,
                                                        uint32_t groups, uint32_t C, uint64_t plane,
                                                        uint32_t chunks_per_block, int8_t* __restrict__ q,
                                                        uint32_t ldq, float* __restrict__ scales) {
    __shared__ float inv[kTile];
    __shared__ float tile[kChunk1 * (kTile + 1)];
    const uint32_t tid = threadIdx.x;
    const uint64_t p0 = static_cast<uint64_t>(blockIdx.x) * kTile;
    const uint32_t valid = static_cast<uint32_t>(min<uint64_t>(kTile, plane - p0));
    if (tid < kTile) {
        float m = 0.0f;
        if (tid < valid)
            for (uint32_t g = 0; g < groups; ++g) m = fmaxf(m, partial[g * plane + p0 + tid]);
        const float s = row_scale(m);
        inv[tid] = 1.0f / s;
        if (blockIdx.y == 0 && tid < valid) scales[p0 + tid] = s;
    }
    const uint32_t chunks = ldq / kChunk1;  // covers the padding as well
    const uint32_t first = blockIdx.y * chunks_per_block;
    const uint32_t last = min(chunks, first + chunks_per_block);
    uint8_t* row_base = reinterpret_cast<uint8_t*>(q) + p0 * ldq;
    for (uint32_t chunk = first; chunk < last; ++chunk) {
        __syncthreads();
        const uint32_t c0 = chunk * kChunk1;
        for (uint32_t idx = tid; idx < kChunk1 * kTile; idx += 256) {
            const uint32_t ch = idx / kTile, p = idx - ch * kTile;
            const float v = (c0 + ch < C && p < valid) ? x[(c0 + ch) * plane + p0 + p] : 0.0f;
            tile[ch * (kTile + 1) + p] = RELU ? fmaxf(v, 0.0f) : v;
        }
        __syncthreads();
        for (uint32_t idx = tid; idx < valid * 16u; idx += 256) {
            const uint32_t p = idx / 16u, w = idx - p * 16u;
            const float sc = inv[p];
            int b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) b[i] = quantize_rne(tile[(4u * w + i) * (kTile + 1) + p] * sc);
            *reinterpret_cast<uint32_t*>(row_base + static_cast<uint64_t>(p) * ldq + c0 + 4u * w) =
                pack4(b[0], b[1], b[2], b[3]);
        }
    }
}

// ---------------------------------------------------------------------------
// LayerNorm, layer_norm.glsl:27-68. One wave per row; lane l accumulates columns
// l, l+64, ... in order and the wave reduction reproduces the 64-entry LDS
// tree, so sums, mean and variance match the reference order exactly.
// CH = ceil(columns / 64) values kept per lane (0 = re-read from memory).
// With QUANT the normalised row is also quantized (per-row rule above) into q/scales;
// out may then be null. EXACT: columns == 64 * CH, a compile-time constant
// (no partial column block, constant offsets, and for 1024 columns the
// divisions by the width become exact multiplications). For CH > 0 the
// quantized bytes go from registers to memory: with EXACT regrouped through
// LDS so that lane l stores bytes 16 l .. 16 l + 15 (one store of the whole
// row per wave), else lane l stores columns l, l + 64, ... (64-byte
// segments); CH = 0 stages the normalised row in LDS.
template <int CH, bool QUANT, bool EXACT>
__global__ __launch_bounds__(64 * kRowsPerBlock) void layer_norm_kernel(
    const float* __restrict__ input, const float* __restrict__ weight,
    const float* __restrict__ bias, uint32_t rows, uint32_t width, float epsilon,
    float* __restrict__ out, int8_t* __restrict__ q, uint32_t ldq,
    float* __restrict__ scales) {
    static_assert(!EXACT || CH > 0, "EXACT needs the row in registers");
    extern __shared__ float lds_rows[];
    __shared__ __attribute__((aligned(16))) int8_t qstage[EXACT && QUANT ? kRowsPerBlock : 1][EXACT ? 64 * CH : 16];
    const uint32_t columns = EXACT ? 64u * CH : width;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t row = blockIdx.x * kRowsPerBlock + wave;
    if (row >= rows) return;
    const float* x = input + static_cast<uint64_t>(row) * columns;
    constexpr int kKept = CH > 0 ? CH : 1;
    float v[kKept], wv[kKept], bv[kKept];
    float s = 0.0f, sq = 0.0f;
    if (CH > 0) {
        // Every load is issued unconditionally (clamped index) before the
        // first use, so the row, weight and bias arrive in one round trip;
        // columns past the row end are masked out of the sums by selects.
        const uint32_t last = columns - 1u;
        auto at = [&](int j) { return EXACT ? lane + 64u * j : min(lane + 64u * j, last); };
#pragma unroll
        for (int j = 0; j < kKept; ++j) v[j] = x[at(j)];
#pragma unroll
        for (int j = 0; j < kKept; ++j) {
            wv[j] = weight[at(j)];
            bv[j] = bias[at(j)];
        }
        // Tie the row values to the weight and bias loads so the compiler
        // cannot sink those loads below the reductions (a second memory
        // round trip): the sums below then start after all three arrived.
#pragma unroll
        for (int j = 0; j < kKept; ++j) asm volatile("" : "+v"(v[j]) : "v"(wv[j]), "v"(bv[j]));
#pragma unroll
        for (int j = 0; j < kKept; ++j) {
            const bool in = EXACT || lane + 64u * j < columns;
            s = in ? s + v[j] : s;
            sq = in ? sq + v[j] * v[j] : sq;
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
    float absmax = 0.0f;
    if (CH > 0) {
#pragma unroll
        for (int j = 0; j < kKept; ++j) {
            const uint32_t c = lane + 64u * j;
            v[j] = (v[j] - mean) * inv * wv[j] + bv[j];
            if (EXACT || c < columns) {
                if (y) y[c] = v[j];
                absmax = fmaxf(absmax, fabsf(v[j]));
            }
        }
        if (QUANT) {
            absmax = wave_max(absmax);
            const float sc = row_scale(absmax), inv_sc = div_rn(1.0f, sc);
            if (lane == 0) scales[row] = sc;
            // Product form first; a lane with any value near a half-integer
            // redoes its values with the guarded quotient (rare).
            int qv[kKept];
            bool near_tie = false;
#pragma unroll
            for (int j = 0; j < kKept; ++j) near_tie |= quantize_product(v[j], inv_sc, qv[j]);
            if (__builtin_expect(near_tie, 0)) {
#pragma unroll
                for (int j = 0; j < kKept; ++j) qv[j] = quantize_div(v[j], sc, inv_sc);
            }
            int8_t* qr = q + static_cast<uint64_t>(row) * ldq;
            if (EXACT && (reinterpret_cast<uintptr_t>(qr) & 15u) == 0) {
                int8_t* st = qstage[EXACT && QUANT ? wave : 0];
#pragma unroll
                for (int j = 0; j < kKept; ++j) st[lane + 64u * j] = static_cast<int8_t>(qv[j]);
                // this wave's bytes are in LDS before its lanes read them back
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                if (16u * lane < columns)
                    *reinterpret_cast<uint4*>(qr + 16u * lane) = *reinterpret_cast<const uint4*>(st + 16u * lane);
            } else {
#pragma unroll
                for (int j = 0; j < kKept; ++j) {
                    const uint32_t c = lane + 64u * j;
                    if (EXACT || c < columns) qr[c] = static_cast<int8_t>(qv[j]);
                }
            }
            for (uint32_t c = columns + lane; c < ldq; c += 64u) qr[c] = 0;
        }
        return;
    }
    float* stage = QUANT ? lds_rows + static_cast<size_t>(wave) * columns : nullptr;
    for (uint32_t c = lane; c < columns; c += 64u) {
        const float r = (x[c] - mean) * inv * weight[c] + bias[c];
        if (y) y[c] = r;
        if (QUANT) {
            stage[c] = r;
            absmax = fmaxf(absmax, fabsf(r));
        }
    }
    if (QUANT) {
        absmax = wave_max(absmax);
        const float sc = row_scale(absmax), inv_sc = div_rn(1.0f, sc);
        if (lane == 0) scales[row] = sc;
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        uint32_t* qo = reinterpret_cast<uint32_t*>(q + static_cast<uint64_t>(row) * ldq);
        const uint32_t words = columns >> 2;
        for (uint32_t w = lane; w < words; w += 64u) {
            const float4 t = *reinterpret_cast<const float4*>(stage + 4u * w);
            qo[w] = pack4(quantize_div(t.x, sc, inv_sc), quantize_div(t.y, sc, inv_sc),
                          quantize_div(t.z, sc, inv_sc), quantize_div(t.w, sc, inv_sc));
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
    const uint32_t ch = (cols + 63u) / 64u;
    const size_t lds = QUANT && ch > 16 ? static_cast<size_t>(kRowsPerBlock) * cols * sizeof(float) : 0;
#define DAV2_LN_CASE(N, E)                                                                   \
    dispatch((layer_norm_kernel<N, QUANT, E>), dim3(grid), dim3(64 * kRowsPerBlock), \
                       lds, stream, in, w, b, rows, cols, eps, out, q, ldq, scales)
    if (cols == 384) DAV2_LN_CASE(6, true);
    else if (cols == 768) DAV2_LN_CASE(12, true);
    else if (cols == 1024) DAV2_LN_CASE(16, true);
    else if (ch <= 6) DAV2_LN_CASE(6, false);
    else if (ch <= 12) DAV2_LN_CASE(12, false);
    else if (ch <= 16) DAV2_LN_CASE(16, false);
    else DAV2_LN_CASE(0, false);
#undef DAV2_LN_CASE
    return hipGetLastError();
}

}  // namespace

hipError_t dav2k::launch_channel_group_absmax(const float* x, uint32_t channels, uint64_t plane, float* partial,
                                              bool relu, hipStream_t stream) {
    const dim3 grid(ceil_div(plane, 256), channel_groups(channels));
    if (relu) dispatch(channel_group_absmax_kernel<true>, grid, dim3(256), 0, stream, x, channels, plane, partial);
    else dispatch(channel_group_absmax_kernel<false>, grid, dim3(256), 0, stream, x, channels, plane, partial);
    return hipGetLastError();
}

// int8 rows of `columns` bytes (the reference GpuModel layout) to rows of
// ld bytes, zero beyond columns: 16 bytes per thread, one row per y block.
__global__ __launch_bounds__(256) void pad_rows_kernel(const int8_t* __restrict__ src, uint32_t columns,
                                                       int8_t* __restrict__ dst, uint32_t ld) {
    const uint64_t row = blockIdx.y;
    const uint32_t c0 = (blockIdx.x * 256u + threadIdx.x) * 16u;
    if (c0 >= ld) return;
    const int8_t* s = src + row * columns;
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint32_t c = c0 + q * 4 + b;
            const uint32_t byte = c < columns ? static_cast<uint8_t>(s[c]) : 0u;
            word |= byte << (8 * b);
        }
        w[q] = word;
    }
    *reinterpret_cast<uint4*>(dst + row * ld + c0) = make_uint4(w[0], w[1], w[2], w[3]);
}

// int8 weights in the reference's transposed layout ([K][N] bytes, element
// (k, n) = weight of output n, input k; src/gpu_model.cpp:241-258) to the GEMM
// layout ([N][ld] bytes, zero for k >= K): 64x64 byte tiles through LDS, the
// reads coalesced along n, the writes along k.
__global__ __launch_bounds__(256) void transpose_rows_kernel(const int8_t* __restrict__ src, uint32_t k_rows,
                                                             uint32_t n_columns, int8_t* __restrict__ dst,
                                                             uint32_t ld) {
    __shared__ int8_t tile[64][65];
    const uint32_t n0 = blockIdx.x * 64u, k0 = blockIdx.y * 64u;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t idx = threadIdx.x + 256u * i, r = idx / 64u, c = idx % 64u;
        const uint32_t k = k0 + r, n = n0 + c;
        tile[r][c] = (k < k_rows && n < n_columns) ? src[uint64_t(k) * n_columns + n] : int8_t(0);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t idx = threadIdx.x + 256u * i, r = idx / 64u, c = idx % 64u;
        const uint32_t n = n0 + r;
        if (n < n_columns) dst[uint64_t(n) * ld + k0 + c] = tile[c][r];
    }
}

extern "C" {

int dav2_hip_transpose_rows_i8(const int8_t* src, uint32_t k_rows, uint32_t n_columns, int8_t* dst, uint32_t ld,
                               void* stream) {
    if (k_rows == 0 || n_columns == 0) return hipSuccess;
    if (!src || !dst || ld < k_rows || ld % 64u || ld / 64u > 65535u) return hipErrorInvalidValue;
    dispatch(transpose_rows_kernel, dim3(ceil_div(n_columns, 64u), ld / 64u), dim3(256), 0,
             static_cast<hipStream_t>(stream), src, k_rows, n_columns, dst, ld);
    return hipGetLastError();
}

int dav2_hip_pad_rows_i8(const int8_t* src, uint32_t rows, uint32_t columns, int8_t* dst, uint32_t ld,
                         void* stream) {
    if (rows == 0) return hipSuccess;
    if (!src || !dst || columns == 0 || ld < columns || ld % 16u || (reinterpret_cast<uintptr_t>(dst) & 15) ||
        rows > 65535u)
        return hipErrorInvalidValue;
    dispatch(pad_rows_kernel, dim3(ceil_div(ld, 256u * 16u), rows), dim3(256), 0,
                       static_cast<hipStream_t>(stream), src, columns, dst, ld);
    return hipGetLastError();
}

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
    // Long rows are split over several waves (more loads in flight per row).
#define DAV2_QR_CASE(N, W, E)                                                                                         \
    dispatch((quantize_rows_kernel<N, W, E>), dim3(ceil_div(rows, kRowsPerBlock / W)), dim3(64 * kRowsPerBlock), \
                       0, s, input, input_offset, rows, columns, q, ldq, scales)
    if (columns == 1024u) DAV2_QR_CASE(4, 1, true);
    else if (columns == 4096u) DAV2_QR_CASE(4, 4, true);
    else if (ch <= 1) DAV2_QR_CASE(1, 1, false);
    else if (ch <= 2) DAV2_QR_CASE(2, 1, false);
    else if (ch <= 4) DAV2_QR_CASE(4, 1, false);
    else if (ch <= 8) DAV2_QR_CASE(4, 2, false);
    else if (ch <= 16) DAV2_QR_CASE(4, 4, false);
    else
        dispatch(quantize_rows_long_kernel, dim3(grid), dim3(64 * kRowsPerBlock), 0, s,
                           input, input_offset, rows, columns, q, ldq, scales);
#undef DAV2_QR_CASE
    return hipGetLastError();
}

int dav2_hip_gelu_quantize_rows_i8(const float* input, uint64_t input_offset, uint32_t rows, uint32_t columns,
                                   int8_t* q, uint32_t ldq, float* scales, void* stream) {
    if (rows == 0) return hipSuccess;
    if (!input || !q || !scales || columns == 0 || columns % 4u || columns > 4096u || ldq < columns ||
        ldq % 64u || input_offset % 4u)
        return hipErrorInvalidValue;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint32_t ch = (columns / 4u + 63u) / 64u;
#define DAV2_QR_CASE(N, W, E)                                                                    \
    dispatch((quantize_rows_kernel<N, W, E, true>), dim3(ceil_div(rows, kRowsPerBlock / W)),     \
             dim3(64 * kRowsPerBlock), 0, s, input, input_offset, rows, columns, q, ldq, scales)
    if (columns == 4096u) DAV2_QR_CASE(4, 4, true);
    else if (ch <= 2) DAV2_QR_CASE(2, 1, false);
    else if (ch <= 4) DAV2_QR_CASE(4, 1, false);
    else if (ch <= 8) DAV2_QR_CASE(4, 2, false);
    else DAV2_QR_CASE(4, 4, false);
#undef DAV2_QR_CASE
    return hipGetLastError();
}

uint64_t dav2_hip_im2col_scratch_floats(uint32_t input_width, uint32_t input_height, uint32_t input_channels) {
    return static_cast<uint64_t>(input_width) * input_height * ((input_channels + kGroupChannels - 1) / kGroupChannels);
}

namespace {

// relu: quantize the rows of max(input, 0); the single-pass path of small
// maps and the tiled 3x3 / 1x1 paths (with scratch) take it, other calls
// return hipErrorInvalidValue.
int im2col_quantize(const float* input, uint32_t input_width, uint32_t input_height, uint32_t input_channels,
                    uint32_t output_width, uint32_t output_height, uint32_t kernel, uint32_t stride, int32_t padding,
                    int8_t* q, uint32_t ldq, float* scales, float* scratch, uint64_t scratch_floats, bool relu,
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
    const uint64_t plane = static_cast<uint64_t>(input_width) * input_height;
    const uint32_t groups = (input_channels + kGroupChannels - 1) / kGroupChannels;
    const bool fast3 = kernel == 3 && stride == 1 && padding == 1 && input_channels % kChunk == 0 &&
                       output_width == input_width && output_height == input_height;
    const bool fast1 = kernel == 1 && stride == 1 && padding == 0 && output_width == input_width &&
                       output_height == input_height;
    const bool have_partial = scratch && scratch_floats >= plane * groups;
    const uint32_t row_words = ldq / 4u;
    if (rows <= kSmallMapRows && row_words <= 4u * 64u * kRowWords && plane * input_channels < (1ull << 29) &&
        plane < (1u << 24) && input_width < (1u << 24) && input_height < (1u << 24) && input_channels < (1u << 24)) {
        const int wpr = row_words <= 64u * kRowWords ? 1 : (row_words <= 128u * kRowWords ? 2 : 4);
#define DAV2_ROWS_CASE(W, K)                                                                                 \
    do {                                                                                                     \
        const dim3 grid(ceil_div(rows, 4u / (W)));                                                           \
        if (relu) dispatch(im2col_rows_kernel<W, true, K>, grid, dim3(256), 0, s, g, rows, ldq, scales, q);  \
        else dispatch(im2col_rows_kernel<W, false, K>, grid, dim3(256), 0, s, g, rows, ldq, scales, q);      \
    } while (0)
        if (kernel == 3) {
            if (wpr == 1) DAV2_ROWS_CASE(1, 3);
            else if (wpr == 2) DAV2_ROWS_CASE(2, 3);
            else DAV2_ROWS_CASE(4, 3);
        } else {
            if (wpr == 1) DAV2_ROWS_CASE(1, 0);
            else if (wpr == 2) DAV2_ROWS_CASE(2, 0);
            else DAV2_ROWS_CASE(4, 0);
        }
#undef DAV2_ROWS_CASE
        return hipGetLastError();
    }
    if ((fast3 || fast1) && have_partial && input_height <= 65535u) {
        const hipError_t e = launch_channel_group_absmax(input, input_channels, plane, scratch, relu, s);
        if (e != hipSuccess) return e;
        // Enough workgroups to fill the chip: split the channel chunks of
        // small maps over blockIdx.z (each split recomputes the 64 scales).
        if (fast3) {
            const unsigned tiles = ceil_div(input_width, kTile) * input_height;
            const uint32_t chunks = input_channels / kChunk;
            const uint32_t splits = std::max(1u, std::min(chunks, static_cast<uint32_t>(2048u / tiles)));
            const uint32_t per = (chunks + splits - 1) / splits;
            const dim3 grid(ceil_div(input_width, kTile), input_height, ceil_div(chunks, per));
            if (relu)
                dispatch(im2col3x3_kernel<true>, grid, dim3(256), 0, s, input, scratch, groups,
                                   input_channels, input_height, input_width, per, q, ldq, scales);
            else
                dispatch(im2col3x3_kernel<false>, grid, dim3(256), 0, s, input, scratch, groups,
                                   input_channels, input_height, input_width, per, q, ldq, scales);
        } else {
            const unsigned tiles = ceil_div(plane, kTile);
            const uint32_t chunks = ldq / kChunk1;
            const uint32_t splits = std::max(1u, std::min(chunks, static_cast<uint32_t>(2048u / tiles)));
            const uint32_t per = (chunks + splits - 1) / splits;
            const dim3 grid(tiles, ceil_div(chunks, per));
            if (relu)
                dispatch(im2col1x1_kernel<true>, grid, dim3(256), 0, s, input, scratch, groups,
                                   input_channels, plane, per, q, ldq, scales);
            else
                dispatch(im2col1x1_kernel<false>, grid, dim3(256), 0, s, input, scratch, groups,
                                   input_channels, plane, per, q, ldq, scales);
        }
        return hipGetLastError();
    }
    if (relu) return hipErrorInvalidValue;
    if (have_partial) {
        // Scales from the channel-group maxima (same values, one thread per row).
        dispatch(channel_group_absmax_kernel<false>, dim3(ceil_div(plane, 256), groups), dim3(256), 0, s,
                           input, input_channels, plane, scratch);
        dispatch(window_scale_kernel, dim3(ceil_div(rows, kRowsPerBlock)), dim3(64 * kRowsPerBlock), 0, s,
                           scratch, groups, plane, input_width, input_height, output_width, rows, kernel, stride,
                           padding, scales);
    } else {
        dispatch(im2col_scale_kernel, dim3(ceil_div(rows, kRowsPerBlock)), dim3(64 * kRowsPerBlock), 0,
                           s, g, rows, scales);
    }
    const uint32_t ldq_words = ldq / 4u;
    const uint64_t total = rows64 * ldq_words;
    dispatch(im2col_quantize_kernel, dim3(ceil_div(total, 256)), dim3(256), 0, s, g, rows,
                       ldq_words, scales, q);
    return hipGetLastError();
}

}  // namespace

int dav2_hip_im2col_quantize_i8(const float* input, uint32_t input_width, uint32_t input_height,
                                uint32_t input_channels, uint32_t output_width,
                                uint32_t output_height, uint32_t kernel, uint32_t stride,
                                int32_t padding, int8_t* q, uint32_t ldq, float* scales,
                                float* scratch, uint64_t scratch_floats, void* stream) {
    return im2col_quantize(input, input_width, input_height, input_channels, output_width, output_height, kernel,
                           stride, padding, q, ldq, scales, scratch, scratch_floats, false, stream);
}

int dav2_hip_im2col_quantize_relu_i8(const float* input, uint32_t input_width, uint32_t input_height,
                                     uint32_t input_channels, uint32_t output_width, uint32_t output_height,
                                     uint32_t kernel, uint32_t stride, int32_t padding, int8_t* q, uint32_t ldq,
                                     float* scales, float* scratch, uint64_t scratch_floats, void* stream) {
    return im2col_quantize(input, input_width, input_height, input_channels, output_width, output_height, kernel,
                           stride, padding, q, ldq, scales, scratch, scratch_floats, true, stream);
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
