// Materialised head-64 fp32 attention on the matrix cores, for the fp32
// precision mode (FORCE_FP32): scores = (0.125 q) k^T on
// v_mfma_f32_16x16x4_f32, row softmax in place, out = P v on MFMA. Exact fp32
// products, fp32 accumulation in the matrix core's order, so within
// tolerance of the reference (src/operators.cpp:1169-1208, bmm.glsl,
// softmax_lastdim.glsl), not bit for bit; the reference-order kernels are in
// attention_ref.hip.
//
// Layouts: qkv [batch*T][3*H*64]; scores [batch][H][T][T].

#include "common.h"
#include "dav2_hip.h"

using namespace dav2k;

namespace {

// ---------------------------------------------------------------------------
// Scores. Workgroup tile 64 (queries) x 64 (keys), 4 waves in 2x2, each wave
// 32x32 = 2x2 MFMA blocks. Q and K tiles are staged through LDS with the
// 0.125 query scale applied first (bmm.glsl:57-63).
constexpr int kScoreStride = 65;  // padded LDS row length (floats)

__global__ __launch_bounds__(256) void attention_scores_kernel(const float* __restrict__ qkv,
                                                               float* __restrict__ scores, uint32_t tokens,
                                                               uint32_t heads) {
    constexpr int S = kScoreStride;
    __shared__ __attribute__((aligned(16))) float qt[64 * S];
    __shared__ __attribute__((aligned(16))) float kt[64 * S];

    const uint32_t bh = blockIdx.z;
    const uint32_t b = bh / heads, h = bh - b * heads;
    const uint32_t D = heads * 64u;
    const uint32_t i0 = blockIdx.y * 64u, j0 = blockIdx.x * 64u;
    const float* base = qkv + static_cast<uint64_t>(b) * tokens * 3u * D + h * 64u;
    const int tid = threadIdx.x;

    // 64 rows x 64 features = 1024 float4 loads per tile, 4 per thread.
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int c = tid + it * 256;
        const int r = c >> 4, f4 = (c & 15) * 4;
        float4 qv = make_float4(0.f, 0.f, 0.f, 0.f), kv = qv;
        if (i0 + r < tokens)
            qv = *reinterpret_cast<const float4*>(base + static_cast<uint64_t>(i0 + r) * 3u * D + f4);
        if (j0 + r < tokens)
            kv = *reinterpret_cast<const float4*>(base + static_cast<uint64_t>(j0 + r) * 3u * D + D + f4);
        float* qd = qt + r * S + f4;
        float* kd = kt + r * S + f4;
        qd[0] = qv.x * 0.125f;
        qd[1] = qv.y * 0.125f;
        qd[2] = qv.z * 0.125f;
        qd[3] = qv.w * 0.125f;
        kd[0] = kv.x;
        kd[1] = kv.y;
        kd[2] = kv.z;
        kd[3] = kv.w;
    }
    __syncthreads();

    const int lane = tid & 63, wave = tid >> 6;
    const int wr = (wave >> 1) * 32, wc = (wave & 1) * 32;
    const int fr = lane & 15, g = lane >> 4;
    v4f acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int c = 0; c < 2; ++c) acc[a][c] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) {
        float af[2], bf[2];
#pragma unroll
        for (int a = 0; a < 2; ++a) af[a] = qt[(wr + a * 16 + fr) * S + ks * 4 + g];
#pragma unroll
        for (int c = 0; c < 2; ++c) bf[c] = kt[(wc + c * 16 + fr) * S + ks * 4 + g];
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int c = 0; c < 2; ++c)
                acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[a], bf[c], acc[a][c], 0, 0, 0);
    }

    const uint64_t plane = static_cast<uint64_t>(bh) * tokens;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const uint32_t j = j0 + wc + c * 16 + fr;
            if (j >= tokens) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t i = i0 + wr + a * 16 + 4 * g + r;
                if (i < tokens) scores[(plane + i) * tokens + j] = acc[a][c][r];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Softmax over rows, in place, one wave per row, the whole row in VGPRs
// (CH values per lane; CH = 0 streams the row three times instead): max,
// e = exp(x - max), sum, e * (1 / max(sum, 1e-20)) as softmax_lastdim.glsl,
// with the lanes and the butterfly in this kernel's own order.
template <int CH>
__global__ __launch_bounds__(256) void softmax_kernel(void* data, uint64_t rows, uint32_t columns,
                                                      uint32_t row_stride) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t row = static_cast<uint64_t>(blockIdx.x) * 4u + (threadIdx.x >> 6);
    if (row >= rows) return;
    float* fr = static_cast<float*>(data) + row * row_stride;
    float v[CH > 0 ? CH : 1];
    float maximum = -3.402823466e+38f;
    if (CH > 0) {
#pragma unroll
        for (int j = 0; j < (CH > 0 ? CH : 1); ++j) {
            const uint32_t c = lane + 64u * j;
            v[j] = c < columns ? fr[c] : -3.402823466e+38f;
            maximum = fmaxf(maximum, v[j]);
        }
    } else {
        for (uint32_t c = lane; c < columns; c += 64u) maximum = fmaxf(maximum, fr[c]);
    }
    maximum = wave_max(maximum);
    float sum = 0.0f;
    if (CH > 0) {
#pragma unroll
        for (int j = 0; j < (CH > 0 ? CH : 1); ++j) {
            const uint32_t c = lane + 64u * j;
            if (c < columns) {
                const float e = expf(v[j] - maximum);
                sum = sum + e;
                v[j] = e;
            }
        }
    } else {
        for (uint32_t c = lane; c < columns; c += 64u) {
            const float e = expf(fr[c] - maximum);
            sum = sum + e;
            fr[c] = e;
        }
    }
    // Every lane holds a complete (though differently associated) sum.
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum = sum + __shfl_xor(sum, o, kWave);
    const float inverse = 1.0f / fmaxf(sum, 1.0e-20f);
    if (CH > 0) {
#pragma unroll
        for (int j = 0; j < (CH > 0 ? CH : 1); ++j) {
            const uint32_t c = lane + 64u * j;
            if (c < columns) fr[c] = v[j] * inverse;
        }
    } else {
        for (uint32_t c = lane; c < columns; c += 64u) fr[c] = fr[c] * inverse;
    }
}

// ---------------------------------------------------------------------------
// out = P v. Workgroup: 128 query rows x 64 features of one (batch, head);
// wave w owns rows 32w..32w+31 (2x4 MFMA blocks). The key axis advances 32
// tokens per step; P (128x32) and v^T (64x32) are staged through LDS.
__global__ __launch_bounds__(256) void attention_values_kernel(const float* __restrict__ probabilities,
                                                               const float* __restrict__ qkv,
                                                               float* __restrict__ out, uint32_t tokens,
                                                               uint32_t heads) {
    constexpr int PS = 33, VS = 33;  // padded LDS row lengths (floats)
    __shared__ __attribute__((aligned(16))) float pt[128 * PS];
    __shared__ __attribute__((aligned(16))) float vt[64 * VS];

    const uint32_t bh = blockIdx.z;
    const uint32_t b = bh / heads, h = bh - b * heads;
    const uint32_t D = heads * 64u;
    const uint32_t i0 = blockIdx.x * 128u;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int fr = lane & 15, g = lane >> 4;
    const float* vbase = qkv + static_cast<uint64_t>(b) * tokens * 3u * D + 2u * D + h * 64u;
    const uint64_t plane = static_cast<uint64_t>(bh) * tokens;

    v4f acc[2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[a][c] = v4f{0.f, 0.f, 0.f, 0.f};

    for (uint32_t j0 = 0; j0 < tokens; j0 += 32u) {
        // Stage v[j0..j0+32)[0..64) transposed: 2048 values, 8 per thread.
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int c = tid + it * 256;  // 512 float4 chunks
            const int jr = c >> 4, f4 = (c & 15) * 4;
            float4 vv = make_float4(0.f, 0.f, 0.f, 0.f);
            if (j0 + jr < tokens)
                vv = *reinterpret_cast<const float4*>(vbase + static_cast<uint64_t>(j0 + jr) * 3u * D + f4);
            vt[(f4 + 0) * VS + jr] = vv.x;
            vt[(f4 + 1) * VS + jr] = vv.y;
            vt[(f4 + 2) * VS + jr] = vv.z;
            vt[(f4 + 3) * VS + jr] = vv.w;
        }
        // Stage P[i0..i0+128)[j0..j0+32): 4096 values, 16 per thread.
#pragma unroll
        for (int it = 0; it < 16; ++it) {
            const int c = tid + it * 256;
            const int ir = c >> 5, jc = c & 31;
            const uint32_t i = i0 + ir, j = j0 + jc;
            pt[ir * PS + jc] = i < tokens && j < tokens ? probabilities[(plane + i) * tokens + j] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            float af[2], bf[4];
#pragma unroll
            for (int a = 0; a < 2; ++a) af[a] = pt[(wave * 32 + a * 16 + fr) * PS + ks * 4 + g];
#pragma unroll
            for (int c = 0; c < 4; ++c) bf[c] = vt[(c * 16 + fr) * VS + ks * 4 + g];
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[a], bf[c], acc[a][c], 0, 0, 0);
        }
        __syncthreads();
    }

#pragma unroll
    for (int a = 0; a < 2; ++a) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t i = i0 + wave * 32 + a * 16 + 4 * g + r;
            if (i >= tokens) continue;
            float* o = out + (static_cast<uint64_t>(b) * tokens + i) * D + h * 64u;
#pragma unroll
            for (int c = 0; c < 4; ++c) o[c * 16 + fr] = acc[a][c][r];
        }
    }
}

void launch_softmax(void* data, uint64_t rows, uint32_t columns, uint32_t stride, hipStream_t s) {
    const unsigned grid = ceil_div(rows, 4);
    const uint32_t ch = (columns + 63u) / 64u;
#define DAV2_SM_CASE(N) \
    dispatch((softmax_kernel<N>), dim3(grid), dim3(256), 0, s, data, rows, columns, stride)
    if (ch <= 4) DAV2_SM_CASE(4);
    else if (ch <= 8) DAV2_SM_CASE(8);
    else if (ch <= 16) DAV2_SM_CASE(16);
    else if (ch <= 24) DAV2_SM_CASE(24);
    else if (ch <= 32) DAV2_SM_CASE(32);
    else if (ch <= 48) DAV2_SM_CASE(48);
    else if (ch <= 64) DAV2_SM_CASE(64);
    else if (ch <= 96) DAV2_SM_CASE(96);
    else DAV2_SM_CASE(0);
#undef DAV2_SM_CASE
}

}  // namespace

extern "C" {

// fp16 != 0 is rejected: binary16 attention is dav2_hip_attention_ref_*.
int dav2_hip_attention_scores(void* scores, const float* qkv, uint32_t tokens, uint32_t heads,
                              uint32_t batch, int fp16, void* stream) {
    if (fp16) return hipErrorInvalidValue;
    if (tokens == 0 || heads == 0 || batch == 0) return hipSuccess;
    if (!scores || !qkv || (reinterpret_cast<uintptr_t>(qkv) & 15) || heads > 65535u / batch)
        return hipErrorInvalidValue;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid(ceil_div(tokens, 64), ceil_div(tokens, 64), heads * batch);
    dispatch(attention_scores_kernel, grid, dim3(256), 0, s, qkv, static_cast<float*>(scores), tokens,
                       heads);
    return hipGetLastError();
}

int dav2_hip_softmax_rows(void* scores, uint64_t rows, uint32_t columns, uint32_t row_stride, int fp16,
                          void* stream) {
    if (fp16) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    if (!scores || columns == 0 || row_stride < columns) return hipErrorInvalidValue;
    launch_softmax(scores, rows, columns, row_stride, static_cast<hipStream_t>(stream));
    return hipGetLastError();
}

int dav2_hip_attention_values(float* out, const void* probabilities, const float* qkv, uint32_t tokens,
                              uint32_t heads, uint32_t batch, int fp16, void* stream) {
    if (fp16) return hipErrorInvalidValue;
    if (tokens == 0 || heads == 0 || batch == 0) return hipSuccess;
    if (!out || !probabilities || !qkv || (reinterpret_cast<uintptr_t>(qkv) & 15) || heads > 65535u / batch)
        return hipErrorInvalidValue;
    const dim3 grid(ceil_div(tokens, 128), 1, heads * batch);
    dispatch(attention_values_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const float*>(probabilities), qkv, out, tokens, heads);
    return hipGetLastError();
}

uint64_t dav2_hip_attention_scratch_bytes(uint32_t tokens, uint32_t heads, uint32_t batch, int fp16) {
    if (fp16) return 0;
    return static_cast<uint64_t>(batch) * heads * tokens * tokens * sizeof(float);
}

}  // extern "C"
