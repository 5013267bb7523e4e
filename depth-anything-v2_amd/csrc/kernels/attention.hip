// Materialised head-64 attention for gfx950: scores = (0.125 q) k^T on MFMA,
// row softmax in place, out = P v on MFMA.
//
// Reference: src/operators.cpp:1098-1209 with bmm.glsl / softmax_lastdim.glsl
// (fp32 scores) and bmm_score_fp16.glsl / softmax_lastdim_half.glsl /
// bmm_value_fp16.glsl (binary16 scores, the reference's int8-mode default).
//
// fp32 path: v_mfma_f32_16x16x4_f32 (exact fp32 products, fp32 accumulation).
// fp16 path: v_mfma_f32_16x16x32_f16 on binary16 operands (fp16(q*0.125),
// fp16(k), fp16(p), fp16(v)) with fp32 accumulation; the reference rounds each
// product to binary16 before accumulating, the matrix core does not.
//
// Layouts: qkv [batch*T][3*H*64]; fp32 scores [batch][H][T][T]; fp16 scores
// [batch][H][T][ldt] with ldt = T rounded up to a multiple of 8 (16-byte rows).

#include "common.h"
#include "dav2_hip.h"

using namespace dav2k;

namespace {

typedef float v1f;

inline uint32_t half_ld(uint32_t tokens) { return (tokens + 7u) & ~7u; }

// ---------------------------------------------------------------------------
// Scores. Workgroup tile 64 (queries) x 64 (keys), 4 waves in 2x2, each wave
// 32x32 = 2x2 MFMA blocks. Q and K tiles are staged through LDS in the
// operand type with the 0.125 query scale applied first (bmm.glsl:57-63).
template <bool HALF>
struct ScoreTile {
    using T = typename std::conditional<HALF, _Float16, float>::type;
    static constexpr int kStride = HALF ? 72 : 65;  // padded row length (elements)
};

template <bool HALF>
__global__ __launch_bounds__(256) void attention_scores_kernel(
    const float* __restrict__ qkv, void* __restrict__ scores_out, uint32_t tokens,
    uint32_t heads, uint32_t ldt) {
    using T = typename ScoreTile<HALF>::T;
    constexpr int S = ScoreTile<HALF>::kStride;
    __shared__ __attribute__((aligned(16))) T qt[64 * S];
    __shared__ __attribute__((aligned(16))) T kt[64 * S];

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
        T* qd = qt + r * S + f4;
        T* kd = kt + r * S + f4;
        qd[0] = static_cast<T>(qv.x * 0.125f);
        qd[1] = static_cast<T>(qv.y * 0.125f);
        qd[2] = static_cast<T>(qv.z * 0.125f);
        qd[3] = static_cast<T>(qv.w * 0.125f);
        kd[0] = static_cast<T>(kv.x);
        kd[1] = static_cast<T>(kv.y);
        kd[2] = static_cast<T>(kv.z);
        kd[3] = static_cast<T>(kv.w);
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

    if (HALF) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            v8h af[2], bf[2];
#pragma unroll
            for (int a = 0; a < 2; ++a)
                af[a] = *reinterpret_cast<const v8h*>(reinterpret_cast<const _Float16*>(qt) +
                                                      (wr + a * 16 + fr) * S + ks * 32 + g * 8);
#pragma unroll
            for (int c = 0; c < 2; ++c)
                bf[c] = *reinterpret_cast<const v8h*>(reinterpret_cast<const _Float16*>(kt) +
                                                      (wc + c * 16 + fr) * S + ks * 32 + g * 8);
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int c = 0; c < 2; ++c)
                    acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[a], bf[c], acc[a][c], 0, 0, 0);
        }
    } else {
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) {
            float af[2], bf[2];
#pragma unroll
            for (int a = 0; a < 2; ++a)
                af[a] = reinterpret_cast<const float*>(qt)[(wr + a * 16 + fr) * S + ks * 4 + g];
#pragma unroll
            for (int c = 0; c < 2; ++c)
                bf[c] = reinterpret_cast<const float*>(kt)[(wc + c * 16 + fr) * S + ks * 4 + g];
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int c = 0; c < 2; ++c)
                    acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[a], bf[c], acc[a][c], 0, 0, 0);
        }
    }

    const uint64_t plane = static_cast<uint64_t>(bh) * tokens;
    if (HALF) {
        // Stage the 64x64 binary16 tile in LDS (reusing the Q tile, same
        // shape) and write it as 16-byte row segments. Columns in [T, ldt)
        // come from zero key rows; the softmax overwrites them with zeros.
        __syncthreads();
        _Float16* st = reinterpret_cast<_Float16*>(qt);
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    st[(wr + a * 16 + 4 * g + r) * S + wc + c * 16 + fr] = static_cast<_Float16>(acc[a][c][r]);
        __syncthreads();
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int idx = tid + it * 256;  // 64 rows x 8 chunks of 8 halves
            const int row = idx >> 3, chunk = idx & 7;
            const uint32_t i = i0 + row, j = j0 + chunk * 8;
            if (i < tokens && j < ldt)
                *reinterpret_cast<v8h*>(static_cast<_Float16*>(scores_out) + (plane + i) * ldt + j) =
                    *reinterpret_cast<const v8h*>(st + row * S + chunk * 8);
        }
    } else {
#pragma unroll
        for (int a = 0; a < 2; ++a) {
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const uint32_t j = j0 + wc + c * 16 + fr;
                if (j >= tokens) continue;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t i = i0 + wr + a * 16 + 4 * g + r;
                    if (i < tokens) static_cast<float*>(scores_out)[(plane + i) * tokens + j] = acc[a][c][r];
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Softmax over rows, in place, one wave per row, the whole row in VGPRs
// (CH values per lane; CH = 0 streams the row three times instead).
// fp32: softmax_lastdim.glsl:19-69. fp16: softmax_lastdim_half.glsl:16-65 -
// exponentials are rounded to binary16, the denominator sums the unrounded
// fp32 exponentials, and p = fp16(float(fp16(e)) * (1/max(sum, 1e-20))).
// Padding columns [columns, row_stride) of fp16 rows are written as zero.
template <int CH, bool HALF>
__global__ __launch_bounds__(256) void softmax_kernel(void* data, uint64_t rows, uint32_t columns,
                                                      uint32_t row_stride) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t row = static_cast<uint64_t>(blockIdx.x) * 4u + (threadIdx.x >> 6);
    if (row >= rows) return;
    float* fr = HALF ? nullptr : static_cast<float*>(data) + row * row_stride;
    _Float16* hr = HALF ? static_cast<_Float16*>(data) + row * row_stride : nullptr;
    auto load = [&](uint32_t c) -> float {
        return HALF ? static_cast<float>(hr[c]) : fr[c];
    };
    float v[CH > 0 ? CH : 1];
    float maximum = -3.402823466e+38f;
    if (CH > 0) {
#pragma unroll
        for (int j = 0; j < (CH > 0 ? CH : 1); ++j) {
            const uint32_t c = lane + 64u * j;
            v[j] = c < columns ? load(c) : -3.402823466e+38f;
            maximum = fmaxf(maximum, v[j]);
        }
    } else {
        for (uint32_t c = lane; c < columns; c += 64u) maximum = fmaxf(maximum, load(c));
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
                v[j] = HALF ? static_cast<float>(static_cast<_Float16>(e)) : e;
            }
        }
    } else {
        for (uint32_t c = lane; c < columns; c += 64u) {
            const float e = expf(load(c) - maximum);
            sum = sum + e;
            if (HALF) hr[c] = static_cast<_Float16>(e);
            else fr[c] = e;
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
            if (c < columns) {
                if (HALF) hr[c] = static_cast<_Float16>(v[j] * inverse);
                else fr[c] = v[j] * inverse;
            }
        }
    } else {
        for (uint32_t c = lane; c < columns; c += 64u) {
            if (HALF) hr[c] = static_cast<_Float16>(static_cast<float>(hr[c]) * inverse);
            else fr[c] = fr[c] * inverse;
        }
    }
    if (HALF)
        for (uint32_t c = columns + lane; c < row_stride; c += 64u) hr[c] = static_cast<_Float16>(0.0f);
}

// ---------------------------------------------------------------------------
// out = P v. Workgroup: 128 query rows x 64 features of one (batch, head);
// wave w owns rows 32w..32w+31 (2x4 MFMA blocks). The key axis advances 32
// tokens per step; P (128x32) and v^T (64x32) are staged through LDS.
template <bool HALF>
__global__ __launch_bounds__(256) void attention_values_kernel(
    const void* __restrict__ probabilities, const float* __restrict__ qkv,
    float* __restrict__ out, uint32_t tokens, uint32_t heads, uint32_t ldt) {
    using T = typename std::conditional<HALF, _Float16, float>::type;
    constexpr int PS = HALF ? 40 : 33;  // padded LDS row lengths (elements)
    constexpr int VS = HALF ? 40 : 33;
    __shared__ __attribute__((aligned(16))) T pt[128 * PS];
    __shared__ __attribute__((aligned(16))) T vt[64 * VS];

    const uint32_t bh = blockIdx.z;
    const uint32_t b = bh / heads, h = bh - b * heads;
    const uint32_t D = heads * 64u;
    const uint32_t i0 = blockIdx.x * 128u;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int fr = lane & 15, g = lane >> 4;
    const float* vbase = qkv + static_cast<uint64_t>(b) * tokens * 3u * D + 2u * D + h * 64u;
    const uint64_t plane = static_cast<uint64_t>(bh) * tokens;
    const uint32_t pstride = HALF ? ldt : tokens;

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
            vt[(f4 + 0) * VS + jr] = static_cast<T>(vv.x);
            vt[(f4 + 1) * VS + jr] = static_cast<T>(vv.y);
            vt[(f4 + 2) * VS + jr] = static_cast<T>(vv.z);
            vt[(f4 + 3) * VS + jr] = static_cast<T>(vv.w);
        }
        // Stage P[i0..i0+128)[j0..j0+32): 4096 values, 16 per thread.
#pragma unroll
        for (int it = 0; it < 16; ++it) {
            const int c = tid + it * 256;
            const int ir = c >> 5, jc = c & 31;
            const uint32_t i = i0 + ir, j = j0 + jc;
            T p = static_cast<T>(0.0f);
            if (i < tokens && j < tokens) p = static_cast<const T*>(probabilities)[(plane + i) * pstride + j];
            pt[ir * PS + jc] = p;
        }
        __syncthreads();
        if (HALF) {
            v8h af[2], bf[4];
#pragma unroll
            for (int a = 0; a < 2; ++a)
                af[a] = *reinterpret_cast<const v8h*>(reinterpret_cast<const _Float16*>(pt) +
                                                      (wave * 32 + a * 16 + fr) * PS + g * 8);
#pragma unroll
            for (int c = 0; c < 4; ++c)
                bf[c] = *reinterpret_cast<const v8h*>(reinterpret_cast<const _Float16*>(vt) +
                                                      (c * 16 + fr) * VS + g * 8);
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[a], bf[c], acc[a][c], 0, 0, 0);
        } else {
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                float af[2], bf[4];
#pragma unroll
                for (int a = 0; a < 2; ++a)
                    af[a] = reinterpret_cast<const float*>(pt)[(wave * 32 + a * 16 + fr) * PS + ks * 4 + g];
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    bf[c] = reinterpret_cast<const float*>(vt)[(c * 16 + fr) * VS + ks * 4 + g];
#pragma unroll
                for (int a = 0; a < 2; ++a)
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[a], bf[c], acc[a][c], 0, 0, 0);
            }
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

// ---------------------------------------------------------------------------
// binary16 path, tuned kernels.
//
// V is first packed to binary16, feature-major: vt[bh][f][j], j padded with
// zeros to ldv = T rounded up to 32, so a PV operand fragment (8 consecutive
// tokens of one feature) is one 16-byte load.
inline uint32_t value_ld(uint32_t tokens) { return (tokens + 31u) & ~31u; }

__global__ __launch_bounds__(256) void pack_values_half_kernel(const float* __restrict__ qkv,
                                                               _Float16* __restrict__ vt, uint32_t tokens,
                                                               uint32_t heads, uint32_t ldv) {
    __shared__ float tile[64][65];
    const uint32_t bh = blockIdx.z;
    const uint32_t b = bh / heads, h = bh - b * heads;
    const uint32_t D = heads * 64u;
    const uint32_t j0 = blockIdx.x * 64u;
    const int tid = threadIdx.x;
    const float* vbase = qkv + static_cast<uint64_t>(b) * tokens * 3u * D + 2u * D + h * 64u;
#pragma unroll
    for (int it = 0; it < 4; ++it) {  // 64 tokens x 16 float4
        const int c = tid + it * 256;
        const int jr = c >> 4, f4 = (c & 15) * 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (j0 + jr < tokens) v = *reinterpret_cast<const float4*>(vbase + static_cast<uint64_t>(j0 + jr) * 3u * D + f4);
        tile[jr][f4 + 0] = v.x;
        tile[jr][f4 + 1] = v.y;
        tile[jr][f4 + 2] = v.z;
        tile[jr][f4 + 3] = v.w;
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 2; ++it) {  // 64 features x 8 chunks of 8 tokens
        const int c = tid + it * 256;
        const int f = c >> 3, jc = (c & 7) * 8;
        if (j0 + jc >= ldv) continue;
        v8h out;
#pragma unroll
        for (int k = 0; k < 8; ++k) out[k] = static_cast<_Float16>(tile[jc + k][f]);
        *reinterpret_cast<v8h*>(vt + (static_cast<uint64_t>(bh) * 64u + f) * ldv + j0 + jc) = out;
    }
}

// out = P v for 64 query rows of one (batch, head): the four waves split the
// key axis (wave w takes every fourth 32-token step), each accumulating a
// 64x64 partial on 4x4 MFMA blocks with operands loaded straight from global
// memory (P rows: 16 bytes per lane; vt: 16 bytes per lane). The partials are
// summed through LDS.
__global__ __launch_bounds__(256) void attention_values_half_kernel(const _Float16* __restrict__ p,
                                                                    const _Float16* __restrict__ vt,
                                                                    float* __restrict__ out, uint32_t tokens,
                                                                    uint32_t heads, uint32_t ldt, uint32_t ldv) {
    extern __shared__ float red[];  // [waves 1..3][64 rows][64 features]
    const uint32_t bh = blockIdx.z;
    const uint32_t b = bh / heads, h = bh - b * heads;
    const uint32_t D = heads * 64u;
    const uint32_t i0 = blockIdx.x * 64u;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int fr = lane & 15, g = lane >> 4;
    const _Float16* prow = p + static_cast<uint64_t>(bh) * tokens * ldt;
    const _Float16* vrow = vt + static_cast<uint64_t>(bh) * 64u * ldv;
    v4f acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[a][c] = v4f{0.f, 0.f, 0.f, 0.f};
    const uint32_t steps = (tokens + 31u) / 32u;
    for (uint32_t st = wave; st < steps; st += 4) {
        const uint32_t j = st * 32u + g * 8u;
        v8h af[4], bf[4];
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            const uint32_t i = i0 + a * 16 + fr;
            v8h v = {};
            if (i < tokens && j < ldt) v = *reinterpret_cast<const v8h*>(prow + static_cast<uint64_t>(i) * ldt + j);
            af[a] = v;
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) bf[c] = *reinterpret_cast<const v8h*>(vrow + static_cast<uint64_t>(c * 16 + fr) * ldv + j);
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int c = 0; c < 4; ++c)
                acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[a], bf[c], acc[a][c], 0, 0, 0);
    }
    // 16x16 result layout: lane holds rows 4*g + r of column fr. Waves 1-3
    // park their partials in LDS; wave 0 adds them to its own and stores.
    if (wave > 0) {
        float* mine = red + (wave - 1) * 4096;
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r) mine[(a * 16 + 4 * g + r) * 64 + c * 16 + fr] = acc[a][c][r];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = a * 16 + 4 * g + r;
                const uint32_t i = i0 + row;
                if (i >= tokens) continue;
                float* o = out + (static_cast<uint64_t>(b) * tokens + i) * D + h * 64u;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int idx = row * 64 + c * 16 + fr;
                    o[c * 16 + fr] = ((acc[a][c][r] + red[idx]) + red[4096 + idx]) + red[8192 + idx];
                }
            }
    }
}

// binary16 softmax, one wave per row, 16-byte loads: lane l owns the 8-column
// chunks l, l+64, ... (CPL chunks per lane). Same arithmetic as softmax_kernel.
template <int CPL>
__global__ __launch_bounds__(256) void softmax_half_kernel(_Float16* data, uint64_t rows, uint32_t columns,
                                                           uint32_t row_stride) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t row = static_cast<uint64_t>(blockIdx.x) * 4u + (threadIdx.x >> 6);
    if (row >= rows) return;
    _Float16* hr = data + row * row_stride;
    const uint32_t chunks = row_stride / 8u;
    float v[CPL][8];
    float maximum = -3.402823466e+38f;
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
        const uint32_t c = lane + 64u * k;
        v8h raw = {};
        if (c < chunks) raw = *reinterpret_cast<const v8h*>(hr + 8u * c);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const bool ok = c < chunks && 8u * c + e < columns;
            v[k][e] = ok ? static_cast<float>(raw[e]) : -3.402823466e+38f;
            maximum = fmaxf(maximum, v[k][e]);
        }
    }
    maximum = wave_max(maximum);
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
        const uint32_t c = lane + 64u * k;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const bool ok = c < chunks && 8u * c + e < columns;
            const float ex = ok ? expf(v[k][e] - maximum) : 0.0f;
            sum = sum + ex;
            v[k][e] = static_cast<float>(static_cast<_Float16>(ex));
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum = sum + __shfl_xor(sum, o, kWave);
    const float inverse = 1.0f / fmaxf(sum, 1.0e-20f);
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
        const uint32_t c = lane + 64u * k;
        if (c >= chunks) continue;
        v8h o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = static_cast<_Float16>(v[k][e] * inverse);  // padding: 0 * inverse
        *reinterpret_cast<v8h*>(hr + 8u * c) = o;
    }
}

template <bool HALF>
void launch_softmax(void* data, uint64_t rows, uint32_t columns, uint32_t stride, hipStream_t s) {
    const unsigned grid = ceil_div(rows, 4);
    if (HALF && stride % 8u == 0) {
        const uint32_t cpl = (stride / 8u + 63u) / 64u;
        _Float16* d = static_cast<_Float16*>(data);
#define DAV2_SMH_CASE(N) \
    hipLaunchKernelGGL((softmax_half_kernel<N>), dim3(grid), dim3(256), 0, s, d, rows, columns, stride)
        if (cpl <= 1) { DAV2_SMH_CASE(1); return; }
        if (cpl <= 2) { DAV2_SMH_CASE(2); return; }
        if (cpl <= 3) { DAV2_SMH_CASE(3); return; }
        if (cpl <= 4) { DAV2_SMH_CASE(4); return; }
        if (cpl <= 6) { DAV2_SMH_CASE(6); return; }
        if (cpl <= 8) { DAV2_SMH_CASE(8); return; }
        if (cpl <= 12) { DAV2_SMH_CASE(12); return; }
#undef DAV2_SMH_CASE
    }
    const uint32_t ch = (columns + 63u) / 64u;
#define DAV2_SM_CASE(N) \
    hipLaunchKernelGGL((softmax_kernel<N, HALF>), dim3(grid), dim3(256), 0, s, data, rows, columns, stride)
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

int dav2_hip_attention_scores(void* scores, const float* qkv, uint32_t tokens, uint32_t heads,
                              uint32_t batch, int fp16, void* stream) {
    if (tokens == 0 || heads == 0 || batch == 0) return hipSuccess;
    if (!scores || !qkv || (reinterpret_cast<uintptr_t>(qkv) & 15) || heads > 65535u / batch)
        return hipErrorInvalidValue;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid(ceil_div(tokens, 64), ceil_div(tokens, 64), heads * batch);
    if (fp16)
        hipLaunchKernelGGL(attention_scores_kernel<true>, grid, dim3(256), 0, s, qkv, scores, tokens, heads,
                           half_ld(tokens));
    else
        hipLaunchKernelGGL(attention_scores_kernel<false>, grid, dim3(256), 0, s, qkv, scores, tokens, heads,
                           tokens);
    return hipGetLastError();
}

int dav2_hip_softmax_rows(void* scores, uint64_t rows, uint32_t columns, uint32_t row_stride, int fp16,
                          void* stream) {
    if (rows == 0) return hipSuccess;
    if (!scores || columns == 0 || row_stride < columns) return hipErrorInvalidValue;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (fp16) launch_softmax<true>(scores, rows, columns, row_stride, s);
    else launch_softmax<false>(scores, rows, columns, row_stride, s);
    return hipGetLastError();
}

int dav2_hip_attention_values(float* out, const void* probabilities, const float* qkv, uint32_t tokens,
                              uint32_t heads, uint32_t batch, int fp16, void* stream) {
    if (tokens == 0 || heads == 0 || batch == 0) return hipSuccess;
    if (!out || !probabilities || !qkv || (reinterpret_cast<uintptr_t>(qkv) & 15) || heads > 65535u / batch)
        return hipErrorInvalidValue;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (fp16) {
        // The packed binary16 copy of v lives right after the scores.
        const uint32_t ldt = half_ld(tokens), ldv = value_ld(tokens);
        const uint64_t score_bytes = static_cast<uint64_t>(batch) * heads * tokens * ldt * 2u;
        _Float16* vt = reinterpret_cast<_Float16*>(const_cast<char*>(static_cast<const char*>(probabilities)) +
                                                   ((score_bytes + 255u) & ~255ull));
        hipLaunchKernelGGL(pack_values_half_kernel, dim3(ceil_div(ldv, 64), 1, heads * batch), dim3(256), 0, s, qkv,
                           vt, tokens, heads, ldv);
        hipLaunchKernelGGL(attention_values_half_kernel, dim3(ceil_div(tokens, 64), 1, heads * batch), dim3(256),
                           3 * 64 * 64 * sizeof(float), s, static_cast<const _Float16*>(probabilities), vt, out,
                           tokens, heads, ldt, ldv);
    } else {
        const dim3 grid(ceil_div(tokens, 128), 1, heads * batch);
        hipLaunchKernelGGL(attention_values_kernel<false>, grid, dim3(256), 0, s, probabilities, qkv, out, tokens,
                           heads, tokens);
    }
    return hipGetLastError();
}

uint64_t dav2_hip_attention_scratch_bytes(uint32_t tokens, uint32_t heads, uint32_t batch, int fp16) {
    const uint64_t bh = static_cast<uint64_t>(batch) * heads;
    if (!fp16) return bh * tokens * tokens * sizeof(float);
    const uint64_t score_bytes = bh * tokens * half_ld(tokens) * 2u;
    return ((score_bytes + 255u) & ~255ull) + bh * 64u * value_ld(tokens) * 2u;
}

}  // extern "C"
