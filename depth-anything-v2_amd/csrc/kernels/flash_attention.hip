// Integer-exact fused attention for head_dim 64 on gfx950 int8 matrix cores.
//
// Replaces the int8-mode attention of src/operators.cpp:1132-1167
// (bmm_score_fp16.glsl -> softmax_lastdim_half.glsl -> bmm_value_fp16.glsl),
// which materialises binary16 scores [H][T][T]. Here every sum is an exact
// integer, so the result does not depend on summation order and a CPU
// restatement reproduces it bit for bit:
//
//   q*0.125 and k per token row, v per feature column (over the tokens), in
//   15-bit block floating point: x ~= X * 2^e, |X| <= 16383, X = 128*d1 + d0
//   with digits d1 in [-128, 127] and d0 in [0, 127] (two int8 planes);
//   s_ij = fp32(Q_i . K_j * 2^(eq_i + ek_j))        exact dot, one rounding
//   E_ij = min(rint(exp_cw(s_ij - max_j s_ij) * 2^21), 2^21 - 1)
//        = 2^14 e2 + 2^7 e1 + e0 (three 7-bit digits)
//   o_if = ldexp(fp32(sum_j E_ij V_jf) / fp32(sum_j E_ij), ev_f)
//
// Digit products run on v_mfma_i32_16x16x64_i8 (exact int32 sums); the
// partial sums are recombined in double precision, where they are exact.
//
// Kernels: zero the column maxima; pack q/k rows into digit planes and
// take column maxima of v; pack v into digit planes (key-permuted, see
// below); attention. Attention: one workgroup = 4 waves = 64 queries of one
// (batch, head), wave w owns 16 queries. Key blocks of 64 are staged through
// LDS (double buffered, one barrier per block). Pass 1 computes the row
// maxima, pass 2 recomputes the same scores and accumulates E V.
//
// The wave computes S^T = K Q^T (keys x queries), so after the score MFMAs
// lane l holds, for its query l%16, keys 16j + 4g + r of the block (j, r in
// 0..3, g = l/16). Those 16 values, packed as bytes in slot 4j + r, are the
// B operand of the PV MFMA without any register exchange when the value
// planes store key 16j + 4g + r at block position 16g + 4j + r.

#include <math.h>

#include "common.h"
#include "dav2_hip.h"

using namespace dav2k;

namespace {

constexpr uint32_t kBlock = 64;   // keys per LDS block, queries per workgroup
constexpr int kRow = 80;          // LDS bytes per 64-byte digit row (16 padding)
constexpr int kPlane = 64 * kRow; // one digit plane of a block in LDS
constexpr float kE = 2097152.0f;  // 2^21
constexpr int kEMax = 2097151;

inline uint32_t padded_tokens(uint32_t tokens) { return (tokens + kBlock - 1u) / kBlock * kBlock; }

// Block position p (0..63) of the value planes holds key perm64(p).
DAV2_DEV uint32_t perm64(uint32_t p) { return ((p >> 2) & 3u) * 16u + 4u * (p >> 4) + (p & 3u); }

struct Layout {
    uint64_t planes_q, planes_k, planes_v;  // byte offsets of the digit planes
    uint64_t exp_q, exp_k, exp_v, colmax;   // byte offsets of int32/uint32 arrays
    uint64_t bytes;
};

inline Layout layout_for(uint32_t tokens, uint32_t heads, uint32_t batch) {
    const uint64_t bh = static_cast<uint64_t>(batch) * heads, tp = padded_tokens(tokens);
    Layout l{};
    l.planes_q = 0;
    l.planes_k = l.planes_q + bh * 2 * tp * 64;
    l.planes_v = l.planes_k + bh * 2 * tp * 64;
    l.exp_q = l.planes_v + bh * 2 * 64 * tp;
    l.exp_k = l.exp_q + bh * tp * 4;
    l.exp_v = l.exp_k + bh * tp * 4;
    l.colmax = l.exp_v + bh * 64 * 4;
    l.bytes = l.colmax + bh * 64 * 4;
    return l;
}

// x -> (digit1, digit0) of clamp(rint(x * 2^shift), +-16383).
DAV2_DEV void digits15(float x, int shift, int8_t& d1, int8_t& d0) {
    const float v = fminf(fmaxf(__builtin_rintf(ldexpf(x, shift)), -16383.0f), 16383.0f);
    const int X = static_cast<int>(v);
    d1 = static_cast<int8_t>(X >> 7);
    d0 = static_cast<int8_t>(X & 127);
}

__global__ void zero_colmax_kernel(uint32_t* colmax, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) colmax[i] = 0u;
}

// One wave per q or k row (lane = feature): 64 tokens x {q, k} per
// workgroup. Also folds |v| of the workgroup's tokens into colmax.
__global__ __launch_bounds__(256) void pack_rows_kernel(const float* __restrict__ qkv, int8_t* __restrict__ qd,
                                                        int8_t* __restrict__ kd, int* __restrict__ qe,
                                                        int* __restrict__ ke, uint32_t* __restrict__ colmax,
                                                        uint32_t tokens, uint32_t heads, uint32_t tp) {
    __shared__ float vmax[4][64];
    const uint32_t h = blockIdx.y, b = blockIdx.z, bh = b * heads + h;
    const uint32_t D = heads * 64u;
    const uint32_t j0 = blockIdx.x * kBlock;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float* base = qkv + static_cast<uint64_t>(b) * tokens * 3u * D + h * 64u + lane;
    for (int r = wave; r < 128; r += 4) {
        const bool is_k = r >= 64;
        const uint32_t t = j0 + (r & 63);
        float x = 0.0f;
        if (t < tokens) {
            x = base[static_cast<uint64_t>(t) * 3u * D + (is_k ? D : 0u)];
            if (!is_k) x = x * 0.125f;
        }
        const float a = wave_max(fabsf(x));
        int e = 0;
        int8_t d1 = 0, d0 = 0;
        if (a != 0.0f) {
            frexpf(a, &e);
            digits15(x, 14 - e, d1, d0);
        }
        int8_t* planes = is_k ? kd : qd;
        const uint64_t o = (static_cast<uint64_t>(bh) * 2u * tp + t) * 64u + lane;
        planes[o + static_cast<uint64_t>(tp) * 64u] = d1;  // plane 1
        planes[o] = d0;                                    // plane 0
        if (lane == 0) (is_k ? ke : qe)[static_cast<uint64_t>(bh) * tp + t] = a != 0.0f ? e - 14 : 0;
    }
    float m = 0.0f;
    for (int i = 0; i < 16; ++i) {
        const uint32_t t = j0 + wave * 16 + i;
        if (t < tokens) m = fmaxf(m, fabsf(base[static_cast<uint64_t>(t) * 3u * D + 2u * D]));
    }
    vmax[wave][lane] = m;
    __syncthreads();
    if (wave == 0) {
        m = fmaxf(fmaxf(vmax[0][lane], vmax[1][lane]), fmaxf(vmax[2][lane], vmax[3][lane]));
        // |v| >= 0: the IEEE bit patterns order like the values
        atomicMax(colmax + static_cast<uint64_t>(bh) * 64u + lane, __float_as_uint(m));
    }
}

// v of 64 tokens -> two digit planes [64 features][tp], key-permuted.
__global__ __launch_bounds__(256) void pack_values_kernel(const float* __restrict__ qkv,
                                                          const uint32_t* __restrict__ colmax,
                                                          int8_t* __restrict__ vd, int* __restrict__ ve,
                                                          uint32_t tokens, uint32_t heads, uint32_t tp) {
    __shared__ float tile[64][65];  // [token][feature]
    const uint32_t h = blockIdx.y, b = blockIdx.z, bh = b * heads + h;
    const uint32_t D = heads * 64u;
    const uint32_t j0 = blockIdx.x * kBlock;
    const int tid = threadIdx.x;
    const float* base = qkv + static_cast<uint64_t>(b) * tokens * 3u * D + 2u * D + h * 64u;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int c = tid + it * 256;
        const uint32_t jr = static_cast<uint32_t>(c) >> 4, f4 = (static_cast<uint32_t>(c) & 15u) * 4u;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (j0 + jr < tokens) v = *reinterpret_cast<const float4*>(base + static_cast<uint64_t>(j0 + jr) * 3u * D + f4);
        tile[jr][f4 + 0] = v.x;
        tile[jr][f4 + 1] = v.y;
        tile[jr][f4 + 2] = v.z;
        tile[jr][f4 + 3] = v.w;
    }
    __syncthreads();
    const uint32_t f = static_cast<uint32_t>(tid) >> 2, p0 = (static_cast<uint32_t>(tid) & 3u) * 16u;
    const float a = __uint_as_float(colmax[static_cast<uint64_t>(bh) * 64u + f]);
    int e = 0;
    if (a != 0.0f) frexpf(a, &e);
    int8_t hi[16], lo[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        hi[i] = 0;
        lo[i] = 0;
        if (a != 0.0f) digits15(tile[perm64(p0 + i)][f], 14 - e, hi[i], lo[i]);
    }
    int8_t* row1 = vd + ((static_cast<uint64_t>(bh) * 2u + 1u) * 64u + f) * tp + j0 + p0;
    int8_t* row0 = vd + ((static_cast<uint64_t>(bh) * 2u) * 64u + f) * tp + j0 + p0;
    v4i w1, w0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        w1[q] = static_cast<int>(pack4(hi[4 * q], hi[4 * q + 1], hi[4 * q + 2], hi[4 * q + 3]));
        w0[q] = static_cast<int>(pack4(lo[4 * q], lo[4 * q + 1], lo[4 * q + 2], lo[4 * q + 3]));
    }
    *reinterpret_cast<v4i*>(row1) = w1;
    *reinterpret_cast<v4i*>(row0) = w0;
    if (blockIdx.x == 0 && (tid & 3) == 0) ve[static_cast<uint64_t>(bh) * 64u + f] = a != 0.0f ? e - 14 : 0;
}

DAV2_DEV v4i mfma8(v4i a, v4i b, v4i c) { return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0); }

__global__ __launch_bounds__(256) void attention_exact_kernel(const int8_t* __restrict__ qd,
                                                              const int8_t* __restrict__ kd,
                                                              const int8_t* __restrict__ vd,
                                                              const int* __restrict__ qe,
                                                              const int* __restrict__ ke,
                                                              const int* __restrict__ ve,
                                                              float* __restrict__ out, uint32_t tokens,
                                                              uint32_t heads, uint32_t tp) {
    // [buffer][K1 | K0 | V1 | V0] digit rows, then [buffer][64] key exponents
    __shared__ __attribute__((aligned(16))) int8_t lds[2][4 * kPlane];
    __shared__ int kexp[2][64];
    const uint32_t h = blockIdx.y, b = blockIdx.z, bh = b * heads + h;
    const uint32_t D = heads * 64u;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, g = lane >> 4;
    const uint32_t q0 = blockIdx.x * kBlock + wave * 16u;
    const uint64_t plane_qk = static_cast<uint64_t>(tp) * 64u;

    const int8_t* kbase = kd + static_cast<uint64_t>(bh) * 2u * plane_qk;
    const int8_t* vbase = vd + static_cast<uint64_t>(bh) * 2u * plane_qk;
    const int* kebase = ke + static_cast<uint64_t>(bh) * tp;

    // B operand of S^T = K Q^T: lane holds features 16g..16g+15 of query col.
    const int8_t* qrow = qd + static_cast<uint64_t>(bh) * 2u * plane_qk + static_cast<uint64_t>(q0 + col) * 64u + g * 16;
    const v4i q1 = *reinterpret_cast<const v4i*>(qrow + plane_qk);
    const v4i q0v = *reinterpret_cast<const v4i*>(qrow);
    const int qexp = qe[static_cast<uint64_t>(bh) * tp + q0 + col];

    // Staging: K planes (2 x 64 rows x 64 B) and V planes, 16-byte chunks:
    // chunk c < 512: plane c >> 8, row (c >> 2) & 63, 16-byte column c & 3.
    v4i stage[4];
    int kstage = 0;
    auto fetch = [&](uint32_t kb, bool values) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t c = static_cast<uint32_t>(tid) + 256u * i;
            const uint32_t plane = c >> 8, row = (c >> 2) & 63u, c16 = (c & 3u) * 16u;
            stage[i] = *reinterpret_cast<const v4i*>(kbase + plane * plane_qk +
                                                     (static_cast<uint64_t>(kb) * kBlock + row) * 64u + c16);
            if (values)
                stage[2 + i] = *reinterpret_cast<const v4i*>(vbase + (plane * 64u + row) * static_cast<uint64_t>(tp) +
                                                             kb * kBlock + c16);
        }
        if (tid < 64) kstage = kebase[kb * kBlock + tid];
    };
    auto store = [&](int buf, bool values) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t c = static_cast<uint32_t>(tid) + 256u * i;
            const uint32_t plane = c >> 8, row = (c >> 2) & 63u, c16 = (c & 3u) * 16u;
            // LDS planes: K1 = 0, K0 = 1, V1 = 2, V0 = 3 (global plane 1 is the high digit)
            *reinterpret_cast<v4i*>(&lds[buf][(1u - plane) * kPlane + row * kRow + c16]) = stage[i];
            if (values) *reinterpret_cast<v4i*>(&lds[buf][(3u - plane) * kPlane + row * kRow + c16]) = stage[2 + i];
        }
        if (tid < 64) kexp[buf][tid] = kstage;
    };
    // Scores of sub-block j for this lane: keys 16j + 4g + r, query col.
    auto scores = [&](int buf, int j, uint32_t kb, float s[4]) {
        const int8_t* k1 = &lds[buf][0 * kPlane + (j * 16 + col) * kRow + g * 16];
        const int8_t* k0 = &lds[buf][1 * kPlane + (j * 16 + col) * kRow + g * 16];
        const v4i a1 = *reinterpret_cast<const v4i*>(k1);
        const v4i a0 = *reinterpret_cast<const v4i*>(k0);
        const v4i zero = {0, 0, 0, 0};
        const v4i hi = mfma8(a1, q1, zero);
        const v4i mid = mfma8(a0, q1, mfma8(a1, q0v, zero));
        const v4i lo = mfma8(a0, q0v, zero);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t key = kb * kBlock + j * 16 + 4 * g + r;
            // exact: |hi| <= 2^20, |mid| <= 2^21, |lo| <= 2^20
            const double dot = (static_cast<double>(hi[r]) * 16384.0 + static_cast<double>(mid[r]) * 128.0) +
                               static_cast<double>(lo[r]);
            const float v = static_cast<float>(ldexp(dot, qexp + kexp[buf][j * 16 + 4 * g + r]));
            s[r] = key < tokens ? v : -INFINITY;
        }
    };

    const uint32_t blocks = tp / kBlock;
    // Pass 1: row maxima.
    float m = -INFINITY;
    fetch(0, false);
    store(0, false);
    __syncthreads();
    for (uint32_t kb = 0; kb < blocks; ++kb) {
        const int buf = static_cast<int>(kb & 1u);
        if (kb + 1 < blocks) fetch(kb + 1, false);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float s[4];
            scores(buf, j, kb, s);
            m = fmaxf(fmaxf(m, fmaxf(s[0], s[1])), fmaxf(s[2], s[3]));
        }
        if (kb + 1 < blocks) store(buf ^ 1, false);
        __syncthreads();
    }
    m = fmaxf(m, __shfl_xor(m, 16, kWave));
    m = fmaxf(m, __shfl_xor(m, 32, kWave));

    // Pass 2: E = 21-bit softmax numerators, sum_j E, sum_j E V.
    v4i c0[4], c7[4], c14[4], c21[4];
#pragma unroll
    for (int fb = 0; fb < 4; ++fb) c0[fb] = c7[fb] = c14[fb] = c21[fb] = v4i{0, 0, 0, 0};
    uint64_t lsum = 0;
    fetch(0, true);
    store(0, true);
    __syncthreads();
    for (uint32_t kb = 0; kb < blocks; ++kb) {
        const int buf = static_cast<int>(kb & 1u);
        if (kb + 1 < blocks) fetch(kb + 1, true);
        v4i e0, e1, e2;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float s[4];
            scores(buf, j, kb, s);
            int d0[4], d1[4], d2[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = exp_cw(s[r] - m) * kE;
                const int E = min(static_cast<int>(__builtin_rintf(e)), kEMax);
                lsum += static_cast<uint32_t>(E);
                d0[r] = E & 127;
                d1[r] = (E >> 7) & 127;
                d2[r] = E >> 14;
            }
            e0[j] = static_cast<int>(pack4(d0[0], d0[1], d0[2], d0[3]));
            e1[j] = static_cast<int>(pack4(d1[0], d1[1], d1[2], d1[3]));
            e2[j] = static_cast<int>(pack4(d2[0], d2[1], d2[2], d2[3]));
        }
#pragma unroll
        for (int fb = 0; fb < 4; ++fb) {
            const v4i v1 = *reinterpret_cast<const v4i*>(&lds[buf][2 * kPlane + (fb * 16 + col) * kRow + g * 16]);
            const v4i v0 = *reinterpret_cast<const v4i*>(&lds[buf][3 * kPlane + (fb * 16 + col) * kRow + g * 16]);
            c0[fb] = mfma8(v0, e0, c0[fb]);
            c7[fb] = mfma8(v1, e0, mfma8(v0, e1, c7[fb]));
            c14[fb] = mfma8(v1, e1, mfma8(v0, e2, c14[fb]));
            c21[fb] = mfma8(v1, e2, c21[fb]);
        }
        if (kb + 1 < blocks) store(buf ^ 1, true);
        __syncthreads();
    }
    double l = static_cast<double>(lsum);
    l = l + __shfl_xor(l, 16, kWave);
    l = l + __shfl_xor(l, 32, kWave);
    const float lf = static_cast<float>(l);
    const uint32_t q = q0 + col;
    if (q < tokens) {
        const int* vexp = ve + static_cast<uint64_t>(bh) * 64u;
        float* dst = out + (static_cast<uint64_t>(b) * tokens + q) * D + h * 64u + 4u * g;
#pragma unroll
        for (int fb = 0; fb < 4; ++fb) {
            float o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                // exact: every term is an integer below 2^52
                const double num = (static_cast<double>(c21[fb][r]) * 2097152.0 + static_cast<double>(c14[fb][r]) * 16384.0) +
                                   (static_cast<double>(c7[fb][r]) * 128.0 + static_cast<double>(c0[fb][r]));
                o[r] = ldexpf(static_cast<float>(num) / lf, vexp[fb * 16 + 4 * g + r]);
            }
            *reinterpret_cast<float4*>(dst + fb * 16) = make_float4(o[0], o[1], o[2], o[3]);
        }
    }
}

}  // namespace

extern "C" {

DAV2_API uint64_t dav2_hip_attention_fused_scratch_bytes(uint32_t tokens, uint32_t heads, uint32_t batch) {
    return layout_for(tokens, heads, batch).bytes;
}

DAV2_API int dav2_hip_attention_fused(float* out, const float* qkv, uint32_t tokens, uint32_t heads,
                                      uint32_t batch, void* scratch, uint64_t scratch_bytes, void* stream) {
    if (!out || !qkv || !scratch || tokens == 0 || heads == 0 || batch == 0) return hipErrorInvalidValue;
    if (heads > 65535u || batch > 65535u || tokens > 65536u) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(qkv) |
         reinterpret_cast<uintptr_t>(scratch)) & 15u)
        return hipErrorInvalidValue;
    const Layout l = layout_for(tokens, heads, batch);
    if (scratch_bytes < l.bytes) return hipErrorInvalidValue;
    const uint32_t tp = padded_tokens(tokens);
    uint8_t* base = static_cast<uint8_t*>(scratch);
    int8_t* qd = reinterpret_cast<int8_t*>(base + l.planes_q);
    int8_t* kd = reinterpret_cast<int8_t*>(base + l.planes_k);
    int8_t* vd = reinterpret_cast<int8_t*>(base + l.planes_v);
    int* qe = reinterpret_cast<int*>(base + l.exp_q);
    int* ke = reinterpret_cast<int*>(base + l.exp_k);
    int* ve = reinterpret_cast<int*>(base + l.exp_v);
    uint32_t* colmax = reinterpret_cast<uint32_t*>(base + l.colmax);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint32_t ncol = batch * heads * 64u;
    const dim3 grid(tp / kBlock, heads, batch);
    hipLaunchKernelGGL(zero_colmax_kernel, dim3(ceil_div(ncol, 256)), dim3(256), 0, s, colmax, ncol);
    hipLaunchKernelGGL(pack_rows_kernel, grid, dim3(256), 0, s, qkv, qd, kd, qe, ke, colmax, tokens, heads, tp);
    hipLaunchKernelGGL(pack_values_kernel, grid, dim3(256), 0, s, qkv, colmax, vd, ve, tokens, heads, tp);
    hipLaunchKernelGGL(attention_exact_kernel, grid, dim3(256), 0, s, qd, kd, vd, qe, ke, ve, out, tokens, heads, tp);
    return hipGetLastError();
}

}  // extern "C"
