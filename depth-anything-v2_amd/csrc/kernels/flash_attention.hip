// Integer-exact fused attention for head_dim 64 on gfx950 int8 matrix cores.
//
// Replaces the int8-mode attention of src/operators.cpp:1132-1167
// (bmm_score_fp16.glsl -> softmax_lastdim_half.glsl -> bmm_value_fp16.glsl),
// which materialises binary16 scores [H][T][T]. Here every sum is an exact
// integer, so the result does not depend on summation order and a CPU
// restatement reproduces it bit for bit:
//
//   q*0.125 per token row, k per (batch, head) and v per feature column, in
//   15-bit block floating point: x ~= X * 2^e, |X| <= 16383, X = 128*d1 + d0
//   with digits d1 in [-128, 127] and d0 in [0, 127] (two int8 planes);
//   u_ij = fma(H, 2^14, fp32(R)) with the exact digit sums
//          H = sum_f d1(q) d1(k) and R = Q_i . K_j - 2^14 H
//   (the score is u_ij * 2^(eq_i + ek): one exponent per query row)
//   x_ij = (u_ij - max_j u_ij) * (log2(e) * 2^(eq_i + ek))
//   E_ij = min(rint(pow2(x_ij) * 2^21), 2^21 - 1)
//        = 2^14 e2 + 2^7 e1 + e0 (three 7-bit digits)
//   o_if = ldexp(fp32(sum_j E_ij V_jf) / fp32(sum_j E_ij), ev_f)
//   pow2: n = rint(x), f = x - n, degree-6 Taylor polynomial of 2^f, * 2^n.
//
// Digit products run on v_mfma_i32_16x16x64_i8 (exact int32 sums); the
// output sums are recombined in double precision, where they are exact.
//
// Kernels: pack (q rows into digit planes, per-block maxima of |k| and of
// |v| per column), pack k and v (reduce the block maxima, digit planes, v
// key-permuted as below), attention.
//
// Attention: one workgroup = 4 waves = 2 query groups of 16 x 2 key halves.
// The two waves of a key half share its key blocks of 64, staged through a
// ring of three 8 KB LDS slots per half (48 KB per workgroup, three
// workgroups per CU). Pass 1 computes the row maxima,
// pass 2 recomputes the same scores and accumulates E and E V; the halves
// combine their maxima and their (exact integer) sums through LDS.
//
// The wave computes S^T = K Q^T (keys x queries), so after the score MFMAs
// lane l holds, for its query l%16, keys 16j + 4g + r of the block (j, r in
// 0..3, g = l/16). Those 16 values, packed as bytes in slot 4j + r, are the
// B operand of the PV MFMA without any register exchange when the value
// planes store key 16j + 4g + r at block position 16g + 4j + r.

#include <math.h>

#include <type_traits>

#include "common.h"
#include "dav2_hip.h"

using namespace dav2k;

namespace {

constexpr uint32_t kBlock = 64;    // keys per LDS block, tokens per pack workgroup
constexpr int kPlane = 64 * 64;   // one digit plane of a block in LDS (64 rows x 64 B)
constexpr int kSlot = 2 * kPlane;  // one block's K1 | K0 or V1 | V0 planes
constexpr int kSlots = 3;          // ring slots per key half
constexpr int kEMax = 2097151;     // 2^21 - 1
constexpr int kAttnThreads = 256;  // 2 query groups x 2 key halves
constexpr size_t kAttnLds = 2 * kSlots * kSlot;  // [key half][slot]
static_assert(2 * 64 * 67 * 4 <= kAttnLds, "the sums hand-over fits in the slots");

inline uint32_t padded_tokens(uint32_t tokens) { return (tokens + kBlock - 1u) / kBlock * kBlock; }

// Block position p (0..63) of the value planes holds key perm64(p).
DAV2_DEV uint32_t perm64(uint32_t p) { return ((p >> 2) & 3u) * 16u + 4u * (p >> 4) + (p & 3u); }

// LDS byte offset of 16-byte chunk c (0..3) of digit row r: chunks are XOR
// swizzled with bits 2..3 of the row, so the 16 rows one MFMA operand load
// touches (same logical chunk) fall on 16 distinct 16-byte bank groups.
DAV2_DEV uint32_t lds_chunk(uint32_t r, uint32_t c) { return r * 64u + ((c ^ (r >> 2)) & 3u) * 16u; }

struct Layout {
    uint64_t planes_q, planes_k, planes_v;     // byte offsets of the digit planes
    uint64_t exp_q, exp_k, exp_v, kmax, vmax;  // int32 exponents, fp32 block maxima
    uint64_t bytes;
};

inline Layout layout_for(uint32_t tokens, uint32_t heads, uint32_t batch) {
    const uint64_t bh = static_cast<uint64_t>(batch) * heads, tp = padded_tokens(tokens);
    const uint64_t nblk = tp / kBlock;
    Layout l{};
    l.planes_q = 0;
    l.planes_k = l.planes_q + bh * 2 * tp * 64;
    l.planes_v = l.planes_k + bh * 2 * tp * 64;
    l.exp_q = l.planes_v + bh * 2 * 64 * tp;
    l.exp_k = l.exp_q + bh * tp * 4;
    l.exp_v = l.exp_k + bh * 4;
    l.kmax = l.exp_v + bh * 64 * 4;  // [bh][nblk]
    l.vmax = l.kmax + bh * nblk * 4;  // [bh][nblk][64]
    l.bytes = l.vmax + bh * nblk * 64 * 4;
    return l;
}

// x -> (digit1, digit0) of clamp(rint(x * 2^shift), +-16383).
DAV2_DEV void digits15(float x, int shift, int8_t& d1, int8_t& d0) {
    const float v = fminf(fmaxf(__builtin_rintf(ldexpf(x, shift)), -16383.0f), 16383.0f);
    const int X = static_cast<int>(v);
    d1 = static_cast<int8_t>(X >> 7);
    d0 = static_cast<int8_t>(X & 127);
}

DAV2_DEV void store_digits16(int8_t* plane1, int8_t* plane0, const int8_t d1[16], const int8_t d0[16]) {
    v4i w1, w0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        w1[q] = static_cast<int>(pack4(d1[4 * q], d1[4 * q + 1], d1[4 * q + 2], d1[4 * q + 3]));
        w0[q] = static_cast<int>(pack4(d0[4 * q], d0[4 * q + 1], d0[4 * q + 2], d0[4 * q + 3]));
    }
    *reinterpret_cast<v4i*>(plane1) = w1;
    *reinterpret_cast<v4i*>(plane0) = w0;
}

// 64 tokens per workgroup; thread t owns token row t/4, features 16*(t%4)..
// q*0.125 rows -> digit planes; maxima of |k| and of |v| per column over the
// block -> kmax[bh][block], vmax[bh][block][64].
__global__ __launch_bounds__(256) void pack_q_kernel(const float* __restrict__ qkv, int8_t* __restrict__ qd,
                                                     int* __restrict__ qe, float* __restrict__ kmax,
                                                     float* __restrict__ vmax, uint32_t tokens, uint32_t heads,
                                                     uint32_t tp) {
    __shared__ float vcol[64][65];
    __shared__ float kpart[4];
    const uint32_t h = blockIdx.y, b = blockIdx.z, bh = b * heads + h;
    const uint32_t D = heads * 64u;
    const uint32_t nblk = tp / kBlock;
    const int tid = threadIdx.x, row = tid >> 2, c16 = (tid & 3) * 16;
    const uint32_t t = blockIdx.x * kBlock + row;
    float q[16], mk = 0.0f;
    if (t < tokens) {
        const float* src = qkv + (static_cast<uint64_t>(b) * tokens + t) * 3u * D + h * 64u + c16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 vq = *reinterpret_cast<const float4*>(src + 4 * i);
            const float4 vk = *reinterpret_cast<const float4*>(src + D + 4 * i);
            const float4 vv = *reinterpret_cast<const float4*>(src + 2u * D + 4 * i);
            q[4 * i + 0] = vq.x * 0.125f;
            q[4 * i + 1] = vq.y * 0.125f;
            q[4 * i + 2] = vq.z * 0.125f;
            q[4 * i + 3] = vq.w * 0.125f;
            mk = fmaxf(mk, fmaxf(fmaxf(fabsf(vk.x), fabsf(vk.y)), fmaxf(fabsf(vk.z), fabsf(vk.w))));
            vcol[row][c16 + 4 * i + 0] = fabsf(vv.x);
            vcol[row][c16 + 4 * i + 1] = fabsf(vv.y);
            vcol[row][c16 + 4 * i + 2] = fabsf(vv.z);
            vcol[row][c16 + 4 * i + 3] = fabsf(vv.w);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            q[i] = 0.0f;
            vcol[row][c16 + i] = 0.0f;
        }
    }
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) a = fmaxf(a, fabsf(q[i]));
    a = fmaxf(a, __shfl_xor(a, 1, kWave));
    a = fmaxf(a, __shfl_xor(a, 2, kWave));
    int e = 0;
    if (a != 0.0f) frexpf(a, &e);
    int8_t d1[16], d0[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        d1[i] = 0;
        d0[i] = 0;
        if (a != 0.0f) digits15(q[i], 14 - e, d1[i], d0[i]);
    }
    int8_t* p0 = qd + (static_cast<uint64_t>(bh) * 2u * tp + t) * 64u + c16;
    store_digits16(p0 + static_cast<uint64_t>(tp) * 64u, p0, d1, d0);
    if ((tid & 3) == 0) qe[static_cast<uint64_t>(bh) * tp + t] = a != 0.0f ? e - 14 : 0;

    mk = wave_max(mk);
    if ((tid & 63) == 0) kpart[tid >> 6] = mk;
    __syncthreads();
    if (tid == 0) kmax[static_cast<uint64_t>(bh) * nblk + blockIdx.x] = fmaxf(fmaxf(kpart[0], kpart[1]), fmaxf(kpart[2], kpart[3]));
    if (tid < 64) {
        float m = 0.0f;
        for (int r = 0; r < 64; ++r) m = fmaxf(m, vcol[r][tid]);
        vmax[(static_cast<uint64_t>(bh) * nblk + blockIdx.x) * 64u + tid] = m;
    }
}

// k (per-head exponent) and v (per-column exponent) of 64 tokens into digit
// planes: k row-major [tp][64], v feature-major [64][tp] and key-permuted.
__global__ __launch_bounds__(256) void pack_kv_kernel(const float* __restrict__ qkv, const float* __restrict__ kmax,
                                                      const float* __restrict__ vmax, int8_t* __restrict__ kd,
                                                      int8_t* __restrict__ vd, int* __restrict__ ke,
                                                      int* __restrict__ ve, uint32_t tokens, uint32_t heads,
                                                      uint32_t tp) {
    __shared__ float tile[64][65];  // v [token][feature]
    __shared__ float kred[4];
    __shared__ float vred[4][64];
    const uint32_t h = blockIdx.y, b = blockIdx.z, bh = b * heads + h;
    const uint32_t D = heads * 64u;
    const uint32_t nblk = tp / kBlock;
    const uint32_t j0 = blockIdx.x * kBlock;
    const int tid = threadIdx.x, hi4 = tid >> 2, c16 = (tid & 3) * 16;

    // Head maximum of |k| and column maxima of |v| from the block maxima
    // (wave w folds blocks w, w + 4, ...; lane = feature).
    float mk = 0.0f, mv = 0.0f;
    for (uint32_t i = static_cast<uint32_t>(tid); i < nblk; i += 256u) mk = fmaxf(mk, kmax[static_cast<uint64_t>(bh) * nblk + i]);
    for (uint32_t i = static_cast<uint32_t>(tid >> 6); i < nblk; i += 4u)
        mv = fmaxf(mv, vmax[(static_cast<uint64_t>(bh) * nblk + i) * 64u + (tid & 63)]);
    mk = wave_max(mk);
    if ((tid & 63) == 0) kred[tid >> 6] = mk;
    vred[tid >> 6][tid & 63] = mv;

    const uint32_t t = j0 + hi4;  // k: token row hi4, features c16..c16+15
    float k[16];
    const float* src = qkv + (static_cast<uint64_t>(b) * tokens + t) * 3u * D + D + h * 64u + c16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float4 vk = make_float4(0.f, 0.f, 0.f, 0.f), vv = vk;
        if (t < tokens) {
            vk = *reinterpret_cast<const float4*>(src + 4 * i);
            vv = *reinterpret_cast<const float4*>(src + D + 4 * i);
        }
        k[4 * i + 0] = vk.x;
        k[4 * i + 1] = vk.y;
        k[4 * i + 2] = vk.z;
        k[4 * i + 3] = vk.w;
        tile[hi4][c16 + 4 * i + 0] = vv.x;
        tile[hi4][c16 + 4 * i + 1] = vv.y;
        tile[hi4][c16 + 4 * i + 2] = vv.z;
        tile[hi4][c16 + 4 * i + 3] = vv.w;
    }
    __syncthreads();
    mv = fmaxf(fmaxf(vred[0][hi4], vred[1][hi4]), fmaxf(vred[2][hi4], vred[3][hi4]));
    int8_t d1[16], d0[16];
    {
        const float a = fmaxf(fmaxf(kred[0], kred[1]), fmaxf(kred[2], kred[3]));
        int e = 0;
        if (a != 0.0f) frexpf(a, &e);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            d1[i] = 0;
            d0[i] = 0;
            if (a != 0.0f) digits15(k[i], 14 - e, d1[i], d0[i]);
        }
        int8_t* p0 = kd + ((static_cast<uint64_t>(bh) * 2u) * tp + t) * 64u + c16;
        store_digits16(p0 + static_cast<uint64_t>(tp) * 64u, p0, d1, d0);
        if (blockIdx.x == 0 && tid == 0) ke[bh] = a != 0.0f ? e - 14 : 0;
    }
    {  // v: feature hi4, block positions c16..c16+15
        int e = 0;
        if (mv != 0.0f) frexpf(mv, &e);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            d1[i] = 0;
            d0[i] = 0;
            if (mv != 0.0f) digits15(tile[perm64(c16 + i)][hi4], 14 - e, d1[i], d0[i]);
        }
        int8_t* p0 = vd + ((static_cast<uint64_t>(bh) * 2u) * 64u + hi4) * tp + j0 + c16;
        store_digits16(p0 + static_cast<uint64_t>(tp) * 64u, p0, d1, d0);
        if (blockIdx.x == 0 && (tid & 3) == 0) ve[static_cast<uint64_t>(bh) * 64u + hi4] = mv != 0.0f ? e - 14 : 0;
    }
}

// One image: q, k or v (blockIdx.z = 0, 1, 2) of 64 tokens of head h into
// digit planes in one pass (pack_q_kernel + pack_kv_kernel for batch 1),
// the maxima of |k| and |v| per column coming from the qkv GEMM's row-tile
// partials col_absmax[t][c] (c < D: k column c, c >= D: v column c - D).
// Thread t owns token row t/4, features 16*(t%4)..+15 of q or k, and
// feature t/4, block positions 16*(t%4)..+15 of v.
__global__ __launch_bounds__(256) void pack_qkv_kernel(const float* __restrict__ qkv,
                                                       const float* __restrict__ col_absmax, uint32_t partial_rows,
                                                       int8_t* __restrict__ qd, int8_t* __restrict__ kd,
                                                       int8_t* __restrict__ vd, int* __restrict__ qe,
                                                       int* __restrict__ ke, int* __restrict__ ve, uint32_t tokens,
                                                       uint32_t heads, uint32_t tp) {
    __shared__ float tile[64][65];  // v [token][feature]
    __shared__ float red[4][64];    // k: per-wave maxima; v: per-wave column maxima
    const uint32_t h = blockIdx.y, part = blockIdx.z;
    const uint32_t D = heads * 64u;
    const uint32_t j0 = blockIdx.x * kBlock;
    const int tid = threadIdx.x, hi4 = tid >> 2, c16 = (tid & 3) * 16;
    const uint32_t t = j0 + hi4;

    // The row's values and (k, v) the first four partial maxima of the
    // lane's column are loaded together, so that their latencies overlap.
    float x[16];
    {
        const float* src = qkv + static_cast<uint64_t>(t) * 3u * D + part * D + h * 64u + c16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (t < tokens) v = *reinterpret_cast<const float4*>(src + 4 * i);
            x[4 * i + 0] = v.x;
            x[4 * i + 1] = v.y;
            x[4 * i + 2] = v.z;
            x[4 * i + 3] = v.w;
        }
    }
    // Head maximum of |k| (part 1) or column maxima of |v| (part 2) from the
    // partials: wave w folds row tiles w, w + 4, ...; lane = feature. The
    // first 16 row tiles are loaded at once (indices clamped: a repeated row
    // leaves a maximum unchanged), further ones in a loop.
    const uint32_t f = static_cast<uint32_t>(tid & 63);
    const float* cols = col_absmax + (part == 0 ? 0u : (part - 1u) * D) + h * 64u + f;
    float pm[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (part != 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t r = min(static_cast<uint32_t>(tid >> 6) + 4u * i, partial_rows - 1u);
            pm[i] = cols[static_cast<uint64_t>(r) * 2u * D];
        }
    }
    // digits of every value (a zero maximum means zero values; the select
    // keeps NaN inputs at 0 digits there, as before)
    int8_t d1[16], d0[16];
    auto digits_of = [&](const float (&v)[16], float maximum, int e) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            int8_t a1, a0;
            digits15(v[i], 14 - e, a1, a0);
            d1[i] = maximum != 0.0f ? a1 : int8_t(0);
            d0[i] = maximum != 0.0f ? a0 : int8_t(0);
        }
    };
    if (part == 0) {  // q * 0.125: exponent of the row maximum over the four lanes of the row
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            x[i] = x[i] * 0.125f;
            a = fmaxf(a, fabsf(x[i]));
        }
        a = fmaxf(a, __shfl_xor(a, 1, kWave));
        a = fmaxf(a, __shfl_xor(a, 2, kWave));
        int e = 0;
        if (a != 0.0f) frexpf(a, &e);
        digits_of(x, a, e);
        int8_t* p0 = qd + (static_cast<uint64_t>(h) * 2u * tp + t) * 64u + c16;
        store_digits16(p0 + static_cast<uint64_t>(tp) * 64u, p0, d1, d0);
        if ((tid & 3) == 0) qe[static_cast<uint64_t>(h) * tp + t] = a != 0.0f ? e - 14 : 0;
        return;
    }
    if (part == 2) {
#pragma unroll
        for (int i = 0; i < 16; ++i) tile[hi4][c16 + i] = x[i];
    }
    {
        float m = fmaxf(fmaxf(pm[0], pm[1]), fmaxf(pm[2], pm[3]));
        for (uint32_t r = static_cast<uint32_t>(tid >> 6) + 16u; r < partial_rows; r += 4u)
            m = fmaxf(m, cols[static_cast<uint64_t>(r) * 2u * D]);
        if (part == 1) m = wave_max(m);
        red[tid >> 6][f] = m;
    }
    __syncthreads();
    if (part == 1) {  // k: one exponent per head
        const float a = fmaxf(fmaxf(red[0][0], red[1][0]), fmaxf(red[2][0], red[3][0]));
        int e = 0;
        if (a != 0.0f) frexpf(a, &e);
        digits_of(x, a, e);
        int8_t* p0 = kd + (static_cast<uint64_t>(h) * 2u * tp + t) * 64u + c16;
        store_digits16(p0 + static_cast<uint64_t>(tp) * 64u, p0, d1, d0);
        if (blockIdx.x == 0 && tid == 0) ke[h] = a != 0.0f ? e - 14 : 0;
        return;
    }
    {  // v: feature hi4, block positions c16..c16+15 (all 16 read before use)
        const float mv = fmaxf(fmaxf(red[0][hi4], red[1][hi4]), fmaxf(red[2][hi4], red[3][hi4]));
        int e = 0;
        if (mv != 0.0f) frexpf(mv, &e);
        float vv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) vv[i] = tile[perm64(c16 + i)][hi4];
        digits_of(vv, mv, e);
        int8_t* p0 = vd + (static_cast<uint64_t>(h) * 2u * 64u + hi4) * tp + j0 + c16;
        store_digits16(p0 + static_cast<uint64_t>(tp) * 64u, p0, d1, d0);
        if (blockIdx.x == 0 && (tid & 3) == 0) ve[static_cast<uint64_t>(h) * 64u + hi4] = mv != 0.0f ? e - 14 : 0;
    }
}

DAV2_DEV v4i mfma8(v4i a, v4i b, v4i c) { return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0); }

// E = rint(min(pow2(x) * 2^21, 2^21 - 1)) for x <= 0 (or -inf: 0), returned
// as the bits of E + 2^23, i.e. 0x4B000000 + E. pow2(x) = 2^n p(x - n),
// n = rint(max(x, -100)), p the degree-5 minimax polynomial of 2^f on
// [-1/2, 1/2] (relative error 7.5e-8 before rounding), its coefficients times
// 2^21, which scales every Horner step exactly. Adding 2^23 rounds ties to
// even. The clamp to -100 matters only for x = -inf (masked keys, CLAMP):
// every finite x below -100 gives E = 0 with or without it.
template <bool CLAMP>
DAV2_DEV uint32_t numerator21_bits(float x) {
    constexpr float k21 = 2097152.0f;
    const float xc = CLAMP ? fmaxf(x, -100.0f) : x;
    const float n = __builtin_rintf(xc);
    const float f = xc - n;
    float p = 1.327647245e-3f * k21;
    p = fmaf(p, f, 9.675540961e-3f * k21);
    p = fmaf(p, f, 5.550713092e-2f * k21);
    p = fmaf(p, f, 2.402212024e-1f * k21);
    p = fmaf(p, f, 6.931469440e-1f * k21);
    p = fmaf(p, f, 1.000000119e+0f * k21);
    const float v = fminf(ldexpf(p, static_cast<int>(n)), static_cast<float>(kEMax));
    return __float_as_uint(v + 8388608.0f);
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

DAV2_DEV uint32_t shr16x2(uint32_t v, int s) {  // each 16-bit half shifted right
    u16x2 h = __builtin_bit_cast(u16x2, v);
    h = h >> static_cast<unsigned short>(s);
    return __builtin_bit_cast(uint32_t, h);
}

// 7-bit digits of E_k = R_k - 0x4B000000 (k = 0..3, E_k < 2^21) as the bytes
// of three words: w0 = E_k & 127, w1 = (E_k >> 7) & 127, w2 = E_k >> 14.
DAV2_DEV void digits21(const uint32_t R[4], int& w0, int& w1, int& w2) {
    const uint32_t lo01 = __builtin_amdgcn_perm(R[1], R[0], 0x05040100u);  // R0 bits 0..15 | R1 bits 0..15
    const uint32_t lo23 = __builtin_amdgcn_perm(R[3], R[2], 0x05040100u);
    const uint32_t hi01 = __builtin_amdgcn_perm(R[1], R[0], 0x06050201u);  // R0 bits 8..23 | R1 bits 8..23
    const uint32_t hi23 = __builtin_amdgcn_perm(R[3], R[2], 0x06050201u);
    // byte 0 of each 16-bit half, gathered: [x01.b0, x01.b2, x23.b0, x23.b2]
    w0 = static_cast<int>(__builtin_amdgcn_perm(lo23, lo01, 0x06040200u) & 0x7f7f7f7fu);
    w1 = static_cast<int>(__builtin_amdgcn_perm(shr16x2(lo23, 7), shr16x2(lo01, 7), 0x06040200u) & 0x7f7f7f7fu);
    // bits 14..21 of R: bit 21 is 0 (E < 2^21)
    w2 = static_cast<int>(__builtin_amdgcn_perm(shr16x2(hi23, 6), shr16x2(hi01, 6), 0x06040200u));
}

// Wave w: query group w & 1 (16 queries), key half w >> 1.
// Three workgroups per CU need at most 168 VGPRs (3 waves per SIMD).
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(3))) void attention_exact_kernel(
    const int8_t* __restrict__ qd, const int8_t* __restrict__ kd, const int8_t* __restrict__ vd,
    const int* __restrict__ qe, const int* __restrict__ ke, const int* __restrict__ ve, float* __restrict__ out,
    uint32_t tokens, uint32_t heads, uint32_t tp) {
    extern __shared__ __attribute__((aligned(16))) int8_t lds[];  // [half][slot][kSlot]
    // Workgroups are dealt to the 8 XCDs round robin; give each XCD one
    // contiguous run of (head, query tile) pairs, so that the key and value
    // planes of a head are read by one XCD and stay in its L2.
    const uint32_t qtiles = gridDim.x, total = gridDim.x * gridDim.y * gridDim.z;
    const uint32_t id = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
    const uint32_t xcd = id & 7u, slot = id >> 3, per = total >> 3, extra = total & 7u;
    const uint32_t lin = xcd * per + min(xcd, extra) + slot;
    const uint32_t qtile = lin % qtiles, bh = lin / qtiles, b = bh / heads, h = bh - b * heads;
    const uint32_t D = heads * 64u;
    const int tid = threadIdx.x, lane = tid & 63;
    // wave-uniform values kept in scalar registers (uniform branches)
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int group = wave & 1, half = wave >> 1;
    const int col = lane & 15, g = lane >> 4;
    const uint32_t q0 = qtile * 32u + group * 16u;
    const uint64_t plane_qk = static_cast<uint64_t>(tp) * 64u;
    const uint32_t blocks = tp / kBlock;
    const uint32_t first_half = (blocks + 1u) / 2u;  // blocks of half 0; half 1 has the rest
    const uint32_t kb0 = half ? first_half : 0u;
    const uint32_t nkb = half ? blocks - first_half : first_half;
    int8_t* slots = lds + half * kSlots * kSlot;

    const int8_t* kbase = kd + static_cast<uint64_t>(bh) * 2u * plane_qk;
    const int8_t* vbase = vd + static_cast<uint64_t>(bh) * 2u * plane_qk;

    // B operand of S^T = K Q^T: lane holds features 16g..16g+15 of query col.
    const int8_t* qrow = qd + static_cast<uint64_t>(bh) * 2u * plane_qk + static_cast<uint64_t>(q0 + col) * 64u + g * 16;
    const v4i q1 = *reinterpret_cast<const v4i*>(qrow + plane_qk);
    const v4i q0v = *reinterpret_cast<const v4i*>(qrow);
    // log2(e) * 2^(eq + ek): turns u - max u into the exponent of 2
    const float row_scale = ldexpf(1.44269504f, qe[static_cast<uint64_t>(bh) * tp + q0 + col] + ke[bh]);

    // Staging of one key half, global memory straight into LDS
    // (global_load_lds_dwordx4, no registers). A slot holds the two digit
    // planes (0 = high, 1 = low: 2 x 64 rows x 64 B) of a block's keys or of
    // its values. Each 1 KB piece (16 rows of one plane) is one wave
    // instruction: lane l lands at piece + 16 l, i.e. row 16 q + l / 4,
    // physical chunk l % 4, and fetches the logical chunk that lds_chunk()
    // stores there. The two waves of a key half issue 4 pieces each per slot.
    const int wave_in_half = group;
    auto issue_planes = [&](uint32_t kb, int8_t* slot, bool values) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t piece = static_cast<uint32_t>(wave_in_half) * 4u + i;  // 0..7
            const uint32_t lplane = piece >> 2;                                   // 0: high, 1: low digit
            const uint32_t row = (piece & 3u) * 16u + (static_cast<uint32_t>(lane) >> 2);
            const uint32_t c = ((static_cast<uint32_t>(lane) & 3u) ^ (row >> 2)) & 3u;  // logical chunk
            const uint32_t gplane = 1u - lplane;                                   // global plane 1 = high digit
            const int8_t* src = values ? vbase + (gplane * 64u + row) * static_cast<uint64_t>(tp) + kb * kBlock + c * 16u
                                       : kbase + gplane * plane_qk + (static_cast<uint64_t>(kb) * kBlock + row) * 64u + c * 16u;
            copy16_to_lds(src, slot + lplane * kPlane + (piece & 3u) * 1024u);
        }
    };
    // Waits until this wave has at most `later` slots' copies outstanding
    // (copies retire in issue order, 4 per slot and wave), then a plain
    // barrier: the slot issued before those has landed in every wave
    // (__syncthreads would also drain the later slots).
    auto wait_slots = [&](int later) {
        if (later >= 2) DAV2_WAIT_VMCNT(8);
        else if (later == 1) DAV2_WAIT_VMCNT(4);
        else DAV2_WAIT_VMCNT(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };
    // Unscaled scores of the block for this lane: u[j][r] = key 16j + 4g + r,
    // query col; TAIL masks keys >= tokens. The MFMAs of two key groups are
    // issued before their results are converted (fewer live registers than
    // all four).
    auto block_scores = [&](const int8_t* t, uint32_t kb, auto TAIL, float s[4][4]) {
        const v4i zero = {0, 0, 0, 0};
#pragma unroll
        for (int jp = 0; jp < 4; jp += 2) {
            v4i hi[2], mid[2], lo[2];
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const uint32_t at = lds_chunk((jp + jj) * 16 + col, g);
                const v4i a1 = *reinterpret_cast<const v4i*>(t + 0 * kPlane + at);
                const v4i a0 = *reinterpret_cast<const v4i*>(t + 1 * kPlane + at);
                hi[jj] = mfma8(a1, q1, zero);
                mid[jj] = mfma8(a1, q0v, zero);
                lo[jj] = mfma8(a0, q0v, zero);
                mid[jj] = mfma8(a0, q1, mid[jj]);
            }
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int j = jp + jj;
                    // |128 mid + lo| < 2^29 (exact in int32); hi * 2^14 is exact in fp32
                    const int rest = mid[jj][r] * 128 + lo[jj][r];
                    float v = fmaf(static_cast<float>(hi[jj][r]), 16384.0f, static_cast<float>(rest));
                    if (decltype(TAIL)::value && kb * kBlock + j * 16 + 4 * g + r >= tokens) v = -INFINITY;
                    s[j][r] = v;
                }
        }
    };

    const bool ragged = tokens != tp;
    // Pass 1: row maxima of u over this key half, K only, blocks it and
    // it + 1 in flight while it is scored (slot it % 3).
    float m = -INFINITY;
    if (nkb > 0) issue_planes(kb0, slots, false);
    if (nkb > 1) issue_planes(kb0 + 1, slots + kSlot, false);
    for (uint32_t it = 0; it < first_half; ++it) {
        const uint32_t kb = kb0 + it;
        const bool have = it < nkb;
        // this wave has issued blocks up to min(it + 1, nkb - 1)
        wait_slots(have ? min(1, static_cast<int>(nkb) - 1 - static_cast<int>(it)) : 0);
        if (it + 2 < nkb) issue_planes(kb + 2, slots + ((it + 2) % kSlots) * kSlot, false);
        if (have) {
            const int8_t* t = slots + (it % kSlots) * kSlot;
            // block maximum inside each variant: the scores are then fma
            // results, which max needs no canonicalization for
            auto block_max = [&](auto TAIL) {
                float s[4][4];
                block_scores(t, kb, TAIL, s);
                float bm = fmaxf(fmaxf(s[0][0], s[0][1]), s[0][2]);
#pragma unroll
                for (int i = 3; i < 15; i += 2) bm = fmaxf(fmaxf(bm, s[i >> 2][i & 3]), s[(i + 1) >> 2][(i + 1) & 3]);
                return fmaxf(bm, s[3][3]);
            };
            m = fmaxf(m, ragged && kb + 1 == blocks ? block_max(std::true_type{}) : block_max(std::false_type{}));
        }
    }
    __syncthreads();  // every wave is done with the pass-1 ring before it is reused
    m = fmaxf(m, __shfl_xor(m, 16, kWave));
    m = fmaxf(m, __shfl_xor(m, 32, kWave));
    // [half][group][query] maxima; every wave has read them (full barrier)
    // before pass 2 copies anything.
    float* half_max = reinterpret_cast<float*>(lds);
    if (g == 0) half_max[(half * 2 + group) * 16 + col] = m;
    __syncthreads();
    m = fmaxf(half_max[group * 16 + col], half_max[(2 + group) * 16 + col]);
    __syncthreads();

    // Pass 2: E = 21-bit softmax numerators, sum_j E, sum_j E V over this half.
    // Slots rotate: block it has K in slot ks and V in slot vs; K(it + 1) is
    // copied into the free slot once block it - 1 is done everywhere (top
    // barrier), V(it + 1) into ks once every wave has scored block it (middle
    // barrier).
    v4i c0[4], c7[4], c14[4], c21[4];
#pragma unroll
    for (int fb = 0; fb < 4; ++fb) c0[fb] = c7[fb] = c14[fb] = c21[fb] = v4i{0, 0, 0, 0};
    // sum_j E as the three digit sums, on the MFMA (A = all ones)
    v4i l0 = {0, 0, 0, 0}, l7 = l0, l14 = l0;
    const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    // x = (u - max) log2(e) 2^(eq + ek) as fma(u, scale, -(max * scale))
    const float neg_ms = -(m * row_scale);
    int ks = 0, vs = 1, fs = 2;
    if (nkb > 0) {
        issue_planes(kb0, slots, false);
        issue_planes(kb0, slots + kSlot, true);
    }
    for (uint32_t it = 0; it < first_half; ++it) {
        const uint32_t kb = kb0 + it;
        const bool have = it < nkb;
        const bool next = it + 1 < nkb;
        wait_slots(have ? 1 : 0);  // K(it); V(it) may still be in flight
        if (next) issue_planes(kb + 1, slots + fs * kSlot, false);
        float s[4][4];
        if (have) {
            const int8_t* t = slots + ks * kSlot;
            if (ragged && kb + 1 == blocks)
                block_scores(t, kb, std::true_type{}, s);
            else
                block_scores(t, kb, std::false_type{}, s);
        }
        wait_slots(next ? 1 : 0);  // V(it); K(it + 1) may still be in flight
        if (next) issue_planes(kb + 1, slots + ks * kSlot, true);
        if (have) {
            const int8_t* t = slots + vs * kSlot;
            v4i e0, e1, e2;
            auto numerators = [&](auto CLAMP) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    uint32_t R[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        R[r] = numerator21_bits<decltype(CLAMP)::value>(fmaf(s[j][r], row_scale, neg_ms));
                    int w0, w1, w2;
                    digits21(R, w0, w1, w2);
                    e0[j] = w0;
                    e1[j] = w1;
                    e2[j] = w2;
                }
            };
            if (ragged && kb + 1 == blocks)  // masked keys carry u = -inf
                numerators(std::true_type{});
            else
                numerators(std::false_type{});
            l0 = mfma8(ones, e0, l0);
            l7 = mfma8(ones, e1, l7);
            l14 = mfma8(ones, e2, l14);
#pragma unroll
            for (int fb = 0; fb < 4; ++fb) {
                const uint32_t at = lds_chunk(fb * 16 + col, g);
                const v4i v1 = *reinterpret_cast<const v4i*>(t + 0 * kPlane + at);
                const v4i v0 = *reinterpret_cast<const v4i*>(t + 1 * kPlane + at);
                c0[fb] = mfma8(v0, e0, c0[fb]);
                c7[fb] = mfma8(v1, e0, mfma8(v0, e1, c7[fb]));
                c14[fb] = mfma8(v1, e1, mfma8(v0, e2, c14[fb]));
                c21[fb] = mfma8(v1, e2, c21[fb]);
            }
        }
        const int k2 = fs;
        fs = vs;
        vs = ks;
        ks = k2;
    }
    __syncthreads();  // every wave is done with the ring before the sums reuse it

    // Half 1 hands its integer sums to half 0 (exact adds): [group][lane][67].
    int* red = reinterpret_cast<int*>(lds);
    if (half == 1) {
        int* mine = red + (group * 64 + lane) * 67;
#pragma unroll
        for (int fb = 0; fb < 4; ++fb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                mine[fb * 16 + r] = c0[fb][r];
                mine[fb * 16 + 4 + r] = c7[fb][r];
                mine[fb * 16 + 8 + r] = c14[fb][r];
                mine[fb * 16 + 12 + r] = c21[fb][r];
            }
        mine[64] = l0[0];
        mine[65] = l7[0];
        mine[66] = l14[0];
    }
    __syncthreads();
    if (half == 1) return;
    {
        const int* other = red + (group * 64 + lane) * 67;
#pragma unroll
        for (int fb = 0; fb < 4; ++fb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                c0[fb][r] += other[fb * 16 + r];
                c7[fb][r] += other[fb * 16 + 4 + r];
                c14[fb][r] += other[fb * 16 + 8 + r];
                c21[fb][r] += other[fb * 16 + 12 + r];
            }
        l0[0] += other[64];
        l7[0] += other[65];
        l14[0] += other[66];
    }
    // digit sums < 2^31 each (< 2^17 keys x 127); the total is exact in double
    const double l = static_cast<double>(l14[0]) * 16384.0 + (static_cast<double>(l7[0]) * 128.0 + static_cast<double>(l0[0]));
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

// Digit packing (two passes, or one from the GEMM's column maxima when
// col_absmax is given, batch 1), then the attention kernel.
int run_attention(float* out, const float* qkv, uint32_t tokens, uint32_t heads, uint32_t batch,
                  const float* col_absmax, uint32_t partial_rows, void* scratch, uint64_t scratch_bytes,
                  void* stream) {
    if (!out || !qkv || !scratch || tokens == 0 || heads == 0 || batch == 0) return hipErrorInvalidValue;
    if (heads > 65535u || batch > 65535u || tokens > 65536u) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(qkv) |
         reinterpret_cast<uintptr_t>(scratch)) & 15u)
        return hipErrorInvalidValue;
    const Layout l = layout_for(tokens, heads, batch);
    if (scratch_bytes < l.bytes) return hipErrorInvalidValue;
    static const hipError_t lds_ok = hipFuncSetAttribute(reinterpret_cast<const void*>(attention_exact_kernel),
                                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                                         static_cast<int>(kAttnLds));
    if (lds_ok != hipSuccess) return lds_ok;
    const uint32_t tp = padded_tokens(tokens);
    uint8_t* base = static_cast<uint8_t*>(scratch);
    int8_t* qd = reinterpret_cast<int8_t*>(base + l.planes_q);
    int8_t* kd = reinterpret_cast<int8_t*>(base + l.planes_k);
    int8_t* vd = reinterpret_cast<int8_t*>(base + l.planes_v);
    int* qe = reinterpret_cast<int*>(base + l.exp_q);
    int* ke = reinterpret_cast<int*>(base + l.exp_k);
    int* ve = reinterpret_cast<int*>(base + l.exp_v);
    float* kmax = reinterpret_cast<float*>(base + l.kmax);
    float* vmax = reinterpret_cast<float*>(base + l.vmax);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid(tp / kBlock, heads, batch);
    if (col_absmax) {
        dispatch(pack_qkv_kernel, dim3(tp / kBlock, heads, 3), dim3(256), 0, s, qkv, col_absmax,
                           partial_rows, qd, kd, vd, qe, ke, ve, tokens, heads, tp);
    } else {
        dispatch(pack_q_kernel, grid, dim3(256), 0, s, qkv, qd, qe, kmax, vmax, tokens, heads, tp);
        dispatch(pack_kv_kernel, grid, dim3(256), 0, s, qkv, kmax, vmax, kd, vd, ke, ve, tokens, heads, tp);
    }
    dispatch(attention_exact_kernel, dim3(tp / 32u, heads, batch), dim3(kAttnThreads), kAttnLds, s, qd,
                       kd, vd, qe, ke, ve, out, tokens, heads, tp);
    return hipGetLastError();
}

}  // namespace

extern "C" {

DAV2_API uint64_t dav2_hip_attention_fused_scratch_bytes(uint32_t tokens, uint32_t heads, uint32_t batch) {
    return layout_for(tokens, heads, batch).bytes;
}

DAV2_API int dav2_hip_attention_fused(float* out, const float* qkv, uint32_t tokens, uint32_t heads,
                                      uint32_t batch, void* scratch, uint64_t scratch_bytes, void* stream) {
    return run_attention(out, qkv, tokens, heads, batch, nullptr, 0, scratch, scratch_bytes, stream);
}

DAV2_API int dav2_hip_attention_fused_colmax(float* out, const float* qkv, uint32_t tokens, uint32_t heads,
                                             const float* col_absmax, uint32_t partial_rows, void* scratch,
                                             uint64_t scratch_bytes, void* stream) {
    if (!col_absmax || partial_rows == 0 || (reinterpret_cast<uintptr_t>(col_absmax) & 3u)) return hipErrorInvalidValue;
    return run_attention(out, qkv, tokens, heads, 1, col_absmax, partial_rows, scratch, scratch_bytes, stream);
}

}  // extern "C"
