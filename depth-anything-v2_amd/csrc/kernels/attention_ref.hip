// Head-64 attention in the reference's own arithmetic order, for gfx950.
//
// Reference: src/operators.cpp:1098-1209 (attention_head64) with
//   fp32:     bmm.glsl:31-154 (scores and values), softmax_lastdim.glsl:19-69;
//   binary16: bmm_score_fp16.glsl:13-70, softmax_lastdim_half.glsl:16-65,
//             bmm_value_fp16.glsl:22-80 (the reference's int8-mode default,
//             encoder.cpp:389-396, on devices without the cooperative-matrix
//             score shader).
// Every output element is the same sequence of IEEE operations the shaders
// state: a score is a sum over the 64 features in order 0..63, an output
// element a sum over the source tokens in order 0..T-1, each product
// rounded to binary16 first in the binary16 pipeline; the softmax partitions
// a row over 128 lanes (lane = column % 128, or packed word % 128) and adds
// the lane partials by the halving tree. No multiply-add is contracted
// (-ffp-contract=off), exp is exp_cw and the division is IEEE, the same
// choices as the CPU oracle, so both produce the same bits. These sums are
// sequential per output, so they run on the VALU (a matrix core's
// accumulation order is its own).
//
// Cooperative-matrix scores (bmm_score_coop_fp16.glsl:12-33, the reference's
// int8-mode scores on devices with cooperative_matrix_fp16): the same binary16
// operands, every product exact, summed in fp32 by the matrix unit in its own
// order (coopMatMulAdd), the sum stored as binary16. Here that is
// v_mfma_f32_16x16x32_f16 (two K steps of 32 features per 16 x 16 block);
// softmax and values as above.
//
// Layouts: qkv [batch*T][3*H*64] token-major (q | k | v, head h at h*64);
// fp32 scores [batch][H][T][T] floats; binary16 scores [batch][H][T][words]
// packed half2 words, words = ceil(T/2) (the reference's layout and size);
// out [batch*T][H*64].

#include "common.h"
#include "dav2_hip.h"

using namespace dav2k;

namespace {

constexpr int kQueryTile = 128;  // score tile: 128 queries x 64 keys
constexpr int kKeyTile = 64;
constexpr int kValueRows = 64;   // value tile: 64 queries x 64 features
constexpr int kSourceChunk = 32; // source tokens staged per step

// packHalf2x16: each fp32 value rounded to binary16 (round to nearest even).
// The values are pinned as fp32 first so that the conversion rounds the fp32
// result, never a fused wider intermediate.
DAV2_DEV uint32_t pack_half2(float lo, float hi) {
    const _Float16 a = static_cast<_Float16>(keep_fp32(lo)), b = static_cast<_Float16>(keep_fp32(hi));
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, a)) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b)) << 16);
}

DAV2_DEV float half_lo(uint32_t w) { return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w))); }
DAV2_DEV float half_hi(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
}

// ---------------------------------------------------------------------------
// Scores. Thread (tx, ty) of 16 x 16 owns queries ty*8 .. +7 and keys
// tx*4 .. +3 of the tile, 32 sums. LDS holds the tile's q*0.125 and k
// feature-major so that a thread's 8 query and 4 key values of one feature
// are two and one 16-byte reads. Binary16: the values are rounded to binary16
// when staged (stored as floats: exact).
template <bool HALF>
__global__ __launch_bounds__(256) void ref_scores_kernel(const float* __restrict__ qkv, void* __restrict__ scores,
                                                         uint32_t tokens, uint32_t heads) {
    __shared__ __attribute__((aligned(16))) float qs[64][kQueryTile + 4];
    __shared__ __attribute__((aligned(16))) float ks[64][kKeyTile + 4];
    const uint32_t bh = blockIdx.z;
    const uint32_t b = bh / heads, h = bh - b * heads;
    const uint32_t D = heads * 64u;
    const uint32_t i0 = blockIdx.y * kQueryTile, j0 = blockIdx.x * kKeyTile;
    const float* base = qkv + static_cast<uint64_t>(b) * tokens * 3u * D + h * 64u;
    const int tid = threadIdx.x;

    // 128 query rows x 64 features: 2048 float4, 8 per thread; 64 key rows: 4.
#pragma unroll
    for (int it = 0; it < 8; ++it) {
        const int c = tid + it * 256;
        const int r = c >> 4, f4 = (c & 15) * 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i0 + r < tokens) v = *reinterpret_cast<const float4*>(base + static_cast<uint64_t>(i0 + r) * 3u * D + f4);
        // bmm.glsl:57-63 / bmm_score_fp16.glsl:32-33: q * 0.125 (exact), then binary16
        float q[4] = {v.x * 0.125f, v.y * 0.125f, v.z * 0.125f, v.w * 0.125f};
#pragma unroll
        for (int e = 0; e < 4; ++e)
            qs[f4 + e][r] = HALF ? static_cast<float>(static_cast<_Float16>(keep_fp32(q[e]))) : q[e];
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int c = tid + it * 256;
        const int r = c >> 4, f4 = (c & 15) * 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (j0 + r < tokens)
            v = *reinterpret_cast<const float4*>(base + static_cast<uint64_t>(j0 + r) * 3u * D + D + f4);
        float k[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) ks[f4 + e][r] = HALF ? static_cast<float>(static_cast<_Float16>(k[e])) : k[e];
    }
    __syncthreads();

    const int tx = tid & 15, ty = tid >> 4;
    float s[8][4];
#pragma unroll
    for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) s[r][c] = 0.0f;
#pragma unroll 4
    for (int f = 0; f < 64; ++f) {
        const float4 qa = *reinterpret_cast<const float4*>(&qs[f][ty * 8]);
        const float4 qb = *reinterpret_cast<const float4*>(&qs[f][ty * 8 + 4]);
        const float4 kv = *reinterpret_cast<const float4*>(&ks[f][tx * 4]);
        const float q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        const float k[4] = {kv.x, kv.y, kv.z, kv.w};
        if (HALF) {
            const h2 k01 = {static_cast<_Float16>(k[0]), static_cast<_Float16>(k[1])};
            const h2 k23 = {static_cast<_Float16>(k[2]), static_cast<_Float16>(k[3])};
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const _Float16 qh = static_cast<_Float16>(q[r]);
                const h2 qq = {qh, qh};
                add_half_products(s[r][0], s[r][1], qq, k01);
                add_half_products(s[r][2], s[r][3], qq, k23);
            }
        } else {
#pragma unroll
            for (int r = 0; r < 8; ++r)
#pragma unroll
                for (int c = 0; c < 4; ++c) s[r][c] = s[r][c] + q[r] * k[c];
        }
    }

    const uint64_t plane = static_cast<uint64_t>(bh) * tokens;
    const uint32_t j = j0 + tx * 4;
    if (HALF) {
        // packHalf2x16 of (column, column + 1); a column past the row is 0
        const uint32_t words = (tokens + 1u) >> 1;
        uint32_t* out = static_cast<uint32_t*>(scores);
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const uint32_t i = i0 + ty * 8 + r;
            if (i >= tokens) continue;
#pragma unroll
            for (int c = 0; c < 4; c += 2) {
                if (j + c >= tokens) continue;
                const float hi = j + c + 1 < tokens ? s[r][c + 1] : 0.0f;
                out[(plane + i) * words + (j + c) / 2] = pack_half2(s[r][c], hi);
            }
        }
    } else {
        float* out = static_cast<float*>(scores);
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const uint32_t i = i0 + ty * 8 + r;
            if (i >= tokens) continue;
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (j + c < tokens) out[(plane + i) * tokens + j + c] = s[r][c];
        }
    }
}

// ---------------------------------------------------------------------------
// Cooperative-matrix scores. v_mfma_f32_16x16x32_f16 operands: lane l holds
// row (A) or column (B) l % 16, K elements 8 (l / 16) .. + 7; the result
// element (row 4 (l / 16) + i, column l % 16) is lane l's i-th value.
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));

DAV2_DEV h8 half8(const float4& a, const float4& b, float scale) {
    return h8{static_cast<_Float16>(keep_fp32(a.x * scale)), static_cast<_Float16>(keep_fp32(a.y * scale)),
              static_cast<_Float16>(keep_fp32(a.z * scale)), static_cast<_Float16>(keep_fp32(a.w * scale)),
              static_cast<_Float16>(keep_fp32(b.x * scale)), static_cast<_Float16>(keep_fp32(b.y * scale)),
              static_cast<_Float16>(keep_fp32(b.z * scale)), static_cast<_Float16>(keep_fp32(b.w * scale))};
}

// A operand of the two K steps for query row i (features 32 s + 8 g ..):
// binary16(q * 0.125); rows past T are zeros.
DAV2_DEV void coop_query(const float* qkv, uint32_t b, uint32_t tokens, uint32_t D, uint32_t h, uint32_t i, uint32_t g,
                         h8 (&qa)[2]) {
    const float* q = qkv + (static_cast<uint64_t>(b) * tokens + min(i, tokens - 1u)) * 3u * D + h * 64u + 8u * g;
    const float scale = i < tokens ? 0.125f : 0.0f;
#pragma unroll
    for (int st = 0; st < 2; ++st)
        qa[st] = half8(*reinterpret_cast<const float4*>(q + 32 * st), *reinterpret_cast<const float4*>(q + 32 * st + 4),
                       scale);
}

DAV2_DEV f4v coop_block(const h8 (&qa)[2], const h8 (&kb)[2]) {
    f4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[0], kb[0], acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[1], kb[1], acc, 0, 0, 0);
}

DAV2_DEV uint16_t half_bits(float v) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(keep_fp32(v))); }

// Materialised binary16 scores [batch][H][T][words]: workgroup = 16 queries x
// 64 keys, wave w keys 16 w ..; keys from T on are zeros (so the second half
// of an odd row's last word is 0, as packHalf2x16 writes it).
__global__ __launch_bounds__(256) void ref_scores_coop_kernel(const float* __restrict__ qkv,
                                                              uint16_t* __restrict__ scores, uint32_t tokens,
                                                              uint32_t heads) {
    const uint32_t bh = blockIdx.z, b = bh / heads, h = bh - b * heads;
    const uint32_t D = heads * 64u;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, g = lane >> 4, col = lane & 15u;
    const uint32_t i0 = blockIdx.y * 16u, j = blockIdx.x * 64u + wave * 16u + col;
    h8 qa[2], kb[2];
    coop_query(qkv, b, tokens, D, h, i0 + col, g, qa);
    {
        const float* k = qkv + (static_cast<uint64_t>(b) * tokens + min(j, tokens - 1u)) * 3u * D + D + h * 64u + 8u * g;
        const float one = j < tokens ? 1.0f : 0.0f;
#pragma unroll
        for (int st = 0; st < 2; ++st)
            kb[st] = half8(*reinterpret_cast<const float4*>(k + 32 * st), *reinterpret_cast<const float4*>(k + 32 * st + 4),
                           one);
    }
    const f4v acc = coop_block(qa, kb);
    const uint32_t words = (tokens + 1u) >> 1;
    if (j >= 2u * words) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t i = i0 + 4u * g + r;
        if (i < tokens) scores[(static_cast<uint64_t>(bh) * tokens + i) * 2u * words + j] = half_bits(acc[r]);
    }
}

// ---------------------------------------------------------------------------
// Softmax, in place. The shader's 128 lanes L visit items L, L + 128, ...
// (columns, or packed words in binary16). V = 2: one wave per row, each
// thread holding virtual lanes t and t + 64; V = 1: two waves per row, wave
// half h holding lane t + 64 h (long rows: half the registers per thread).
// A thread keeps up to CH items per virtual lane in registers (CH = 0: the
// row is read again per pass, and the exponentials are stored between the
// passes as the shader does; with the row in registers that intermediate
// store is never observable and is skipped).
// PAIR (V = 2, rows of an even number of items, held in registers): thread t
// holds virtual lanes 2t and 2t + 1 instead, so each access moves two
// adjacent items (8 bytes); the halving tree then splits into one tree per
// parity over the 64 threads (strides 64 .. 2 of the 128 lanes) and the final
// stride-1 sum of the two.
template <int CH, bool HALF, int V, bool PAIR = false>
__global__ __launch_bounds__(256) void ref_softmax_kernel(void* data, uint64_t rows, uint32_t columns) {
    static_assert(V == 1 || V == 2, "virtual lanes per thread");
    static_assert(!PAIR || (V == 2 && CH > 0), "pairs need one wave per row held in registers");
    constexpr uint32_t kRowsPerBlock = 2u * V;  // 4 waves
    __shared__ float exchange[2][2][64];         // [row in block][max | partial][t]
    const uint32_t t = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t slot = V == 2 ? wave : wave >> 1, half = V == 2 ? 0u : wave & 1u;
    const uint64_t row = static_cast<uint64_t>(blockIdx.x) * kRowsPerBlock + slot;
    const bool live = row < rows;  // uniform per wave; both halves of a row agree
    if (V == 2 && !live) return;
    const uint32_t items = HALF ? (columns + 1u) >> 1 : columns;
    float* fr = HALF ? nullptr : static_cast<float*>(data) + (live ? row : 0u) * items;
    uint32_t* wr = HALF ? static_cast<uint32_t*>(data) + (live ? row : 0u) * items : nullptr;
    constexpr int R = CH > 0 ? CH : 1;
    float lo[V][R], hi[V][R];  // hi: the word's upper half (binary16)

    auto load = [&](uint32_t item, float& a, float& b) {
        if (HALF) {
            const uint32_t w = wr[item];
            a = half_lo(w);
            b = half_hi(w);
        } else {
            a = fr[item];
            b = 0.0f;
        }
    };
    // item's value(s) into the running maximum (softmax_lastdim_half.glsl:27-33)
    auto fold_max = [&](float m, uint32_t item, float a, float b) {
        m = fmaxf(m, a);
        if (HALF && item * 2u + 1u < columns) m = fmaxf(m, b);
        return m;
    };
    auto lane_of = [&](int v) {
        return PAIR ? 2u * t + static_cast<uint32_t>(v) : t + 64u * (V == 2 ? static_cast<uint32_t>(v) : half);
    };

    float maximum = -3.402823466e+38f;
    if (PAIR) {
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const uint32_t item = 2u * t + 128u * k;  // even: item + 1 < items too
            if (item < items) {
                if (HALF) {
                    const uint2 w = *reinterpret_cast<const uint2*>(wr + item);
                    lo[0][k] = half_lo(w.x);
                    hi[0][k] = half_hi(w.x);
                    lo[1][k] = half_lo(w.y);
                    hi[1][k] = half_hi(w.y);
                } else {
                    const float2 f = *reinterpret_cast<const float2*>(fr + item);
                    lo[0][k] = f.x;
                    lo[1][k] = f.y;
                    hi[0][k] = hi[1][k] = 0.0f;
                }
                maximum = fold_max(maximum, item, lo[0][k], hi[0][k]);
                maximum = fold_max(maximum, item + 1u, lo[1][k], hi[1][k]);
            }
        }
    } else if (live) {
#pragma unroll
        for (int v = 0; v < V; ++v) {
            const uint32_t lane = lane_of(v);
            if (CH > 0) {
#pragma unroll
                for (int k = 0; k < R; ++k) {
                    const uint32_t item = lane + 128u * k;
                    if (item < items) {
                        load(item, lo[v][k], hi[v][k]);
                        maximum = fold_max(maximum, item, lo[v][k], hi[v][k]);
                    }
                }
            } else {
                for (uint32_t item = lane; item < items; item += 128u) {
                    float a, b;
                    load(item, a, b);
                    maximum = fold_max(maximum, item, a, b);
                }
            }
        }
    }
    maximum = wave_max(maximum);  // order-free
    if (V == 1) {
        if (t == 0) exchange[slot][0][half] = maximum;
        __syncthreads();
        maximum = fmaxf(exchange[slot][0][0], exchange[slot][0][1]);
    }

    // exponentials; per-lane fp32 partials
    float partial[V];
    auto exponentials = [&](uint32_t item, float a, float b, float& ea, float& eb) {
        ea = exp_cw(a - maximum);
        if (HALF) {
            eb = item * 2u + 1u < columns ? exp_cw(b - maximum) : 0.0f;
            if (CH == 0) wr[item] = pack_half2(ea, eb);
            return ea + eb;
        }
        if (CH == 0) fr[item] = ea;
        return ea;
    };
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const uint32_t lane = lane_of(v);
        float d = 0.0f;
        if (live) {
            if (CH > 0) {
#pragma unroll
                for (int k = 0; k < R; ++k) {
                    const uint32_t item = lane + 128u * k;
                    if (item < items) {
                        float ea, eb;
                        d = d + exponentials(item, lo[v][k], hi[v][k], ea, eb);
                        lo[v][k] = ea;
                        hi[v][k] = eb;
                    }
                }
            } else {
                for (uint32_t item = lane; item < items; item += 128u) {
                    float a, b, ea, eb;
                    load(item, a, b);
                    d = d + exponentials(item, a, b, ea, eb);
                }
            }
        }
        partial[v] = d;
    }
    // halving tree over the 128 partials: stride 64 (lane t + lane t + 64),
    // then 32 .. 1 across lanes (lane t adds lane t + stride)
    float sum;
    if (PAIR) {
        sum = wave_sum_tree(partial[0]) + wave_sum_tree(partial[V - 1]);
    } else {
        if (V == 2) {
            sum = partial[0] + partial[V - 1];
        } else {
            if (half == 1) exchange[slot][1][t] = partial[0];
            __syncthreads();
            sum = partial[0] + exchange[slot][1][t];  // meaningful in half 0
        }
        sum = wave_sum_tree(sum);
    }
    if (V == 1) {
        __syncthreads();  // every partial has been read
        if (half == 0 && t == 0) exchange[slot][1][0] = sum;
        __syncthreads();
        sum = exchange[slot][1][0];
    }
    if (!live) return;
    const float inverse = div_rn(1.0f, fmaxf(sum, 1.0e-20f));

    // p = fp16(float(fp16(e)) * inverse) in binary16 (the stored exponentials
    // are fp16(e); pack_half2 keeps the products fp32 until it rounds them)
    auto probability_word = [&](float ea, float eb) {
        const float pa = static_cast<float>(static_cast<_Float16>(ea)) * inverse;
        const float pb = static_cast<float>(static_cast<_Float16>(eb)) * inverse;
        return pack_half2(pa, pb);
    };
    auto normalize = [&](uint32_t item, float ea, float eb) {
        if (HALF) wr[item] = probability_word(ea, eb);
        else fr[item] = ea * inverse;
    };
    if (PAIR) {
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const uint32_t item = 2u * t + 128u * k;
            if (item >= items) continue;
            if (HALF)
                *reinterpret_cast<uint2*>(wr + item) =
                    make_uint2(probability_word(lo[0][k], hi[0][k]), probability_word(lo[1][k], hi[1][k]));
            else
                *reinterpret_cast<float2*>(fr + item) = make_float2(lo[0][k] * inverse, lo[1][k] * inverse);
        }
        return;
    }
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const uint32_t lane = lane_of(v);
        if (CH > 0) {
#pragma unroll
            for (int k = 0; k < R; ++k) {
                const uint32_t item = lane + 128u * k;
                if (item < items) normalize(item, lo[v][k], hi[v][k]);
            }
        } else {
            for (uint32_t item = lane; item < items; item += 128u) {
                float a, b;
                load(item, a, b);  // the stored exponentials
                normalize(item, a, b);
            }
        }
    }
}

// Softmax of long rows, in place: one workgroup of NT threads per row,
// thread t holding items t + NT j (J of them: columns in fp32, packed words
// of two binary16 values with HALF), so that each thread moves few bytes and
// a row's loads are spread over NT / 64 waves (a row held by one or two
// waves keeps too few rows in flight per byte: fp32, T = 1370, 175360 rows:
// 0.59 -> 0.68 of 8 TB/s; T = 5477: 0.51 -> 0.67). The maximum is
// order-free. The shader's sums are not: lane L adds the exponentials of
// items L, L + 128, ... in order (binary16: each word's two exponentials
// added first, softmax_lastdim_half.glsl:48-49), so those per-item terms go
// to LDS and threads 0..127 run the 128 chains from there, then the
// stride-64 step and the in-wave halving tree as in ref_softmax_kernel; the
// exponentials stay in registers for the final products.
template <int NT, int J, bool HALF>
__global__ __launch_bounds__(NT) void ref_softmax_spread_kernel(void* __restrict__ data, uint32_t columns) {
    static_assert(NT % 64 == 0 && NT >= 128, "whole waves, at least the shader's 128 lanes");
    extern __shared__ float terms[];  // [items]
    __shared__ float wave_maxima[NT / 64];
    __shared__ float upper[64];       // lanes 64..127's partial sums
    __shared__ float inverse_lds;
    const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
    const uint32_t items = HALF ? (columns + 1u) >> 1 : columns;
    float* frow = HALF ? nullptr : static_cast<float*>(data) + static_cast<uint64_t>(blockIdx.x) * items;
    uint32_t* wrow = HALF ? static_cast<uint32_t*>(data) + static_cast<uint64_t>(blockIdx.x) * items : nullptr;
    float lo[J], hi[J];  // hi: a word's upper half (binary16)
    const uint32_t last = items - 1u;
    // clamped indices: every load issued before the first use
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t item = min(t + NT * j, last);
        if (HALF) {
            const uint32_t w = wrow[item];
            lo[j] = half_lo(w);
            hi[j] = half_hi(w);
        } else {
            lo[j] = frow[item];
            hi[j] = 0.0f;
        }
    }
    // a word's upper half counts unless it pads an odd row
    auto has_hi = [&](uint32_t item) { return HALF && item * 2u + 1u < columns; };
    float maximum = -3.402823466e+38f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t item = t + NT * j;
        if (item < items) {
            maximum = fmaxf(maximum, lo[j]);
            if (has_hi(item)) maximum = fmaxf(maximum, hi[j]);
        }
    }
    maximum = wave_max(maximum);
    if (lane == 0) wave_maxima[wave] = maximum;
    __syncthreads();
    maximum = wave_maxima[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) maximum = fmaxf(maximum, wave_maxima[w]);
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t item = t + NT * j;
        if (item < items) {
            lo[j] = exp_cw(lo[j] - maximum);
            hi[j] = has_hi(item) ? exp_cw(hi[j] - maximum) : 0.0f;
            terms[item] = HALF ? lo[j] + hi[j] : lo[j];
        }
    }
    __syncthreads();
    float partial = 0.0f;  // lane t's chain (softmax_lastdim.glsl:45-55, _half.glsl:41-50)
    if (t < 128u) {
        for (uint32_t item = t; item < items; item += 128u) partial = partial + terms[item];
        if (t >= 64u) upper[t - 64u] = partial;
    }
    __syncthreads();
    if (t < 64u) {
        const float sum = wave_sum_tree(partial + upper[t]);  // strides 64, then 32 .. 1
        if (t == 0) inverse_lds = div_rn(1.0f, fmaxf(sum, 1.0e-20f));
    }
    __syncthreads();
    const float inverse = inverse_lds;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t item = t + NT * j;
        if (item >= items) continue;
        if (HALF) {
            // p = fp16(float(fp16(e)) * inverse): the stored exponentials are fp16(e)
            const float pa = static_cast<float>(static_cast<_Float16>(lo[j])) * inverse;
            const float pb = static_cast<float>(static_cast<_Float16>(hi[j])) * inverse;
            wrow[item] = pack_half2(pa, pb);
        } else {
            frow[item] = lo[j] * inverse;
        }
    }
}

// ---------------------------------------------------------------------------
// Values. Thread (tx, ty) of 16 x 16 owns queries ty*4 .. +3 and features
// tx*4 .. +3 of a 64 x 64 tile; the source tokens advance in chunks of 32,
// probabilities staged source-major and values (binary16-rounded in that
// pipeline) source-major in LDS.
template <bool HALF>
__global__ __launch_bounds__(256) void ref_values_kernel(float* __restrict__ out, const void* __restrict__ probs,
                                                         const float* __restrict__ qkv, uint32_t tokens,
                                                         uint32_t heads) {
    __shared__ __attribute__((aligned(16))) float ps[kSourceChunk][kValueRows + 4];
    __shared__ __attribute__((aligned(16))) float vs[kSourceChunk][64 + 4];
    const uint32_t bh = blockIdx.z;
    const uint32_t b = bh / heads, h = bh - b * heads;
    const uint32_t D = heads * 64u;
    const uint32_t i0 = blockIdx.x * kValueRows;
    const float* vbase = qkv + static_cast<uint64_t>(b) * tokens * 3u * D + 2u * D + h * 64u;
    const uint64_t plane = static_cast<uint64_t>(bh) * tokens;
    const uint32_t words = (tokens + 1u) >> 1;
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;

    float o[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) o[r][c] = 0.0f;

    for (uint32_t jb = 0; jb < tokens; jb += kSourceChunk) {
        // probabilities: 64 rows x 32 sources (8 per thread), transposed into LDS
#pragma unroll
        for (int it = 0; it < 8; ++it) {
            const int c = tid + it * 256;
            const int r = c >> 5, jj = c & 31;
            const uint32_t i = i0 + r, j = jb + jj;
            float p = 0.0f;
            if (i < tokens && j < tokens) {
                if (HALF) {
                    const uint32_t w = static_cast<const uint32_t*>(probs)[(plane + i) * words + j / 2];
                    p = (j & 1u) ? half_hi(w) : half_lo(w);
                } else {
                    p = static_cast<const float*>(probs)[(plane + i) * tokens + j];
                }
            }
            ps[jj][r] = p;
        }
        // values: 32 sources x 64 features, 2 float4 per thread
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int c = tid + it * 256;
            const int jj = c >> 4, f4 = (c & 15) * 4;
            const uint32_t j = jb + jj;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (j < tokens) v = *reinterpret_cast<const float4*>(vbase + static_cast<uint64_t>(j) * 3u * D + f4);
            if (HALF) {
                v.x = static_cast<float>(static_cast<_Float16>(v.x));
                v.y = static_cast<float>(static_cast<_Float16>(v.y));
                v.z = static_cast<float>(static_cast<_Float16>(v.z));
                v.w = static_cast<float>(static_cast<_Float16>(v.w));
            }
            *reinterpret_cast<float4*>(&vs[jj][f4]) = v;
        }
        __syncthreads();
        const int count = static_cast<int>(min(static_cast<uint32_t>(kSourceChunk), tokens - jb));
        for (int jj = 0; jj < count; ++jj) {
            const float4 pv = *reinterpret_cast<const float4*>(&ps[jj][ty * 4]);
            const float4 vv = *reinterpret_cast<const float4*>(&vs[jj][tx * 4]);
            const float p[4] = {pv.x, pv.y, pv.z, pv.w};
            const float v[4] = {vv.x, vv.y, vv.z, vv.w};
            if (HALF) {
                const h2 v01 = {static_cast<_Float16>(v[0]), static_cast<_Float16>(v[1])};
                const h2 v23 = {static_cast<_Float16>(v[2]), static_cast<_Float16>(v[3])};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const _Float16 ph = static_cast<_Float16>(p[r]);
                    const h2 pp = {ph, ph};
                    add_half_products(o[r][0], o[r][1], pp, v01);
                    add_half_products(o[r][2], o[r][3], pp, v23);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int c = 0; c < 4; ++c) o[r][c] = o[r][c] + p[r] * v[c];
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t i = i0 + ty * 4 + r;
        if (i >= tokens) continue;
        *reinterpret_cast<float4*>(out + (static_cast<uint64_t>(b) * tokens + i) * D + h * 64u + tx * 4) =
            make_float4(o[r][0], o[r][1], o[r][2], o[r][3]);
    }
}

// ---------------------------------------------------------------------------
// The binary16 pipeline fused per block of R query rows: the same arithmetic
// as the three kernels above, and the same bits, without the score round trip
// through memory. A workgroup computes its rows' binary16 scores against every
// key into LDS, runs the softmax on them there and then the value sums.
//
// Keys and values are first rounded to binary16 once (ref16_pack_kernel)
// into chunks of 64 tokens laid out the way the LDS reads want them:
//   keys   chunk c: word (p, kk) = (k[64c+kk][2p], k[64c+kk][2p+1]), p < 32
//   values chunk c: word (q, f)  = (v[64c+2q][f], v[64c+2q+1][f]),   q < 32
// (64 x 32 words = 8 KB each, zero past the last token). One v_pk_mul_f16 on
// a q pair and a key word gives the binary16 products of features 2p and
// 2p+1 of one score, in feature order; on a probability pair and a value word
// the products of keys 2q and 2q+1 of one output, in key order. Each product
// is then added to its fp32 sum by v_fma_mix_f32 (the binary16 half widened
// exactly, times 1.0, plus the sum, one rounding): the shaders'
// sum += float(a16 * b16) at 1.5 VALU instructions per product.
constexpr uint32_t kChunkWords = 32u * 64u;  // one 64-token chunk of keys or values

// acc = acc + float(lo(prod)), one IEEE fp32 addition (the binary16 half
// widened exactly, times 1.0, plus acc: v_fma_mix_f32 rounds once).
DAV2_DEV void add_product_lo(float& acc, uint32_t prod, float one) {
    asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel_hi:[1,0,0]" : "+v"(acc) : "v"(prod), "v"(one));
}
// acc = acc + float(hi(prod))
DAV2_DEV void add_product_hi(float& acc, uint32_t prod, float one) {
    asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(acc) : "v"(prod), "v"(one));
}

// acc[n] = (acc[n] + float(lo(prod[n]))) + float(hi(prod[n])) for N sums;
// the low halves of all N first, so that dependent additions are N apart.
template <int N>
DAV2_DEV void add_product_pairs(float (&acc)[N], const uint32_t (&prod)[N], float one) {
#pragma unroll
    for (int n = 0; n < N; ++n) add_product_lo(acc[n], prod[n], one);
#pragma unroll
    for (int n = 0; n < N; ++n) add_product_hi(acc[n], prod[n], one);
}

DAV2_DEV uint32_t mul_half2(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, a) * __builtin_bit_cast(h2, b));
}

__global__ __launch_bounds__(256) void ref16_pack_kernel(const float* __restrict__ qkv, uint32_t* __restrict__ k16,
                                                         uint32_t* __restrict__ v16, uint32_t tokens, uint32_t heads,
                                                         uint32_t chunks) {
    const uint32_t c = blockIdx.x, bh = blockIdx.y;
    const uint32_t b = bh / heads, h = bh - b * heads;
    const uint32_t D = heads * 64u;
    const float* base = qkv + static_cast<uint64_t>(b) * tokens * 3u * D + h * 64u;
    const uint32_t lane = threadIdx.x & 63u, part = threadIdx.x >> 6;
    const uint64_t chunk = (static_cast<uint64_t>(bh) * chunks + c) * kChunkWords;
    // keys: lane = token of the chunk, part = features 16*part .. +15
    const uint32_t j = c * 64u + lane;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (j < tokens)
            v = *reinterpret_cast<const float4*>(base + static_cast<uint64_t>(j) * 3u * D + D + 16u * part + 4u * i);
        const uint32_t p = 8u * part + 2u * i;
        k16[chunk + p * 64u + lane] = pack_half2(v.x, v.y);
        k16[chunk + (p + 1u) * 64u + lane] = pack_half2(v.z, v.w);
    }
    // values: lane = feature, part = token pairs 8*part .. +7
    const float* vb = base + 2u * D + lane;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t q = 8u * part + i, j0 = c * 64u + 2u * q;
        const float lo = j0 < tokens ? vb[static_cast<uint64_t>(j0) * 3u * D] : 0.0f;
        const float hi = j0 + 1u < tokens ? vb[static_cast<uint64_t>(j0 + 1u) * 3u * D] : 0.0f;
        v16[chunk + q * 64u + lane] = pack_half2(lo, hi);
    }
}

// R query rows per workgroup of 256 threads; thread t owns row t % R and, of
// each 64-token chunk, keys (for the scores) or features (for the values)
// G*(t / R) .. +G-1, G = R / 4. LDS: the chunk buffer (8 KB), then the rows'
// binary16 scores / probabilities, `stride` words per row (4 more than a
// multiple of 32, so the 16 rows' 16-byte reads fall on different banks).
// At T = 1370 that is 53.5 KB: three workgroups per CU.
template <int R, bool COOP>
__global__ __launch_bounds__(256) void ref16_fused_kernel(float* __restrict__ out, const float* __restrict__ qkv,
                                                          const uint32_t* __restrict__ k16,
                                                          const uint32_t* __restrict__ v16, uint32_t tokens,
                                                          uint32_t heads, uint32_t chunks, uint32_t row_blocks,
                                                          uint32_t stride) {
    constexpr int G = R / 4;  // keys or features per thread and chunk
    static_assert(G == 2 || G == 4, "two or four keys per thread");
    typedef uint32_t wordsG __attribute__((ext_vector_type(G)));
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    uint32_t* const kv = lds;                 // [kChunkWords]
    uint32_t* const srows = lds + kChunkWords;  // [R][stride]

    // XCD-banded order: workgroup L runs on XCD L % 8, and each XCD takes a
    // contiguous range of (head, row block) items, so a head's keys and
    // values stay in one L2.
    const uint32_t L = blockIdx.x, n = gridDim.x;
    const uint32_t xcd = L & 7u, per = n >> 3, extra = n & 7u;
    const uint32_t work = xcd * per + min(xcd, extra) + (L >> 3);
    const uint32_t bh = work / row_blocks, rb = work - bh * row_blocks;
    const uint32_t b = bh / heads, h = bh - b * heads;
    const uint32_t D = heads * 64u;
    const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63u;
    const uint32_t r = t % R, grp = t / R;
    const uint32_t i = rb * R + r;
    const uint32_t* kbase = k16 + static_cast<uint64_t>(bh) * chunks * kChunkWords;
    const uint32_t* vbase = v16 + static_cast<uint64_t>(bh) * chunks * kChunkWords;
    const float one = 1.0f;

    // Chunks go through registers: chunk c + 1 is loaded (two 16-byte loads
    // per thread) while chunk c is multiplied, and written to the buffer once
    // every wave is done with chunk c. (Copies straight into LDS would make
    // the compiler wait for them before every LDS read of the loop.)
    uint4 staged0, staged1;
    auto fetch = [t](const uint32_t* src, uint32_t c, uint4& a, uint4& b) {
        const uint4* s0 = reinterpret_cast<const uint4*>(src + static_cast<uint64_t>(c) * kChunkWords);
        a = s0[t];
        b = s0[t + 256u];
    };
    auto put = [t, kv](const uint4& a, const uint4& b) {
        uint4* d = reinterpret_cast<uint4*>(kv);
        d[t] = a;
        d[t + 256u] = b;
    };
    auto next_chunk = [&](uint32_t c) {
        if (c + 1u < chunks) {
            __syncthreads();  // every wave is done with chunk c
            put(staged0, staged1);
            __syncthreads();
        }
    };

    fetch(kbase, 0, staged0, staged1);
    // q row i as binary16 pairs of q * 0.125 (bmm_score_fp16.glsl:32); rows
    // past T compute on zeros and are never stored. Cooperative-matrix
    // scores: the MFMA A operand of query row rb*16 + l%16 instead.
    uint32_t qp[COOP ? 1 : 32];
    h8 qa[2];
    if constexpr (COOP) {
        static_assert(R == 16, "one 16-row MFMA block of queries");
        coop_query(qkv, b, tokens, D, h, rb * R + (lane & 15u), lane >> 4, qa);
    } else {
        const float* q = qkv + (static_cast<uint64_t>(b) * tokens + min(i, tokens - 1u)) * 3u * D + h * 64u;
        float4 v[16];
#pragma unroll
        for (int f4 = 0; f4 < 16; ++f4) v[f4] = *reinterpret_cast<const float4*>(q + 4 * f4);
        const float scale = i < tokens ? 0.125f : 0.0f;
#pragma unroll
        for (int f4 = 0; f4 < 16; ++f4) {
            qp[2 * f4] = pack_half2(v[f4].x * scale, v[f4].y * scale);
            qp[2 * f4 + 1] = pack_half2(v[f4].z * scale, v[f4].w * scale);
        }
    }

    put(staged0, staged1);
    __syncthreads();

    if constexpr (COOP) {
        // bmm_score_coop_fp16.glsl: wave w scores keys 16w .. 16w+15 of each
        // chunk for the 16 rows; B operand words (16 st + 4 g + e, key) of
        // the chunk buffer are features 32 st + 8 g + 2e, +1. Each result is
        // stored as one binary16 half of its row's packed word.
        uint16_t* const halves = reinterpret_cast<uint16_t*>(srows);
        const uint32_t key = 16u * wave + (lane & 15u), g = lane >> 4;
        for (uint32_t c = 0; c < chunks; ++c) {
            if (c + 1u < chunks) fetch(kbase, c + 1u, staged0, staged1);
            h8 kb[2];
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                const uint32_t* w = kv + (16u * st + 4u * g) * 64u + key;
                kb[st] = __builtin_bit_cast(h8, make_uint4(w[0], w[64], w[128], w[192]));
            }
            const f4v acc = coop_block(qa, kb);
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
                halves[((4u * g + rr) * stride + 32u * c) * 2u + key] = half_bits(acc[rr]);
            next_chunk(c);
        }
    }
    // scores: s = sum over features 0..63 of float(q16 * k16), stored binary16
    uint32_t* const myrow = srows + r * stride;
    for (uint32_t c = 0; !COOP && c < chunks; ++c) {
        if (c + 1u < chunks) fetch(kbase, c + 1u, staged0, staged1);
        const uint32_t* kc = kv + grp * G;
        float acc[G];
#pragma unroll
        for (int kk = 0; kk < G; ++kk) acc[kk] = 0.0f;
#pragma unroll
        for (int p = 0; p < 32; ++p) {
            const wordsG kw = *reinterpret_cast<const wordsG*>(kc + p * 64);
            uint32_t prod[G];
#pragma unroll
            for (int kk = 0; kk < G; ++kk) prod[kk] = mul_half2(qp[p], kw[kk]);
            add_product_pairs(acc, prod, one);
        }
        // keys 64c + G*grp + kk -> words 32c + G*grp/2 + kk/2 (packHalf2x16)
        if (G == 4) {
            *reinterpret_cast<uint2*>(myrow + 32u * c + 2u * grp) =
                make_uint2(pack_half2(acc[0], acc[1]), pack_half2(acc[G - 2], acc[G - 1]));
        } else {
            myrow[32u * c + grp] = pack_half2(acc[0], acc[1]);
        }
        next_chunk(c);
    }
    __syncthreads();  // every row's scores are in LDS; the chunk buffer is free

    // the first value chunk arrives during the softmax
    fetch(vbase, 0, staged0, staged1);

    // softmax_lastdim_half.glsl:19-65 on each row: the maximum; e = exp(s -
    // max) stored binary16 while virtual lane L (words L, L + 128, ...; lane
    // holds L and L + 64) sums (e.x + e.y) in fp32; the 128 partials by the
    // halving tree; p = binary16(float(binary16(e)) * (1 / max(sum, 1e-20))).
    const uint32_t words = (tokens + 1u) >> 1;
    for (uint32_t rr = wave; rr < static_cast<uint32_t>(R); rr += 4u) {
        uint32_t* row = srows + rr * stride;
        float maximum = -3.402823466e+38f;
        for (uint32_t w = lane; w < words; w += 64u) {
            const uint32_t pair = row[w];
            maximum = fmaxf(maximum, half_lo(pair));
            if (2u * w + 1u < tokens) maximum = fmaxf(maximum, half_hi(pair));
        }
        maximum = wave_max(maximum);
        float partial[2];
#pragma unroll
        for (uint32_t v = 0; v < 2; ++v) {
            float d = 0.0f;
            for (uint32_t w = lane + 64u * v; w < words; w += 128u) {
                const uint32_t pair = row[w];
                const float ea = exp_cw(half_lo(pair) - maximum);
                const float eb = 2u * w + 1u < tokens ? exp_cw(half_hi(pair) - maximum) : 0.0f;
                row[w] = pack_half2(ea, eb);
                d = d + (ea + eb);
            }
            partial[v] = d;
        }
        const float sum = wave_sum_tree(partial[0] + partial[1]);
        const float inverse = div_rn(1.0f, fmaxf(sum, 1.0e-20f));
        for (uint32_t w = lane; w < words; w += 64u) {
            const uint32_t pair = row[w];
            row[w] = pack_half2(half_lo(pair) * inverse, half_hi(pair) * inverse);
        }
    }

    // values: out = sum over tokens 0..T-1 of float(p16 * v16), in order
    float acc[G];
#pragma unroll
    for (int f = 0; f < G; ++f) acc[f] = 0.0f;
    put(staged0, staged1);
    __syncthreads();  // every row's probabilities and the first value chunk are in LDS
    for (uint32_t c = 0; c < chunks; ++c) {
        if (c + 1u < chunks) fetch(vbase, c + 1u, staged0, staged1);
        const uint32_t* vc = kv + grp * G;
        const uint32_t* pc = myrow + 32u * c;
        if (64u * c + 64u <= tokens) {
#pragma unroll 2
            for (int q4 = 0; q4 < 32; q4 += 4) {
                const uint4 pw = *reinterpret_cast<const uint4*>(pc + q4);
                const uint32_t pq[4] = {pw.x, pw.y, pw.z, pw.w};
#pragma unroll
                for (int qq = 0; qq < 4; ++qq) {
                    const wordsG vw = *reinterpret_cast<const wordsG*>(vc + (q4 + qq) * 64);
                    uint32_t prod[G];
#pragma unroll
                    for (int f = 0; f < G; ++f) prod[f] = mul_half2(pq[qq], vw[f]);
                    add_product_pairs(acc, prod, one);
                }
            }
        } else {
            // the last, partial chunk: tokens 64c .. T-1 only
            const uint32_t left = tokens - 64u * c;
            for (uint32_t q = 0; 2u * q < left; ++q) {
                const uint32_t pw = pc[q];
                const wordsG vw = *reinterpret_cast<const wordsG*>(vc + q * 64u);
                if (2u * q + 1u < left) {
                    uint32_t prod[G];
#pragma unroll
                    for (int f = 0; f < G; ++f) prod[f] = mul_half2(pw, vw[f]);
                    add_product_pairs(acc, prod, one);
                } else {
#pragma unroll
                    for (int f = 0; f < G; ++f) acc[f] = acc[f] + half_lo(mul_half2(pw, vw[f]));
                }
            }
        }
        next_chunk(c);
    }
    if (i < tokens) {
        float* o = out + (static_cast<uint64_t>(b) * tokens + i) * D + h * 64u + grp * G;
        if (G == 4)
            *reinterpret_cast<float4*>(o) = make_float4(acc[0], acc[1], acc[G - 2], acc[G - 1]);
        else
            *reinterpret_cast<float2*>(o) = make_float2(acc[0], acc[1]);
    }
}

uint32_t ref16_chunks(uint32_t tokens) { return (tokens + 63u) / 64u; }

// The fused kernel runs 16 query rows per workgroup while at least two
// workgroups fit a CU's 160 KB of LDS (T up to 2240; three at T = 1370).
// Longer rows would leave one workgroup per CU, slower than the three
// materialised kernels (measured at T = 5477), which serve them instead.
constexpr int kRef16Rows = 16;
struct Ref16Shape {
    uint32_t stride;  // words per score row
    uint32_t lds;     // bytes, 0: T too long for the fused kernel
};

Ref16Shape ref16_shape(uint32_t tokens) {
    const uint32_t stride = ref16_chunks(tokens) * 32u + 4u;
    const uint32_t lds = kChunkWords * 4u + kRef16Rows * stride * 4u;
    return {stride, lds <= 80u * 1024u ? lds : 0u};
}

template <bool HALF>
hipError_t launch_softmax(void* data, uint64_t rows, uint32_t columns, hipStream_t s) {
    const uint32_t items = HALF ? (columns + 1u) >> 1 : columns;
    const uint32_t per_lane = (items + 127u) / 128u;
    const dim3 grid(static_cast<uint32_t>((rows + 3u) / 4u)), grid2(static_cast<uint32_t>((rows + 1u) / 2u)),
        block(256);
    // rows of up to 12 items per lane: one wave per row; longer ones: two
    // (rows of an even number of items on an 8-byte aligned buffer: pairs
    // of adjacent items per thread)
    const bool pairs = items % 2u == 0u && (reinterpret_cast<uintptr_t>(data) & 7u) == 0u;
    // Rows of 961 .. 11264 fp32 columns or 1537 .. 5632 binary16 words: a
    // workgroup per row (256 threads up to 3072 items, 512 beyond; measured
    // best at 1370 and 5477). Fraction of 8 TB/s against the kernels below,
    // fp32 rows of 1000 / 1370 / 2000 / 5477 / 8000 items: 0.72 / 0.72 / 0.69
    // / 0.67 / 0.66 against 0.62 / 0.60 / 0.48 / 0.51 / 0.23 (rows of 300-700
    // items measured faster below); binary16 rows of 2739 / 3100 / 5500
    // words: 0.60 / 0.51 / 0.64 against 0.31 / 0.26 / 0.27 (1000 words: 0.50
    // against 0.57 below).
    if (items > (HALF ? 1536u : 960u) && items <= (HALF ? 5632u : 11264u) && rows <= 0x7fffffffu) {
        const dim3 one_row(static_cast<uint32_t>(rows));
        const size_t lds = static_cast<size_t>(items) * sizeof(float);
        if (items <= 1024u) dispatch((ref_softmax_spread_kernel<256, 4, HALF>), one_row, dim3(256), lds, s, data, columns);
        else if (items <= 1536u) dispatch((ref_softmax_spread_kernel<256, 6, HALF>), one_row, dim3(256), lds, s, data, columns);
        else if (items <= 3072u) dispatch((ref_softmax_spread_kernel<256, 12, HALF>), one_row, dim3(256), lds, s, data, columns);
        else if (items <= 5632u) dispatch((ref_softmax_spread_kernel<512, 11, HALF>), one_row, dim3(512), lds, s, data, columns);
        else dispatch((ref_softmax_spread_kernel<512, 22, HALF>), one_row, dim3(512), lds, s, data, columns);
        return hipGetLastError();
    }
#define DAV2_SOFTMAX_CASE(N, V)                                                                     \
    if (per_lane <= N) {                                                                               \
        if (V == 2 && pairs)                                                                           \
            dispatch((ref_softmax_kernel<N, HALF, V, V == 2>), grid, block, 0, s, data, rows, columns); \
        else                                                                                           \
            dispatch((ref_softmax_kernel<N, HALF, V>), V == 2 ? grid : grid2, block, 0, s, data, rows, columns); \
        return hipGetLastError();                                                                      \
    }
    DAV2_SOFTMAX_CASE(4, 2)
    DAV2_SOFTMAX_CASE(8, 2)
    DAV2_SOFTMAX_CASE(12, 2)
    DAV2_SOFTMAX_CASE(24, 1)
    DAV2_SOFTMAX_CASE(48, 1)
#undef DAV2_SOFTMAX_CASE
    dispatch((ref_softmax_kernel<0, HALF, 2>), grid, block, 0, s, data, rows, columns);
    return hipGetLastError();
}

bool valid(uint32_t tokens, uint32_t heads, uint32_t batch) {
    return tokens > 0 && heads > 0 && batch > 0 && uint64_t(batch) * heads <= 65535u;
}

}  // namespace

extern "C" {

uint64_t dav2_hip_attention_ref_scratch_bytes(uint32_t tokens, uint32_t heads, uint32_t batch, int fp16) {
    const uint64_t planes = static_cast<uint64_t>(batch) * heads * tokens;
    return fp16 ? planes * ((tokens + 1u) / 2u) * 4u : planes * tokens * 4u;
}

int dav2_hip_attention_ref_scores(void* scores, const float* qkv, uint32_t tokens, uint32_t heads, uint32_t batch,
                                  int fp16, void* stream) {
    if (!scores || !qkv || !valid(tokens, heads, batch)) return hipErrorInvalidValue;
    if (reinterpret_cast<uintptr_t>(qkv) & 15) return hipErrorInvalidValue;
    const dim3 grid(ceil_div(tokens, kKeyTile), ceil_div(tokens, kQueryTile), batch * heads);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (fp16)
        dispatch(ref_scores_kernel<true>, grid, dim3(256), 0, s, qkv, scores, tokens, heads);
    else
        dispatch(ref_scores_kernel<false>, grid, dim3(256), 0, s, qkv, scores, tokens, heads);
    return hipGetLastError();
}

int dav2_hip_attention_ref_softmax(void* scores, uint64_t rows, uint32_t columns, int fp16, void* stream) {
    if (!scores || columns == 0) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    hipStream_t s = static_cast<hipStream_t>(stream);
    return fp16 ? launch_softmax<true>(scores, rows, columns, s) : launch_softmax<false>(scores, rows, columns, s);
}

uint64_t dav2_hip_attention_ref16_fused_scratch_bytes(uint32_t tokens, uint32_t heads, uint32_t batch) {
    if (ref16_shape(tokens).lds == 0) return 0;
    return 2ull * batch * heads * ref16_chunks(tokens) * kChunkWords * 4u;
}

}  // extern "C"

namespace {

template <bool COOP>
int run_ref16_fused(float* out, const float* qkv, uint32_t tokens, uint32_t heads, uint32_t batch, void* scratch,
                    uint64_t scratch_bytes, void* stream) {
    if (!out || !qkv || !scratch || !valid(tokens, heads, batch)) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(scratch)) &
        15)
        return hipErrorInvalidValue;
    const Ref16Shape shape = ref16_shape(tokens);
    const uint64_t need = dav2_hip_attention_ref16_fused_scratch_bytes(tokens, heads, batch);
    if (shape.lds == 0 || scratch_bytes < need) return hipErrorInvalidValue;
    const uint32_t chunks = ref16_chunks(tokens), bh = batch * heads;
    const uint32_t row_blocks = (tokens + kRef16Rows - 1u) / kRef16Rows;
    const uint64_t items = static_cast<uint64_t>(row_blocks) * bh;
    if (items > 0x7fffffffull) return hipErrorInvalidValue;
    uint32_t* k16 = static_cast<uint32_t*>(scratch);
    uint32_t* v16 = k16 + static_cast<uint64_t>(bh) * chunks * kChunkWords;
    hipStream_t s = static_cast<hipStream_t>(stream);
    dispatch(ref16_pack_kernel, dim3(chunks, bh), dim3(256), 0, s, qkv, k16, v16, tokens, heads, chunks);
    static const hipError_t lds_ok =
        hipFuncSetAttribute(reinterpret_cast<const void*>(ref16_fused_kernel<kRef16Rows, COOP>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(80u * 1024u));
    if (lds_ok != hipSuccess) return lds_ok;
    dispatch((ref16_fused_kernel<kRef16Rows, COOP>), dim3(static_cast<uint32_t>(items)), dim3(256), shape.lds, s, out,
             qkv, k16, v16, tokens, heads, chunks, row_blocks, shape.stride);
    return hipGetLastError();
}

}  // namespace

extern "C" {

int dav2_hip_attention_ref16_fused(float* out, const float* qkv, uint32_t tokens, uint32_t heads, uint32_t batch,
                                   void* scratch, uint64_t scratch_bytes, void* stream) {
    return run_ref16_fused<false>(out, qkv, tokens, heads, batch, scratch, scratch_bytes, stream);
}

int dav2_hip_attention_ref16_fused_coop(float* out, const float* qkv, uint32_t tokens, uint32_t heads,
                                        uint32_t batch, void* scratch, uint64_t scratch_bytes, void* stream) {
    return run_ref16_fused<true>(out, qkv, tokens, heads, batch, scratch, scratch_bytes, stream);
}

int dav2_hip_attention_ref_scores_coop(void* scores, const float* qkv, uint32_t tokens, uint32_t heads,
                                       uint32_t batch, void* stream) {
    if (!scores || !qkv || !valid(tokens, heads, batch)) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(qkv) & 15) || (reinterpret_cast<uintptr_t>(scores) & 1)) return hipErrorInvalidValue;
    const dim3 grid(ceil_div(tokens, 64), ceil_div(tokens, 16), batch * heads);
    dispatch(ref_scores_coop_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), qkv,
             static_cast<uint16_t*>(scores), tokens, heads);
    return hipGetLastError();
}

int dav2_hip_attention_ref_values(float* out, const void* probabilities, const float* qkv, uint32_t tokens,
                                  uint32_t heads, uint32_t batch, int fp16, void* stream) {
    if (!out || !probabilities || !qkv || !valid(tokens, heads, batch)) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(out)) & 15) return hipErrorInvalidValue;
    const dim3 grid(ceil_div(tokens, kValueRows), 1, batch * heads);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (fp16)
        dispatch(ref_values_kernel<true>, grid, dim3(256), 0, s, out, probabilities, qkv, tokens, heads);
    else
        dispatch(ref_values_kernel<false>, grid, dim3(256), 0, s, out, probabilities, qkv, tokens, heads);
    return hipGetLastError();
}

}  // extern "C"
