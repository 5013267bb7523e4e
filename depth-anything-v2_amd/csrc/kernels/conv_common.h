// Shared pieces of the implicit-GEMM int8 convolution kernels (conv_i8.hip:
// 1x1 and the reference-order helpers; conv3x3_i8.hip: 3x3).
#pragma once

#include <type_traits>

#include "common.h"
#include "dav2_hip.h"

namespace dav2k {

constexpr int kPix = 64;  // output pixels per workgroup
constexpr int kCB = 64;   // input channels per block = one MFMA K step per tap

// Packed weights: the [N][taps * C] int8 matrix with K walked tap-major
// (k = tap * C + c), cut into the MFMA's 16-row x 64-byte operand fragments,
// each stored as the 1 KiB a wave loads for it (lane l: row l % 16, K bytes
// 16 (l / 16) .. + 15), fragment (16-row block nb, K step ks) at byte
// (nb * ksteps + ks) * 1024, ksteps = taps * C / 64. One coalesced 16-byte
// load per lane fetches a fragment (dav2_hip_conv_weights_pack).
struct ConvParams {
    const float* x;        // CHW input
    const float* partial;  // [groups][plane] channel-group |x| maxima
    uint32_t groups;
    uint32_t channels, height, width;
    uint64_t plane;
    uint32_t tiles_x;      // 3x3: pixel tiles per image row
    const int8_t* w;       // packed weights (below)
    uint32_t n_out;        // N
    const float* w_scales;
    const float* bias;     // nullable
    float* out;            // CHW [N][plane]
    const float* residual; // nullable, CHW [N][plane]
    uint32_t flags;        // DAV2_CONV_*
    float* emit;           // channel-group maxima of the output (EMIT flags), [N/32][plane]
};

// Geometry of the 3x3 kernel's tiles: two image rows of kTileCols3 output
// pixels (conv3x3_i8.hip).
constexpr int kTileCols3 = 60;

// Workgroup barrier that orders LDS only: waits for this wave's LDS
// operations (lgkmcnt) but leaves global loads in flight.
DAV2_DEV void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// rne(clamp(v * inv, -127, 127)) of four values packed little-endian, for
// |v| <= absmax of the row and inv = 1 / max(absmax / 127, 1e-8): then
// |v * inv| <= 127 * (1 + 3 * 2^-24) < 127.5 (or below 127 under the 1e-8
// floor), so rounding alone lands in [-127, 127] and the clamp never acts.
// Adding 1.5 * 2^23 rounds to an integer (round to nearest even, the ulp
// there is 1) held in the low mantissa bits, so the low byte of the sum is the
// two's-complement int8; v_perm gathers the bytes. (Finite inputs: the
// reference leaves NaN and infinity to the shader's clamp.)
DAV2_DEV uint32_t quant4(float a, float b, float c, float d, float inv) {
    constexpr float kMagic = 12582912.0f;
    const uint32_t qa = __float_as_uint(a * inv + kMagic);
    const uint32_t qb = __float_as_uint(b * inv + kMagic);
    const uint32_t qc = __float_as_uint(c * inv + kMagic);
    const uint32_t qd = __float_as_uint(d * inv + kMagic);
    const uint32_t lo = __builtin_amdgcn_perm(qb, qa, 0x00000400u);  // bytes: a, b, a, a
    const uint32_t hi = __builtin_amdgcn_perm(qd, qc, 0x00000400u);  // bytes: c, d, c, c
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);               // bytes: a, b, c, d
}

// LDS byte offset of 16-byte chunk c (0..3) of pixel row p in a 64 x 64-byte
// int8 tile: rows are 64 bytes, chunks XOR-swizzled by (p / 4) % 4 so the 16
// rows one MFMA operand read touches cover all banks once.
DAV2_DEV uint32_t a_offset(uint32_t p, uint32_t c) { return p * 64u + ((c ^ ((p >> 2) & 3u)) << 4); }

// Epilogue of the implicit-GEMM kernels: out[ch][pixel] =
// ((acc * s_pixel) * s_weight) + bias, then + residual (add.glsl) and
// max(., 0) (relu.glsl) when asked; the flag tests sit outside the unrolled
// store loops. Accumulator r of lane l in block (i, j): channel
// 16i + 4(l/16) + r, pixel 16j + l%16 of the wave's sub-tile. With an EMIT
// flag the tile's channel-group maxima of the output (the next
// convolution's row scales) are written too: the channels of a group are
// 16-channel blocks i of this lane (rows 4(l/16) + r) and of lanes l^16,
// l^32, l^48.
template <int BN, int WM, int WN, int PIX, typename Locate>
DAV2_DEV void store_tile(const ConvParams& g, const v4i (&acc)[BN / WN / 16][PIX / WM / 16], uint32_t wm,
                         uint32_t wn, uint32_t lane, uint32_t nb, const float* sc_lds, const float* wsc_lds,
                         const float* bias_lds, Locate locate) {
    constexpr int PW = PIX / WM, NW = BN / WN, PB = PW / 16, NB = NW / 16;
    constexpr int kEmitGroups = (NW % 32 == 0) ? NW / 32 : 0;
    const bool emit_relu = (g.flags & DAV2_CONV_EMIT_RELU_MAX) != 0;
    float gmax[PB][kEmitGroups > 0 ? kEmitGroups : 1];
#pragma unroll
    for (int j = 0; j < PB; ++j)
#pragma unroll
        for (int q = 0; q < (kEmitGroups > 0 ? kEmitGroups : 1); ++q) gmax[j][q] = 0.0f;
    auto epilogue = [&](auto residual_tag, auto relu_tag) {
        constexpr bool kResidual = decltype(residual_tag)::value, kRelu = decltype(relu_tag)::value;
        // The residual of pixel block j + 1 is loaded while block j is
        // stored (one round trip per two blocks instead of one per block);
        // pixels outside the map load pixel 0 (never stored).
        float res[2][kResidual ? NB : 1][4];
        auto load_res = [&](int j, float (&dst)[kResidual ? NB : 1][4]) {
            uint64_t pixel;
            if (!locate(wm * PW + 16u * j + (lane & 15u), pixel)) pixel = 0;
#pragma unroll
            for (int i = 0; i < NB; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t cl = wn * NW + 16u * i + 4u * (lane >> 4) + r;
                    dst[i][r] = g.residual[static_cast<uint64_t>(nb * BN + cl) * g.plane + pixel];
                }
        };
        if constexpr (kResidual) load_res(0, res[0]);
#pragma unroll
        for (int j = 0; j < PB; ++j) {
            if constexpr (kResidual)
                if (j + 1 < PB) load_res(j + 1, res[(j + 1) & 1]);
            const uint32_t p = wm * PW + 16u * j + (lane & 15u);
            uint64_t pixel;
            if (!locate(p, pixel)) continue;
            const float sp = sc_lds[p];
#pragma unroll
            for (int i = 0; i < NB; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t cl = wn * NW + 16u * i + 4u * (lane >> 4) + r;
                    float v = static_cast<float>(acc[i][j][r]);
                    v = v * sp;
                    v = v * wsc_lds[cl];
                    v = v + bias_lds[cl];
                    const uint64_t idx = static_cast<uint64_t>(nb * BN + cl) * g.plane + pixel;
                    if constexpr (kResidual) v = v + res[j & 1][i][r];
                    if (kRelu) v = fmaxf(v, 0.0f);
                    g.out[idx] = v;
                    if constexpr (kEmitGroups > 0) {
                        const float m = emit_relu ? fmaxf(v, 0.0f) : fabsf(v);
                        gmax[j][(16 * i) / 32] = fmaxf(gmax[j][(16 * i) / 32], m);
                    }
                }
        }
    };
    const bool relu_out = (g.flags & DAV2_CONV_RELU_OUTPUT) != 0;
    if (g.residual) {
        if (relu_out) epilogue(std::true_type{}, std::true_type{});
        else epilogue(std::true_type{}, std::false_type{});
    } else {
        if (relu_out) epilogue(std::false_type{}, std::true_type{});
        else epilogue(std::false_type{}, std::false_type{});
    }
    if constexpr (kEmitGroups > 0) {
        if (g.emit) {
#pragma unroll
            for (int j = 0; j < PB; ++j) {
                const uint32_t p = wm * PW + 16u * j + (lane & 15u);
                uint64_t pixel;
                const bool ok = locate(p, pixel);
#pragma unroll
                for (int q = 0; q < kEmitGroups; ++q) {
                    float m = gmax[j][q];
                    m = fmaxf(m, __shfl_xor(m, 16, kWave));
                    m = fmaxf(m, __shfl_xor(m, 32, kWave));
                    const uint32_t group = (nb * BN + wn * NW) / 32u + q;
                    if (lane < 16u && ok) g.emit[static_cast<uint64_t>(group) * g.plane + pixel] = m;
                }
            }
        }
    }
}

// Launches the 3x3 kernel (conv3x3_i8.hip) over `tiles` pixel tiles and
// n / BN channel tiles; g.tiles_x = ceil(width / kTileCols3).
hipError_t launch_conv3x3_i8(const ConvParams& g, uint32_t tiles, uint32_t n, hipStream_t s);

}  // namespace dav2k
