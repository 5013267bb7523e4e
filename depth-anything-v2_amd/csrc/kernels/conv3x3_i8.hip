// 3x3 (stride 1, padding 1) implicit-GEMM int8 convolution: the reference's
// conv2d_int8 (src/operators.cpp:1735-1805: im2col_quantize_int8.glsl:26-83
// then linear_int8_tiled.glsl:40-117 with the CHW store) in one kernel, with
// the same arithmetic as conv_i8.hip: im2col row p quantized with
// s = max(absmax/127, 1e-8) of the whole row, q = rne(x * (1/s)), exact int32
// dot products walked tap-major (k = tap * C + c), the GEMM's CHW epilogue
// ((float(acc) * s_pixel) * s_weight) + bias. Every output float equals the
// im2col + GEMM path's bit for bit.
//
// Tiling. A workgroup (4 waves, one per SIMD, one workgroup per CU) owns a
// tile of two image rows x 60 output columns and BN output channels. Window
// column w of the tile is image column x0 - 2 + w (w = 0..63); the tile's 128
// pixel slots are (row i, column j), slots j = 60..63 computed but never
// stored.
//
// Per block of 64 input channels the operand tile is the block's
// 128 x (9 x 64) slice of the im2col matrix, stored [tap][pixel][64 bytes]
// (XOR-swizzled 16-byte chunks) and double-buffered in LDS (2 x 72 KiB).
// While the waves multiply block b's tile (v_mfma_i32_16x16x64_i8, weights as
// the row operand so each lane's accumulators run along pixels and the CHW
// stores coalesce), they quantize block b + 1's into the other buffer, two
// pieces per tap, so the quantizer's VALU work issues between the MFMAs and
// there is one barrier per block of nine K steps. A wave's tile of 128 pixels
// (or 64 when two waves split the pixels) reads each weight fragment once per
// 8 (or 4) pixel blocks, and the packed fragments are one contiguous 1 KiB
// load each.
//
// Quantizer. Wave v quantizes channels 16v .. 16v + 15 of the block; lane l
// owns window columns 2 (l / 2) and 2 (l / 2) + 1 and channels
// 16v + 8 (l % 2) .. + 7. It loads them from the four window rows (image
// rows y0 - 1 .. y0 + 2) with 8-byte raw buffer loads into registers, one
// block ahead (32 loads per block, well inside the wave's 63 outstanding
// loads); positions outside the image get an offset past the buffer's range,
// which reads as zero (the padding). Window row wr is tap row dy = wr - i of
// pixel row i, window column w is tap column dx of pixel column w - 1 - dx:
// each value is quantized with the scales of up to six pixels (twelve
// inverse scales per lane, fixed for the kernel), 18 pieces per block.
//
// Needs an even width and an 8-byte aligned input (conv_i8.hip's kernel
// takes the other maps).

#include <algorithm>

#include "common.h"
#include "conv_common.h"
#include "dav2_hip.h"

using namespace dav2k;

namespace {

constexpr int kTaps = 9;
constexpr int kPixT = 128;                             // pixel slots per tile (2 x 64)
constexpr uint32_t kTapBytes = kPixT * 64u;            // one tap's operand tile
constexpr uint32_t kBufBytes = kTaps * kTapBytes;      // one block's operand tile
constexpr uint32_t kOutside = 0x80000000u;             // buffer offset past every block's range

typedef float v2f __attribute__((ext_vector_type(2)));

// LDS byte offset of 16-byte chunk c (0..3) of pixel slot r (0..127) in one
// tap's operand tile: rows of 64 bytes, row r stored at r ^ bit 2 of r, the
// chunk XOR-ed with bits 3 and 2 ^ 4 of r. Then the 16 rows one MFMA
// operand read takes (16-aligned, one chunk) cover all 64 banks once, and so
// do the 8-byte quantizer writes of 32 lanes (16 rows two apart, both
// halves of a chunk).
DAV2_DEV uint32_t tile_offset(uint32_t r, uint32_t c) {
    const uint32_t phys = r ^ ((r >> 2) & 1u);
    const uint32_t sw = ((r >> 3) & 1u) | ((((r >> 2) ^ (r >> 4)) & 1u) << 1);
    return phys * 64u + ((c ^ sw) << 4);
}
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

// Piece k of a block's quantization: window row, pixel row (tap column
// dx = k % 3). Rows are finished in order (row 0 after piece 2, row 1 after
// 8, row 2 after 14, row 3 after 17) so their registers can be refilled.
constexpr int piece_row(int k) { return k < 3 ? 0 : (k < 9 ? 1 : (k < 15 ? 2 : 3)); }
constexpr int piece_pixel_row(int k) { return (k < 3) ? 0 : (k < 6 ? 0 : (k < 9 ? 1 : (k < 12 ? 0 : 1))); }

// rne(v * inv) of four values as int8 bytes (little-endian) under the
// conditions of quant4: the magic-number sum's low byte is written into byte
// k of the result by the add itself (SDWA destination byte select), two VALU
// operations per value.
DAV2_DEV uint32_t quant4_bytes(float a, float b, float c, float d, float inv) {
    constexpr float kMagic = 12582912.0f;
    const float m = kMagic;
    uint32_t w;
    asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:DWORD"
        : "=v"(w) : "v"(a * inv), "v"(m));
    asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
        : "+v"(w) : "v"(b * inv), "v"(m));
    asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
        : "+v"(w) : "v"(c * inv), "v"(m));
    asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
        : "+v"(w) : "v"(d * inv), "v"(m));
    return w;
}

// SB (channel tiles of at most 128, whose registers then allow two waves
// per SIMD): one operand buffer instead of two, so that two workgroups
// share a CU; a block's MFMAs and the next block's quantization then take
// turns inside a workgroup, and the other workgroup's work (or its load
// latency) fills the gaps.
template <int BN, int WM, int WN, bool RELU_IN, bool SB>
__global__ __launch_bounds__(256, SB ? 2 : 1) void conv3x3_i8_kernel(ConvParams g) {
    constexpr int PW = kPixT / WM, NW = BN / WN, PB = PW / 16, NB = NW / 16;
    constexpr int kRing = 3;  // weight fragments three steps ahead (9 % 3 == 0)
    static_assert(WM * WN == 4 && PW % 16 == 0 && NW % 16 == 0, "wave tiling");

    __shared__ __attribute__((aligned(16))) int8_t at[(SB ? 1 : 2) * kBufBytes];
    __shared__ float amax_lds[4 * 64];
    __shared__ float sc_lds[kPixT];
    __shared__ float wsc_lds[BN], bias_lds[BN];

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave / WN, wn = wave % WN;

    // Workgroups go to the 8 XCDs round robin; each XCD gets a contiguous run
    // of tiles (neighbouring tiles share input rows in that XCD's L2), with
    // all channel tiles of one pixel tile together.
    const uint32_t nblk_n = gridDim.y, total = gridDim.x * gridDim.y;
    const uint32_t id = blockIdx.y * gridDim.x + blockIdx.x;
    const uint32_t xcd = id & 7u, slot = id >> 3, per = total >> 3, extra = total & 7u;
    const uint32_t lin = xcd * per + min(xcd, extra) + slot;
    const uint32_t nb = lin % nblk_n, pt = lin / nblk_n;
    const uint32_t ty = pt / g.tiles_x;
    const uint32_t y0 = 2u * ty, x0 = (pt - ty * g.tiles_x) * kTileCols3;
    const int H = static_cast<int>(g.height), W = static_cast<int>(g.width);

    // ---- input loads -------------------------------------------------------
    const uint32_t cp = lane >> 1, half = lane & 1u;
    // Byte offsets within a channel block of the lane's column pair in
    // window rows 0..3 (its channel half included); the channel goes into
    // the scalar offset. With an even width both columns of a pair lie in
    // or out of the image together.
    const uint32_t plane4 = static_cast<uint32_t>(g.plane) * 4u;
    const int col = static_cast<int>(x0) - 2 + 2 * static_cast<int>(cp);
    const bool col_ok = col >= 0 && col < W;
    uint32_t voff[4];
#pragma unroll
    for (int wr = 0; wr < 4; ++wr) {
        const int gy = static_cast<int>(y0) + wr - 1;
        const bool ok = col_ok && gy >= 0 && gy < H;
        voff[wr] = ok ? (half * 8u * static_cast<uint32_t>(g.plane) + static_cast<uint32_t>(gy) * g.width +
                         static_cast<uint32_t>(col)) * 4u
                      : kOutside;
    }
    auto block_rsrc = [&](uint32_t cb) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(g.x) + static_cast<uint64_t>(cb) * kCB * g.plane,
                                                 static_cast<short>(0), static_cast<int>(kCB * plane4), 0x00020000);
    };
    v2f xv[4][8];
    auto issue_row = [&](uint32_t cb, int wr) {
        const auto rs = block_rsrc(cb);
#pragma unroll
        for (int c = 0; c < 8; ++c)
            xv[wr][c] = __builtin_bit_cast(
                v2f, __builtin_amdgcn_raw_buffer_load_b64(rs, voff[wr], (wave * 16u + c) * plane4, 0));
    };

    // ---- packed weight fragments (conv_common.h) ---------------------------
    const uint32_t cblocks = g.channels / kCB, ksteps = kTaps * cblocks;
    const auto wrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(g.w), static_cast<short>(0),
                                                       static_cast<int>(g.n_out * ksteps * 64u), 0x00020000);
    const uint32_t wvoff = ((nb * BN + wn * NW) / 16u) * ksteps * 1024u + lane * 16u;
    auto load_w = [&](v4i (&b)[NB], uint32_t step) {
        const uint32_t cb = step / kTaps, tap = step - cb * kTaps;
        const uint32_t ks = tap * cblocks + cb;
#pragma unroll
        for (int i = 0; i < NB; ++i)
            b[i] = __builtin_bit_cast(v4i,
                                      __builtin_amdgcn_raw_buffer_load_b128(wrs, wvoff, (i * ksteps + ks) * 1024u, 0));
    };

    const uint32_t nblocks = cblocks, nsteps = ksteps;
    v4i ring[kRing][NB];

    // ---- per-pixel scales: window maxima of the channel-group maxima -----
    // Thread t: window row t / 64 (image row y0 - 1 + t/64), window column
    // t % 64 (image column x0 - 2 + t%64); positions outside the image read
    // as zero (the padding: an offset past the buffer). The first eight
    // groups' maxima are loaded before block 0's values and the first weight
    // fragments, which then stay in flight while the scales are formed
    // (loads return in issue order).
    float gmax[8];
    const int agy = static_cast<int>(y0) + static_cast<int>(tid >> 6) - 1;
    const int agx = static_cast<int>(x0) + static_cast<int>(lane) - 2;
    const bool a_in = agy >= 0 && agy < H && agx >= 0 && agx < W;
    {
        const auto prs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(g.partial), static_cast<short>(0),
                                                           static_cast<int>(g.groups * plane4), 0x00020000);
        const uint32_t aoff = a_in ? (static_cast<uint32_t>(agy) * g.width + static_cast<uint32_t>(agx)) * 4u
                                   : kOutside;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            gmax[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                    prs, aoff, min(static_cast<uint32_t>(k), g.groups - 1u) * plane4, 0));
    }
#pragma unroll
    for (int wr = 0; wr < 4; ++wr) issue_row(0, wr);
#pragma unroll
    for (int d = 0; d < kRing; ++d) load_w(ring[d], min(static_cast<uint32_t>(d), nsteps - 1));
    {
        float t = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) t = fmaxf(t, gmax[k]);
        if (a_in) {
            const float* src = g.partial + static_cast<uint64_t>(agy) * g.width + agx;
            for (uint32_t k = 8; k < g.groups; ++k) t = fmaxf(t, src[k * g.plane]);
        }
        amax_lds[tid] = t;
    }
    if (tid < BN) {
        const uint32_t ch = nb * BN + tid;
        wsc_lds[tid] = g.w_scales[ch];
        bias_lds[tid] = g.bias ? g.bias[ch] : 0.0f;
    }
    lds_barrier();
    // Pixel slot (i, lane): window rows i .. i + 2, columns lane + 1 ..
    // lane + 3 (the unstored slots take what lies inside the 64 columns).
    float s_pix[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        float m = 0.0f;
#pragma unroll
        for (int r = 0; r < 3; ++r)
#pragma unroll
            for (int dx = 0; dx < 3; ++dx) m = fmaxf(m, amax_lds[(i + r) * 64 + min(lane + 1u + dx, 63u)]);
        s_pix[i] = row_scale(m);
    }
    if (wave == 0) {
        sc_lds[lane] = s_pix[0];
        sc_lds[64 + lane] = s_pix[1];
    }
    lds_barrier();
    // This lane's window columns w = 2 cp + t serve pixel w - 1 - dx as tap
    // column dx; 1 / scale of each such pixel, exactly the quantizer's 1.0f / s.
    float inv[2][2][3];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int dx = 0; dx < 3; ++dx) {
                const int p = static_cast<int>(2u * cp) + t - 1 - dx;
                inv[i][t][dx] = 1.0f / sc_lds[i * 64 + (p >= 0 ? p : 0)];
            }

    // ---- quantizer ---------------------------------------------------------
    // Unit u (0..7) of tap t's share: piece 2t + u / 4, window column
    // 2 cp + (u / 2) % 2, channels 4 (u % 2) .. + 3 of the lane's eight; the
    // second unit of a column writes the column's 8 bytes.
    uint32_t qlo = 0;
    auto quant_unit = [&](int8_t* buf, int tap, int u) {
        const int k = 2 * tap + u / 4, t = (u / 2) % 2, part = u % 2;
        const int wr = piece_row(k), i = piece_pixel_row(k), dx = k % 3, dy = wr - i;
        if (RELU_IN && u % 4 == 0 && (k == 0 || k == 3 || k == 9 || k == 15)) {  // a row's first piece
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                xv[wr][c].x = fmaxf(xv[wr][c].x, 0.0f);
                xv[wr][c].y = fmaxf(xv[wr][c].y, 0.0f);
            }
        }
        auto v = [&](int c) { return t == 0 ? xv[wr][c].x : xv[wr][c].y; };
        const uint32_t q = quant4_bytes(v(4 * part + 0), v(4 * part + 1), v(4 * part + 2), v(4 * part + 3),
                                        inv[i][t][dx]);
        if (part == 0) {
            qlo = q;
        } else {
            const int px = static_cast<int>(2u * cp) + t - 1 - dx;
            if (px >= 0)
                *reinterpret_cast<v2u*>(buf + (dy * 3 + dx) * kTapBytes +
                                        tile_offset(i * 64 + static_cast<uint32_t>(px), wave) + 8u * half) = v2u{qlo, q};
        }
    };

    v4i acc[NB][PB];
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < PB; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    // Prologue: block 0's tile, block 1's values in flight.
#pragma unroll
    for (int tap = 0; tap < kTaps; ++tap)
#pragma unroll
        for (int u = 0; u < 8; ++u) quant_unit(at, tap, u);
    {
        const uint32_t c1 = min(1u, nblocks - 1);
#pragma unroll
        for (int wr = 0; wr < 4; ++wr) issue_row(c1, wr);
    }
    lds_barrier();

    // Operand reads: lane l reads pixel slot wm*PW + 16j + l%16, chunk l/16.
    // Fragment j of the next tap is read as soon as this tap's MFMAs on
    // fragment j are issued.
    const uint32_t prow = wm * PW + (lane & 15u), pchunk = lane >> 4;
    v4i bp[PB];
    auto read_frag = [&](int j, const int8_t* tile) {
        bp[j] = *reinterpret_cast<const v4i*>(tile + tile_offset(prow + 16u * j, pchunk));
    };
    constexpr int kUnitsPerChunk = 8 / PB;
    static_assert(PB * kUnitsPerChunk == 8, "quantizer units per MFMA chunk");
    for (uint32_t cb = 0; SB && cb < nblocks; ++cb) {
        // loads past the last block re-read it (unconditional prefetches)
        const uint32_t ahead = min(cb + 2, nblocks - 1);
#pragma unroll
        for (int j = 0; j < PB; ++j) read_frag(j, at);
#pragma unroll
        for (int tap = 0; tap < kTaps; ++tap) {
            const uint32_t step = cb * kTaps + tap;
            v4i (&bw)[NB] = ring[tap % kRing];
#pragma unroll
            for (int j = 0; j < PB; ++j) {
#pragma unroll
                for (int i = 0; i < NB; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bw[i], bp[j], acc[i][j], 0, 0, 0);
                if (tap + 1 < kTaps) read_frag(j, at + (tap + 1) * kTapBytes);
            }
            load_w(bw, min(step + kRing, nsteps - 1));
        }
        if (cb + 1 == nblocks) break;
        lds_barrier();  // every wave has read block cb's tile
        // block cb + 1's tile into the same buffer; a window row whose last
        // piece is done takes block cb + 2's values
#pragma unroll
        for (int tap = 0; tap < kTaps; ++tap) {
#pragma unroll
            for (int u = 0; u < 8; ++u) quant_unit(at, tap, u);
            if (tap == 1) issue_row(ahead, 0);
            if (tap == 4) issue_row(ahead, 1);
            if (tap == 7) issue_row(ahead, 2);
            if (tap == 8) issue_row(ahead, 3);
        }
        lds_barrier();
    }
    for (uint32_t cb = 0; !SB && cb < nblocks; ++cb) {
        // loads past the last block re-read it (unconditional prefetches)
        const uint32_t ahead = min(cb + 2, nblocks - 1);
        const int8_t* cur = at + (cb & 1u) * kBufBytes;
        int8_t* nxt = at + ((cb + 1) & 1u) * kBufBytes;
#pragma unroll
        for (int j = 0; j < PB; ++j) read_frag(j, cur);
#pragma unroll
        for (int tap = 0; tap < kTaps; ++tap) {
            const uint32_t step = cb * kTaps + tap;
            v4i (&bw)[NB] = ring[tap % kRing];
            // Chunks in program order (scheduling fences between them): the
            // MFMAs on fragment j, the read of the next tap's fragment j and
            // a share of the next block's quantizer, so its VALU work issues
            // while the matrix core runs. (Past the last block the quantizer
            // writes a re-read of it into the buffer nothing reads again.)
#pragma unroll
            for (int j = 0; j < PB; ++j) {
#pragma unroll
                for (int i = 0; i < NB; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bw[i], bp[j], acc[i][j], 0, 0, 0);
                if (tap + 1 < kTaps) read_frag(j, cur + (tap + 1) * kTapBytes);
#pragma unroll
                for (int u = 0; u < kUnitsPerChunk; ++u) quant_unit(nxt, tap, j * kUnitsPerChunk + u);
                __builtin_amdgcn_sched_barrier(0);
            }
            load_w(bw, min(step + kRing, nsteps - 1));
            // a window row whose last piece is done takes block cb + 2's
            // values (issued after the weights, which are waited on sooner)
            if (tap == 1) issue_row(ahead, 0);
            if (tap == 4) issue_row(ahead, 1);
            if (tap == 7) issue_row(ahead, 2);
            if (tap == 8) issue_row(ahead, 3);
            __builtin_amdgcn_sched_barrier(0);
        }
        // block cb + 1's tile is complete; block cb's buffer is free
        lds_barrier();
    }

    // ---- epilogue: pixel slot p = (row p / 64, column p % 64) --------------
    store_tile<BN, WM, WN, kPixT>(g, acc, wm, wn, lane, nb, sc_lds, wsc_lds, bias_lds,
                                  [&](uint32_t p, uint64_t& pixel) {
                                      const uint32_t i = p >> 6, j = p & 63u;
                                      pixel = static_cast<uint64_t>(y0 + i) * g.width + x0 + j;
                                      return j < static_cast<uint32_t>(kTileCols3) && x0 + j < g.width &&
                                             y0 + i < g.height;
                                  });
}

template <int BN, int WM, int WN, bool SB>
void launch(const ConvParams& g, uint32_t tiles, uint32_t n, hipStream_t s) {
    if (g.flags & DAV2_CONV_RELU_INPUT)
        dispatch((conv3x3_i8_kernel<BN, WM, WN, true, SB>), dim3(tiles, n / BN), dim3(256), 0, s, g);
    else
        dispatch((conv3x3_i8_kernel<BN, WM, WN, false, SB>), dim3(tiles, n / BN), dim3(256), 0, s, g);
}

}  // namespace

// 256 output channels over at least 128 tiles: each wave 128 pixels x 64
// channels, double-buffered, one workgroup per CU. Otherwise 2 x 2 waves of
// 64 pixels (one tile row) x BN/2 channels, single-buffered, two workgroups
// per CU (296x296, 256 -> 128: 86 -> 72 us; 74x74, 256 -> 256 as two
// 128-channel tiles: 31 -> 26 us; 518x518, 128 -> 32: 139 -> 88 us).
hipError_t dav2k::launch_conv3x3_i8(const ConvParams& g, uint32_t tiles, uint32_t n, hipStream_t s) {
    if (n % 256 == 0 && tiles >= 128) launch<256, 1, 4, false>(g, tiles, n, s);
    else if (n % 128 == 0) launch<128, 2, 2, true>(g, tiles, n, s);
    else if (n % 64 == 0) launch<64, 2, 2, true>(g, tiles, n, s);
    else launch<32, 2, 2, true>(g, tiles, n, s);
    return hipGetLastError();
}
