// Implicit-GEMM int8 convolution on CDNA4 matrix cores: im2col, per-pixel
// quantization and the int8 GEMM of the reference's conv2d_int8
// (src/operators.cpp:1735-1805: im2col_quantize_int8.glsl:26-83 then
// linear_int8_tiled.glsl:40-117 with the CHW store) in one kernel, without
// the im2col matrix ever reaching HBM.
//
// Scope: kernel 1 (stride 1, no padding), and kernel 3 (stride 1, padding 1)
// on maps conv3x3_i8.hip does not take (odd widths, inputs not 8-byte
// aligned); input channels a multiple of 64, output channels a multiple of
// 32.
//
// Arithmetic. Output pixel p's im2col row is quantized with the scale
// s = max(absmax/127, 1e-8) of that whole row and q = rne(clamp(x * (1/s))),
// exactly as im2col_quantize_int8.glsl; the int32 dot products are exact, so
// the order in which K is walked is free. This kernel walks K tap-major
// (k = tap * C + c, tap = ky * ks + kx) so that one 64-byte K step is 64
// channels of one tap; the weights are stored in that order
// (packed by dav2_hip_conv_weights_pack). The epilogue is the GEMM's CHW epilogue,
// ((float(acc) * s_pixel) * s_weight) + bias, so every output float equals
// the im2col + GEMM path's bit for bit.
//
// Tiling. A workgroup (4 waves) owns 64 output pixels (a segment of one image
// row for 3x3, 64 consecutive pixels for 1x1) and BN output channels. Per
// block of 64 input channels it stages the fp32 input window (64 channels x
// 3 rows x 66 columns for 3x3) in LDS; per tap every thread quantizes 16
// channels of one pixel into a double-buffered 64 x 64-byte int8 tile
// (XOR-swizzled rows, conflict-free for the MFMA operand reads), and the
// waves multiply it against weight fragments read straight from global
// memory (v_mfma_i32_16x16x64_i8, weights as the row operand so each lane's
// accumulators run along pixels and the CHW stores coalesce). Each wave
// stages the window of the 16 channels it quantizes itself. For 3x3 the next
// channel block's window rows are copied global->LDS without registers
// (global_load_lds_dword) as soon as the current block's taps are done with
// each row (row 0 after tap 2, row 1 after tap 5, row 2 after tap 8), seven
// steps before they are read; 1x1 loads the next block into registers.
// Weight fragments come three steps ahead, so global latency hides behind
// the quantize and MFMA work. One LDS-only barrier per tap.

#include <algorithm>
#include <type_traits>

#include "common.h"
#include "conv_common.h"
#include "dav2_hip.h"

using namespace dav2k;

namespace {

// Source of the 3x3 window positions outside the image (zero padding): the
// copies of those positions read it instead of the input.
__device__ float g_conv_zero_row[64];

template <int KS, int BN, int WM, int WN, bool RELU_IN>
__global__ __launch_bounds__(256) void conv_i8_kernel(ConvParams g) {
    constexpr int kRowsT = KS;                   // input rows per channel in the window
    constexpr int kColsT = kPix + KS - 1;        // input columns per row (halo for 3x3)
    constexpr int kPlaneT = kRowsT * kColsT;     // floats per channel in LDS
    constexpr int kLoads = kCB * kRowsT / 4;     // 64-wide row loads per wave per block
    constexpr int kTaps = KS * KS;
    constexpr int PW = kPix / WM, NW = BN / WN;  // pixels / channels per wave
    constexpr int PB = PW / 16, NB = NW / 16;
    static_assert(WM * WN == 4 && PW % 16 == 0 && NW % 16 == 0, "wave tiling");

    __shared__ float xt[kCB * kPlaneT];
    __shared__ __attribute__((aligned(16))) int8_t at[2][kPix * 64];
    __shared__ float sc_lds[kPix];
    __shared__ float wsc_lds[BN], bias_lds[BN];
    __shared__ float amax_lds[KS == 3 ? 3 * kColsT : 1];

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave / WN, wn = wave % WN;

    // Workgroups go to the 8 XCDs round robin; give each XCD a contiguous run
    // of pixel tiles (neighbouring tiles share input rows in that XCD's L2),
    // with all channel blocks of one pixel tile together.
    const uint32_t nblk_n = gridDim.y, total = gridDim.x * gridDim.y;
    const uint32_t id = blockIdx.y * gridDim.x + blockIdx.x;
    const uint32_t xcd = id & 7u, slot = id >> 3, per = total >> 3, extra = total & 7u;
    const uint32_t lin = xcd * per + min(xcd, extra) + slot;
    const uint32_t nb = lin % nblk_n, pt = lin / nblk_n;

    // The image as rows of `rowlen` pixels: 3x3 tiles are row segments, 1x1
    // tiles are runs of the flattened map (one row of `plane` pixels).
    const uint32_t rowlen = KS == 3 ? g.width : static_cast<uint32_t>(g.plane);
    const uint32_t nrows = KS == 3 ? g.height : 1u;
    const uint32_t y = KS == 3 ? pt / g.tiles_x : 0u;
    const uint32_t x0 = KS == 3 ? (pt - y * g.tiles_x) * kPix : pt * kPix;
    const uint64_t mbase = static_cast<uint64_t>(y) * rowlen + x0;
    const uint32_t valid = min(static_cast<uint32_t>(kPix), rowlen - x0);

    // ---- per-pixel scale: window maximum of the channel-group maxima -----
    float m = 0.0f;
    if constexpr (KS == 3) {
        if (tid < 3u * kColsT) {
            const int r = static_cast<int>(tid) / kColsT, col = static_cast<int>(tid) % kColsT;
            const int gy = static_cast<int>(y) + r - 1, gx = static_cast<int>(x0) + col - 1;
            float t = 0.0f;
            if (gy >= 0 && gy < static_cast<int>(g.height) && gx >= 0 && gx < static_cast<int>(g.width)) {
                const float* src = g.partial + static_cast<uint64_t>(gy) * g.width + gx;
                for (uint32_t k = 0; k < g.groups; ++k) t = fmaxf(t, src[k * g.plane]);
            }
            amax_lds[tid] = t;
        }
        lds_barrier();
#pragma unroll
        for (int r = 0; r < 3; ++r)
#pragma unroll
            for (int dx = 0; dx < 3; ++dx) m = fmaxf(m, amax_lds[r * kColsT + lane + dx]);
    } else {
        if (lane < valid)
            for (uint32_t k = 0; k < g.groups; ++k) m = fmaxf(m, g.partial[k * g.plane + mbase + lane]);
    }
    const float s_pix = row_scale(m);
    const float inv = 1.0f / s_pix;  // this thread quantizes pixel `lane`
    if (wave == 0) sc_lds[lane] = s_pix;
    if (tid < BN) {
        const uint32_t ch = nb * BN + tid;
        wsc_lds[tid] = g.w_scales[ch];
        bias_lds[tid] = g.bias ? g.bias[ch] : 0.0f;
    }

    // ---- input window staging ---------------------------------------------
    // Wave w loads LDS rows R = w*kLoads + j (channel R / kRowsT, window row
    // R % kRowsT), 64 columns per load with lane = column; the two halo
    // columns of every row (3x3) are loaded by threads 0..383 of the block.
    // Every load reads a valid address (rows and columns clamped into the
    // image); the padding zeros are substituted when the window is written to
    // LDS, so no load sits behind a branch or waits before that point.
    // Addresses are the tensor base plus a 32-bit byte offset (the host
    // checks that the input is below 4 GiB): a wave-uniform row offset and
    // one per-lane column offset. The block index goes through an empty asm
    // statement so the row arithmetic is redone with scalar instructions in
    // every block instead of being hoisted into 48 live vector registers.
    const bool col_ok = x0 + lane < rowlen;
    const uint32_t col4 = min(x0 + lane, rowlen - 1u) * 4u;
    const uint32_t plane32 = static_cast<uint32_t>(g.plane);
    const char* xbase = reinterpret_cast<const char*>(g.x);
    float xs[KS == 3 ? 1 : kLoads];  // 3x3 windows bypass registers
    float xh[2] = {0.0f, 0.0f};
    constexpr bool relu_in = RELU_IN;
    // Byte offsets of the window rows within a channel plane (clamped).
    uint32_t row4[kRowsT];
#pragma unroll
    for (int r = 0; r < kRowsT; ++r) {
        const int gy = static_cast<int>(y) + r - KS / 2;
        row4[r] = static_cast<uint32_t>(min(max(gy, 0), static_cast<int>(nrows) - 1)) * rowlen * 4u;
    }
    // Wave w's rows j = 0..kLoads-1 are channel 16w + j / kRowsT, window row
    // j % kRowsT. The channel offset advances through an opaque register so
    // the compiler does not precompute (and keep live) all kLoads offsets.
    auto issue_rows = [&](uint32_t cb, int j0, int j1) {
        if constexpr (KS == 3) return;
        uint32_t chan = ((cb * kCB + wave * (kCB / 4) + j0 / kRowsT) * plane32) * 4u;
        asm volatile("" : "+s"(chan));
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            if (j < j0 || j >= j1) continue;
            if (j > j0 && j % kRowsT == 0) {
                chan += plane32 * 4u;
                asm volatile("" : "+s"(chan));
            }
            xs[j] = *reinterpret_cast<const float*>(xbase + (chan + row4[j % kRowsT] + col4));
        }
    };
    // 3x3 halo columns x0 - 1 and x0 + 64 of the wave's 16 channels: value
    // h = 6 c + 2 r + side (96 per wave) is lane h % 64's register h / 64.
    auto issue_halo = [&](uint32_t cb) {
        if constexpr (KS == 3) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint32_t h = min(lane + 64u * i, 95u);
                const uint32_t c = wave * 16u + h / 6u, r = (h >> 1) % 3u;
                const int gy = static_cast<int>(y) + static_cast<int>(r) - 1;
                const int gx = (h & 1u) ? static_cast<int>(x0) + kPix : static_cast<int>(x0) - 1;
                const uint32_t gyc = static_cast<uint32_t>(min(max(gy, 0), static_cast<int>(g.height) - 1));
                const uint32_t gxc = static_cast<uint32_t>(min(max(gx, 0), static_cast<int>(g.width) - 1));
                const uint32_t off = ((cb * kCB + c) * plane32 + gyc * g.width + gxc) * 4u;
                xh[i] = *reinterpret_cast<const float*>(xbase + off);
            }
        }
    };
    auto write_halo = [&]() {
        if constexpr (KS == 3) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint32_t h = lane + 64u * i;
                if (h < 96u) {
                    const uint32_t c = wave * 16u + h / 6u, r = (h >> 1) % 3u;
                    const int gy = static_cast<int>(y) + static_cast<int>(r) - 1;
                    const int gx = (h & 1u) ? static_cast<int>(x0) + kPix : static_cast<int>(x0) - 1;
                    const bool ok =
                        gy >= 0 && gy < static_cast<int>(g.height) && gx >= 0 && gx < static_cast<int>(g.width);
                    xt[c * kPlaneT + r * kColsT + ((h & 1u) ? kColsT - 1u : 0u)] = ok ? xh[i] : 0.0f;
                }
            }
        }
    };
    // 3x3: window row r (image row y + r - 1) of the wave's 16 channels of
    // block cb, columns x0 .. x0 + 63, straight into LDS: one copy per
    // channel, lane = column; positions outside the image read zeros.
    const char* zero_lane = reinterpret_cast<const char*>(g_conv_zero_row + lane);
    auto copy_rows = [&](uint32_t cb, int r) {
        if constexpr (KS == 3) {
            const int gy = static_cast<int>(y) + r - 1;
            const bool ok = col_ok && gy >= 0 && gy < static_cast<int>(nrows);
            uint32_t chan = ((cb * kCB + wave * 16u) * plane32) * 4u + row4[r] + col4;
            asm volatile("" : "+v"(chan));
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const char* src = ok ? xbase + (chan + static_cast<uint32_t>(e) * plane32 * 4u) : zero_lane;
                copy4_to_lds(src, xt + (wave * 16u + e) * kPlaneT + r * kColsT + 1);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto write_window = [&]() {
        if constexpr (KS == 3) return;
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const uint32_t R = wave * kLoads + j;
            const uint32_t c = R / kRowsT, r = R - c * kRowsT;
            const int gy = static_cast<int>(y) + static_cast<int>(r) - KS / 2;
            const bool ok = col_ok && gy >= 0 && gy < static_cast<int>(nrows);
            const float v = ok ? xs[j] : 0.0f;
            xt[c * kPlaneT + r * kColsT + (KS == 3 ? 1u : 0u) + lane] = relu_in ? fmaxf(v, 0.0f) : v;
        }
        if constexpr (KS == 3) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t idx = tid + 256u * h;
                if (idx < 2u * kCB * 3u) {
                    const uint32_t R = idx >> 1, c = R / 3u, r = R - 3u * c;
                    const int gy = static_cast<int>(y) + static_cast<int>(r) - 1;
                    const int gx = (idx & 1u) ? static_cast<int>(x0) + kPix : static_cast<int>(x0) - 1;
                    const bool ok =
                        gy >= 0 && gy < static_cast<int>(g.height) && gx >= 0 && gx < static_cast<int>(g.width);
                    const float v = ok ? xh[h] : 0.0f;
                    xt[c * kPlaneT + r * kColsT + ((idx & 1u) ? kColsT - 1u : 0u)] = relu_in ? fmaxf(v, 0.0f) : v;
                }
            }
        }
    };

    // ---- weight fragments (packed: one contiguous 1 KiB per fragment) -------
    const uint32_t ksteps = kTaps * (g.channels / kCB);
    const uint32_t wbase = ((nb * BN + wn * NW) / 16u) * ksteps * 1024u + lane * 16u;
    auto load_w = [&](v4i (&b)[NB], uint32_t step) {
        const uint32_t cb = step / kTaps, tap = step - cb * kTaps;
        const uint32_t ks = tap * (g.channels / kCB) + cb;
#pragma unroll
        for (int i = 0; i < NB; ++i)
            b[i] = *reinterpret_cast<const v4i*>(g.w + (wbase + (i * ksteps + ks) * 1024u));
    };

    v4i acc[NB][PB];
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < PB; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    // Weight fragments go through a ring of kRing steps. Global loads retire
    // in issue order (one vmcnt counter per wave), so the slow input-window
    // loads of the next block are issued once per block, right after a
    // weight load: only the weight load kRing steps later queues behind them.
    constexpr int kRing = kTaps % 3 == 0 ? 3 : 1;
    const uint32_t nblocks = g.channels / kCB, nsteps = nblocks * kTaps;
    v4i ring[kRing][NB];
    issue_rows(0, 0, kLoads);
#pragma unroll
    for (int r = 0; r < kRowsT; ++r) copy_rows(0, r);
    issue_halo(0);
#pragma unroll
    for (int d = 0; d < kRing; ++d) load_w(ring[d], min(static_cast<uint32_t>(d), nsteps - 1));
    write_window();
    write_halo();  // its loads follow the row copies, so those have landed too
    lds_barrier();

    // Operand reads of this wave's pixel blocks: lane l reads pixel
    // wm*PW + 16j + l%16, chunk l/16.
    const uint32_t prow = wm * PW + (lane & 15u), pchunk = lane >> 4;
    // Quantizer: pixel `lane`, channels 16*wave .. +15 of the block.
    const float* qsrc = xt + (wave * 16u) * kPlaneT + lane;
    const uint32_t qdst = a_offset(lane, wave);

    // Pipeline per step (tap t): barrier; the step's operand reads are issued;
    // the next tap is quantized into the other operand buffer and the window
    // values of the tap after that are read (both overlap the operand read
    // latency); then the MFMAs. Tap 0 of a block is quantized before the
    // block's first barrier.
    float f[16];
    auto read_tap = [&](int tap) {
        uint32_t qoff = (tap / KS) * kColsT + (tap % KS);
        asm volatile("" : "+v"(qoff));  // keep the read bases from being hoisted
        const float* src = qsrc + qoff;
#pragma unroll
        for (int e = 0; e < 16; ++e) f[e] = src[e * kPlaneT];
    };
    auto quantize_into = [&](int8_t* abuf) {
        uint32_t w4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            // 3x3 windows arrive unmodified: the input ReLU is taken here
            const bool r = KS == 3 && relu_in;
            w4[q] = quant4(r ? fmaxf(f[4 * q + 0], 0.0f) : f[4 * q + 0], r ? fmaxf(f[4 * q + 1], 0.0f) : f[4 * q + 1],
                           r ? fmaxf(f[4 * q + 2], 0.0f) : f[4 * q + 2], r ? fmaxf(f[4 * q + 3], 0.0f) : f[4 * q + 3],
                           inv);
        }
        *reinterpret_cast<v4i*>(abuf + qdst) =
            v4i{static_cast<int>(w4[0]), static_cast<int>(w4[1]), static_cast<int>(w4[2]), static_cast<int>(w4[3])};
    };
    // Tap 0 of the block starting at step s0 into its operand buffer, and
    // the window values of tap 1.
    auto block_start = [&](uint32_t s0) {
        read_tap(0);
        quantize_into(at[s0 & 1u]);
        if (kTaps > 1) read_tap(1);
    };
    block_start(0);

    for (uint32_t cb = 0; cb < nblocks; ++cb) {
        const bool more = cb + 1 < nblocks;
        const uint32_t next_cb = more ? cb + 1 : cb;
#pragma unroll
        for (int tap = 0; tap < kTaps; ++tap) {
            const uint32_t step = cb * kTaps + tap;
            lds_barrier();  // operand tile `step` is complete
            const int8_t* abuf = at[step & 1u];
            v4i bp[PB];
#pragma unroll
            for (int j = 0; j < PB; ++j) bp[j] = *reinterpret_cast<const v4i*>(abuf + a_offset(prow + 16u * j, pchunk));
            if (tap + 1 < kTaps) {
                // the other buffer was last read by step - 1, which every
                // wave finished before this step's barrier
                quantize_into(at[(step + 1u) & 1u]);
                if (tap + 2 < kTaps) {
                    // 3x3: rows 1 and 2 of this block were copied during the
                    // previous one and 16 copies (the next row's) follow
                    // each, so at most 16 outstanding operations mean the
                    // row has landed (copies retire in issue order)
                    if (KS == 3 && (tap + 2 == 3 || tap + 2 == 6)) DAV2_WAIT_VMCNT(16);
                    read_tap(tap + 2);
                }
            }
            v4i (&bw)[NB] = ring[tap % kRing];
#pragma unroll
            for (int j = 0; j < PB; ++j)
#pragma unroll
                for (int i = 0; i < NB; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bw[i], bp[j], acc[i][j], 0, 0, 0);
            // Prefetches are unconditional (a branch around a load makes the
            // compiler wait for it at the merge); past the end they re-read
            // the last step / block, which is harmless.
            load_w(bw, min(step + kRing, nsteps - 1));
            if (tap == 0) {
                issue_rows(next_cb, 0, kLoads);
                issue_halo(next_cb);
            }
            // 3x3: a row of the window is free once every tap reading it has
            // read (reads run two taps ahead, before the next barrier); past
            // the last block the copies repeat the current rows
            if (tap == 1) copy_rows(next_cb, 0);
            if (tap == 4) copy_rows(next_cb, 1);
            if (tap == 7) copy_rows(next_cb, 2);
        }
        if (more) {
            if constexpr (KS == 3) {
                // the window is wave-local: halo values, then row 0 of the
                // next block (rows 1 and 2, 32 copies, were issued after it)
                write_halo();
                DAV2_WAIT_VMCNT(32);
            } else {
                // Every wave is past the last tap's barrier, so no quantizer
                // still reads the window: replace it with the next block's.
                write_window();
                lds_barrier();
            }
            // the buffer of step (cb + 1) * kTaps was last read two steps ago
            block_start((cb + 1) * kTaps);
        }
    }

    store_tile<BN, WM, WN, kPix>(g, acc, wm, wn, lane, nb, sc_lds, wsc_lds, bias_lds,
                                 [&](uint32_t p, uint64_t& pixel) {
                                     pixel = mbase + p;
                                     return p < valid;
                                 });
}

// 1x1 convolution to at most kNarrowN output channels: one thread per pixel
// holds its (at most 64) input values, takes their absmax, quantizes them with
// the im2col rule rne(clamp(x * (1/s))) and forms the dot products on the
// VALU; the epilogue is the GEMM's ((acc * s) * s_w) + bias.
constexpr uint32_t kNarrowN = 4, kNarrowC = 64;

__global__ __launch_bounds__(256) void conv1x1_narrow_kernel(const float* __restrict__ x, uint64_t plane,
                                                             uint32_t channels, const int8_t* __restrict__ w,
                                                             uint32_t ldw, const float* __restrict__ w_scales,
                                                             const float* __restrict__ bias, uint32_t n,
                                                             float* __restrict__ out, float* __restrict__ pre_relu,
                                                             uint32_t flags) {
    const uint64_t p = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    if (p >= plane) return;
    const bool relu_in = (flags & DAV2_CONV_RELU_INPUT) != 0, relu_out = (flags & DAV2_CONV_RELU_OUTPUT) != 0;
    float v[kNarrowC];
    float m = 0.0f;
#pragma unroll
    for (uint32_t c = 0; c < kNarrowC; ++c) {
        if (c < channels) {
            const float t = x[c * plane + p];
            v[c] = relu_in ? fmaxf(t, 0.0f) : t;
            m = fmaxf(m, fabsf(v[c]));
        }
    }
    const float s = row_scale(m), inv = 1.0f / s;
    int q[kNarrowC];
#pragma unroll
    for (uint32_t c = 0; c < kNarrowC; ++c) q[c] = c < channels ? quantize_rne(v[c] * inv) : 0;
    for (uint32_t o = 0; o < n; ++o) {
        int32_t acc = 0;
#pragma unroll
        for (uint32_t c = 0; c < kNarrowC; ++c)
            if (c < channels) acc += q[c] * static_cast<int32_t>(w[static_cast<uint64_t>(o) * ldw + c]);
        float r = static_cast<float>(acc);
        r = r * s;
        r = r * w_scales[o];
        r = r + (bias ? bias[o] : 0.0f);
        if (pre_relu) pre_relu[o * plane + p] = r;
        out[o * plane + p] = relu_out ? fmaxf(r, 0.0f) : r;
    }
}

// The same for a compile-time channel count on planes of an even number of
// pixels: each thread takes two adjacent pixels (8-byte loads and stores),
// the same arithmetic per pixel.
template <int C>
__global__ __launch_bounds__(256) void conv1x1_narrow_pairs_kernel(const float* __restrict__ x, uint64_t plane,
                                                                   const int8_t* __restrict__ w, uint32_t ldw,
                                                                   const float* __restrict__ w_scales,
                                                                   const float* __restrict__ bias, uint32_t n,
                                                                   float* __restrict__ out,
                                                                   float* __restrict__ pre_relu, uint32_t flags) {
    const uint64_t p = 2u * (static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x);
    if (p >= plane) return;
    const bool relu_in = (flags & DAV2_CONV_RELU_INPUT) != 0, relu_out = (flags & DAV2_CONV_RELU_OUTPUT) != 0;
    float2 v[C];
#pragma unroll
    for (int c = 0; c < C; ++c) v[c] = *reinterpret_cast<const float2*>(x + c * plane + p);
    float m0 = 0.0f, m1 = 0.0f;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        if (relu_in) {
            v[c].x = fmaxf(v[c].x, 0.0f);
            v[c].y = fmaxf(v[c].y, 0.0f);
        }
        m0 = fmaxf(m0, fabsf(v[c].x));
        m1 = fmaxf(m1, fabsf(v[c].y));
    }
    const float s0 = row_scale(m0), inv0 = 1.0f / s0;
    const float s1 = row_scale(m1), inv1 = 1.0f / s1;
    int q0[C], q1[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {
        q0[c] = quantize_rne(v[c].x * inv0);
        q1[c] = quantize_rne(v[c].y * inv1);
    }
    for (uint32_t o = 0; o < n; ++o) {
        int32_t a0 = 0, a1 = 0;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const int32_t wc = static_cast<int32_t>(w[static_cast<uint64_t>(o) * ldw + c]);
            a0 += q0[c] * wc;
            a1 += q1[c] * wc;
        }
        const float ws = w_scales[o], b = bias ? bias[o] : 0.0f;
        float r0 = static_cast<float>(a0);
        r0 = r0 * s0;
        r0 = r0 * ws;
        r0 = r0 + b;
        float r1 = static_cast<float>(a1);
        r1 = r1 * s1;
        r1 = r1 * ws;
        r1 = r1 + b;
        if (pre_relu) *reinterpret_cast<float2*>(pre_relu + o * plane + p) = make_float2(r0, r1);
        *reinterpret_cast<float2*>(out + o * plane + p) =
            relu_out ? make_float2(fmaxf(r0, 0.0f), fmaxf(r1, 0.0f)) : make_float2(r0, r1);
    }
}

// Packed convolution weights (conv_common.h): dst byte
// ((nb * ksteps + ks) * 64 + l) * 16 + b holds weight row 16 nb + l % 16 at
// tap-major K index k = 64 ks + 16 (l / 16) + b (k = tap * C + c), which is
// src[row][c * taps + tap].
__global__ __launch_bounds__(256) void weights_pack_kernel(int8_t* __restrict__ dst, const int8_t* __restrict__ src,
                                                           uint32_t n, uint32_t channels, uint32_t taps, uint64_t ldb) {
    const uint64_t row_len = static_cast<uint64_t>(taps) * channels;
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    if (idx >= row_len * n) return;
    const uint32_t ksteps = static_cast<uint32_t>(row_len / 64u);
    const uint32_t b = static_cast<uint32_t>(idx & 15u), l = static_cast<uint32_t>((idx >> 4) & 63u);
    const uint64_t frag = idx >> 10;
    const uint32_t nb = static_cast<uint32_t>(frag / ksteps), ks = static_cast<uint32_t>(frag - uint64_t(nb) * ksteps);
    const uint64_t row = uint64_t(nb) * 16u + (l & 15u);
    const uint32_t k = ks * 64u + (l >> 4) * 16u + b;
    const uint32_t tap = k / channels, c = k - tap * channels;
    dst[idx] = src[row * ldb + static_cast<uint64_t>(c) * taps + tap];
}

template <int KS, int BN, int WM, int WN>
void launch(const ConvParams& g, uint32_t tiles, uint32_t n, hipStream_t s) {
    if (g.flags & DAV2_CONV_RELU_INPUT)
        dispatch((conv_i8_kernel<KS, BN, WM, WN, true>), dim3(tiles, n / BN), dim3(256), 0, s, g);
    else
        dispatch((conv_i8_kernel<KS, BN, WM, WN, false>), dim3(tiles, n / BN), dim3(256), 0, s, g);
}

template <int KS>
void launch_ks(const ConvParams& g, uint32_t tiles, uint32_t n, hipStream_t s) {
    // Measured on the DPT shapes: one channel slice per wave (each wave
    // reads the whole pixel tile) beats 2x2 wave grids, and the widest
    // channel tile wins; 32-channel maps use a 2x2 grid.
    if (n % 256 == 0) launch<KS, 256, 1, 4>(g, tiles, n, s);
    else if (n % 128 == 0) launch<KS, 128, 1, 4>(g, tiles, n, s);
    else if (n % 64 == 0) launch<KS, 64, 1, 4>(g, tiles, n, s);
    else launch<KS, 32, 2, 2>(g, tiles, n, s);
}

}  // namespace

extern "C" {

int dav2_hip_conv_weights_pack(int8_t* dst, const int8_t* src, uint32_t out_channels, uint32_t channels,
                               uint32_t kernel, uint64_t ldb, void* stream) {
    if (out_channels == 0) return hipSuccess;
    const uint64_t taps = static_cast<uint64_t>(kernel) * kernel;
    if (!dst || !src || kernel == 0 || channels == 0 || ldb < taps * channels || out_channels % 16 != 0 ||
        (taps * channels) % 64 != 0)
        return hipErrorInvalidValue;
    const uint64_t total = taps * channels * out_channels;
    dispatch(weights_pack_kernel, dim3(ceil_div(total, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), dst, src, out_channels, channels,
                       static_cast<uint32_t>(taps), ldb);
    return hipGetLastError();
}

int dav2_hip_conv2d_i8_supported(uint32_t width, uint32_t height, uint32_t channels, uint32_t out_channels,
                                 uint32_t kernel, uint32_t stride, uint32_t padding) {
    return width > 0 && height > 0 && height <= 65535u && (kernel == 3 || kernel == 1) && stride == 1 &&
           padding == (kernel - 1) / 2 && channels > 0 && channels % kCB == 0 && out_channels > 0 &&
           out_channels % 32 == 0 && static_cast<uint64_t>(width) * height < (1ull << 31);
}

int dav2_hip_conv2d_i8_emits(uint32_t out_channels, uint32_t kernel) {
    // launch_ks: 256- and 128-channel tiles give each wave 64 or 32 channels,
    // whole groups; the narrower tiles split a group over waves.
    return (kernel == 1 || kernel == 3) && out_channels > 0 && out_channels % 128 == 0;
}

int dav2_hip_conv2d_i8(const dav2_conv_i8_args* a, void* stream) {
    if (!a) return hipErrorInvalidValue;
    if (!dav2_hip_conv2d_i8_supported(a->width, a->height, a->channels, a->out_channels, a->kernel, 1,
                                      (a->kernel - 1) / 2))
        return hipErrorInvalidValue;
    if (!a->input || !a->weight || !a->weight_scales || !a->out || (!a->scratch && !a->partial_in))
        return hipErrorInvalidValue;
    const uint64_t plane = static_cast<uint64_t>(a->width) * a->height;
    const uint32_t groups = channel_groups(a->channels);
    if (!a->partial_in && a->scratch_floats < plane * groups) return hipErrorInvalidValue;
    const uint32_t emit = a->flags & (DAV2_CONV_EMIT_ABSMAX | DAV2_CONV_EMIT_RELU_MAX);
    if (emit == (DAV2_CONV_EMIT_ABSMAX | DAV2_CONV_EMIT_RELU_MAX) ||
        (emit && (!a->partial_out || !dav2_hip_conv2d_i8_emits(a->out_channels, a->kernel))))
        return hipErrorInvalidValue;
    // The kernels address input and weights with 32-bit byte offsets; the
    // 3x3 kernel's buffer offsets of one channel block stay below 2^31.
    if (plane * a->channels * sizeof(float) >= (1ull << 32) || plane * kCB * sizeof(float) >= (1ull << 31) ||
        static_cast<uint64_t>(a->out_channels) * a->kernel * a->kernel * a->channels >= (1ull << 32))
        return hipErrorInvalidValue;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (a->flags & ~static_cast<uint32_t>(DAV2_CONV_RELU_INPUT | DAV2_CONV_RELU_OUTPUT | DAV2_CONV_EMIT_ABSMAX |
                                          DAV2_CONV_EMIT_RELU_MAX))
        return hipErrorInvalidValue;
    if (!a->partial_in) {
        const hipError_t e = launch_channel_group_absmax(a->input, a->channels, plane, a->scratch,
                                                         (a->flags & DAV2_CONV_RELU_INPUT) != 0, s);
        if (e != hipSuccess) return e;
    }
    ConvParams g;
    g.x = a->input;
    g.partial = a->partial_in ? a->partial_in : a->scratch;
    g.groups = groups;
    g.channels = a->channels;
    g.height = a->height;
    g.width = a->width;
    g.plane = plane;
    // 3x3: the two-row kernel needs an even width and an 8-byte aligned
    // input (8-byte column-pair loads); other maps take conv_i8_kernel.
    const bool two_row = a->kernel == 3 && a->width % 2 == 0 && reinterpret_cast<uintptr_t>(a->input) % 8 == 0;
    g.tiles_x = two_row ? ceil_div(a->width, kTileCols3) : ceil_div(a->width, kPix);
    g.w = a->weight;
    g.n_out = a->out_channels;
    g.w_scales = a->weight_scales;
    g.bias = a->bias;
    g.out = a->out;
    g.residual = a->residual;
    g.flags = a->flags;
    g.emit = emit ? a->partial_out : nullptr;
    if (two_row) return launch_conv3x3_i8(g, g.tiles_x * ceil_div(a->height, 2), a->out_channels, s);
    if (a->kernel == 3) launch_ks<3>(g, g.tiles_x * a->height, a->out_channels, s);
    else launch_ks<1>(g, ceil_div(plane, kPix), a->out_channels, s);
    return hipGetLastError();
}

int dav2_hip_conv1x1_narrow_i8(const float* input, uint32_t width, uint32_t height, uint32_t channels,
                               const int8_t* weight, uint32_t ldw, const float* weight_scales, const float* bias,
                               uint32_t out_channels, float* out, float* pre_relu, uint32_t flags, void* stream) {
    const uint64_t plane = static_cast<uint64_t>(width) * height;
    if (plane == 0 || out_channels == 0) return hipSuccess;
    if (!input || !weight || !weight_scales || !out || channels == 0 || channels > kNarrowC ||
        out_channels > kNarrowN || ldw < channels ||
        (flags & ~static_cast<uint32_t>(DAV2_CONV_RELU_INPUT | DAV2_CONV_RELU_OUTPUT)))
        return hipErrorInvalidValue;
    const bool pairs = channels == 32u && plane % 2u == 0u &&
                       ((reinterpret_cast<uintptr_t>(input) | reinterpret_cast<uintptr_t>(out) |
                         reinterpret_cast<uintptr_t>(pre_relu)) & 7u) == 0u;
    if (pairs)
        dispatch(conv1x1_narrow_pairs_kernel<32>, dim3(ceil_div(plane / 2u, 256)), dim3(256), 0,
                 static_cast<hipStream_t>(stream), input, plane, weight, ldw, weight_scales, bias, out_channels, out,
                 pre_relu, flags);
    else
        dispatch(conv1x1_narrow_kernel, dim3(ceil_div(plane, 256)), dim3(256), 0,
                 static_cast<hipStream_t>(stream), input, plane, channels, weight, ldw, weight_scales, bias,
                 out_channels, out, pre_relu, flags);
    return hipGetLastError();
}

}  // extern "C"
