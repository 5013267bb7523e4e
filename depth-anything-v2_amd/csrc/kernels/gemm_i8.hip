// int8 x int8 -> int32 GEMM on CDNA4 matrix cores (v_mfma_i32_16x16x64_i8)
// with fused dequant / bias / GELU / LayerScale-residual / CHW / ConvTranspose
// epilogues. Reference semantics: linear_int8_tiled.glsl:40-117 and
// conv_transpose_int8.glsl:31-58.
//
// Operands are K-contiguous ("NT"): activations A[m][lda], weights B[n][ldb],
// K a multiple of 64 with zero padding. Internally the kernel computes
// D[p][q] = sum_k P[p][k] * Q[q][k]; row-major epilogues use (P, Q) = (A, B),
// channel-major ones use (P, Q) = (B, A) so the lanes of one MFMA column run
// along output pixels and their stores coalesce.
//
// Tiling: a workgroup owns a BM x BN output tile, its waves a (BM/WAVES_M) x
// (BN/WAVES_N) sub-tile of 16x16 MFMA blocks. K advances in stages of BK
// bytes copied straight from global memory into an LDS ring of STAGES slots
// (global_load_lds_dwordx4, no register staging), XOR-swizzled so the MFMA
// operand reads are free of bank conflicts; the copies of the next
// STAGES - 1 stages are in flight while a stage is multiplied, with one
// workgroup barrier per stage. Workgroups are remapped so that each XCD
// works on one contiguous band of tiles.

#include "common.h"
#include "dav2_hip.h"

using namespace dav2k;

namespace {


struct GemmParams {
    const int8_t* p;
    const int8_t* q;
    uint64_t ldp, ldq;
    uint32_t rows_p, rows_q, k;
    uint32_t n;  // logical weight rows
    const float* a_scales;
    const float* b_scales;
    const float* bias;
    int32_t* out_i32;
    float* out;
    uint64_t out_row_offset, out_row_stride;
    const float* residual;
    const float* gamma;
    uint32_t convt_k, convt_w, convt_h, convt_c;
};

DAV2_DEV float dequant(int32_t acc, float s_in, float s_w, float b) {
    float v = static_cast<float>(acc);
    v = v * s_in;
    v = v * s_w;
    return v + b;
}

DAV2_DEV float gelu_erf(float v) {
    return gelu_erfcc(v);
}

template <int EPI>
struct Orientation {
    // Channel-major epilogues swap operands (see file comment).
    static constexpr bool swapped = EPI == DAV2_GEMM_EPI_TRANSPOSED || EPI == DAV2_GEMM_EPI_CONVT;
};

template <int EPI>
DAV2_DEV void store_one(const GemmParams& g, uint32_t prow, uint32_t qcol, int32_t acc) {
    const bool sw = Orientation<EPI>::swapped;
    const uint32_t m = sw ? qcol : prow;
    const uint32_t n = sw ? prow : qcol;
    if (EPI == DAV2_GEMM_EPI_RAW_I32) {
        g.out_i32[static_cast<uint64_t>(m) * g.n + n] = acc;
        return;
    }
    if (EPI == DAV2_GEMM_EPI_CONVT) {
        const uint32_t k = g.convt_k;
        const uint32_t iy = m / g.convt_w, ix = m - iy * g.convt_w;
        const uint32_t kidx = n / g.convt_c, oc = n - kidx * g.convt_c;
        const uint32_t ky = kidx / k, kx = kidx - ky * k;
        const uint32_t ow = g.convt_w * k, oh = g.convt_h * k;
        const uint64_t idx = (static_cast<uint64_t>(oc) * oh + iy * k + ky) * ow + ix * k + kx;
        g.out[idx] = dequant(acc, g.a_scales[m], g.b_scales[n], g.bias[oc]);
        return;
    }
    const float v = dequant(acc, g.a_scales[m], g.b_scales[n], g.bias ? g.bias[n] : 0.0f);
    if (EPI == DAV2_GEMM_EPI_TRANSPOSED) {
        g.out[static_cast<uint64_t>(n) * g.out_row_stride + m + g.out_row_offset] = v;
        return;
    }
    const uint64_t idx = (static_cast<uint64_t>(m) + g.out_row_offset) * g.n + n;
    if (EPI == DAV2_GEMM_EPI_ROW) {
        g.out[idx] = v;
    } else if (EPI == DAV2_GEMM_EPI_ROW_GELU) {
        g.out[idx] = gelu_erf(v);
    } else if (EPI == DAV2_GEMM_EPI_ROW_LAYERSCALE) {
        // add_scaled.glsl:26-30: residual + (addend * gamma), no contraction.
        const float scaled = v * g.gamma[n];
        g.out[idx] = g.residual[idx] + scaled;
    }
}

// Tile index of this workgroup. Workgroups are dealt to the 8 XCDs round
// robin (id % 8); remap so that each XCD owns one contiguous run of tiles,
// ordered along M first: the tiles of one weight-column band then share that
// XCD's L2.
DAV2_DEV void tile_of(uint32_t& tm, uint32_t& tn) {
    const uint32_t mt = gridDim.x, total = gridDim.x * gridDim.y;
    const uint32_t id = blockIdx.y * gridDim.x + blockIdx.x;
    const uint32_t xcd = id & 7u, idx = id >> 3;
    const uint32_t base = total >> 3, extra = total & 7u;
    const uint32_t lin = xcd * base + min(xcd, extra) + idx;
    tm = lin % mt;
    tn = lin / mt;
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 16 bytes per lane from global memory straight into LDS
// (global_load_lds_dwordx4): lane l's bytes land at lds_base + 16*l; the
// base must be the same for the whole wave.
DAV2_DEV void copy16_to_lds(const int8_t* src, int8_t* lds_base) {
    __builtin_amdgcn_global_load_lds(src, (lds_ptr_t)lds_base, 16, 0, 0);
}

// LDS byte offset of logical 16-byte chunk c of row r in a stage of BK-byte
// rows: chunks are XOR-swizzled with the row's 256-byte period index, so the
// 16 rows that one MFMA operand load reads at the same logical chunk hit 16
// distinct bank groups (256 bytes = all banks once).
template <int BK>
DAV2_DEV uint32_t swz(uint32_t r, uint32_t c) {
    constexpr uint32_t cpr = BK / 16, rows_per_period = 256 / BK;
    return r * BK + ((c ^ ((r / rows_per_period) & (cpr - 1))) << 4);
}

// s_waitcnt with vmcnt = n (expcnt, lgkmcnt not waited on), n < 64.
#define DAV2_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

template <int BM, int BN, int WAVES_M, int WAVES_N, int BK, int STAGES, int EPI>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void gemm_i8_kernel(GemmParams g) {
    constexpr int NW = WAVES_M * WAVES_N;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int TM = WM / 16, TN = WN / 16;
    constexpr int kBK = BK;
    constexpr int CPR = BK / 16;                  // 16-byte chunks per row
    constexpr int STAGE_BYTES = (BM + BN) * BK;
    // one global_load_lds_dwordx4 moves 64 x 16 bytes = 1024 / BK rows
    constexpr int RPL = 1024 / BK;
    constexpr int LOADS = (BM + BN) / RPL;        // per stage, all waves
    constexpr int LOADS_PER_WAVE = LOADS / NW;
    static_assert(BK == 64 || BK == 128 || BK == 256, "stage depth");
    static_assert(STAGES >= 2 && STAGES <= 4 && 2 * LOADS_PER_WAVE < 64, "pipeline depth / vmcnt range");
    static_assert(LOADS % NW == 0 && BM % RPL == 0, "stage rows must split evenly over the waves");
    static_assert(TM >= 1 && TN >= 1, "wave tile must hold at least one MFMA block");

    extern __shared__ __attribute__((aligned(16))) int8_t smem[];  // [STAGES][BM + BN][128]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    uint32_t tm, tn;
    tile_of(tm, tn);
    const uint32_t row0 = tm * BM;
    const uint32_t col0 = tn * BN;
    // K is a multiple of 64: full stages, then possibly a partial one
    const int ksteps = static_cast<int>((g.k + kBK - 1) / kBK);

    // Loads of this wave: instruction i covers stage rows RPL*(wave*LPW + i)
    // .. +RPL-1; lane l brings row +l/CPR, physical chunk l%CPR, i.e. the
    // logical chunk that swz maps there. Rows past the matrix read a valid
    // row (their results are never stored); chunks past K are never
    // multiplied.
    const int8_t* src[LOADS_PER_WAVE];
    uint32_t chunk_bytes[LOADS_PER_WAVE];
#pragma unroll
    for (int i = 0; i < LOADS_PER_WAVE; ++i) {
        const uint32_t srow = RPL * (wave * LOADS_PER_WAVE + i) + lane / CPR;  // stage row
        chunk_bytes[i] = ((lane % CPR) ^ ((srow / (256 / BK)) & (CPR - 1))) * 16u;
        if (srow < static_cast<uint32_t>(BM)) {  // uniform per instruction (BM % RPL == 0)
            const uint32_t r = min(row0 + srow, g.rows_p - 1);
            src[i] = g.p + r * g.ldp + chunk_bytes[i];
        } else {
            const uint32_t r = min(col0 + srow - BM, g.rows_q - 1);
            src[i] = g.q + r * g.ldq + chunk_bytes[i];
        }
    }
    auto issue = [&](int ks) {
        const int slot = ks % STAGES;
        const uint32_t kofs = static_cast<uint32_t>(ks) * kBK;
#pragma unroll
        for (int i = 0; i < LOADS_PER_WAVE; ++i) {
            // In a partial stage chunks past K re-read bytes of the same row
            // inside K (never multiplied).
            int64_t off = static_cast<int64_t>(kofs);
            while (off + chunk_bytes[i] >= g.k) off -= 64;
            copy16_to_lds(src[i] + off, smem + slot * STAGE_BYTES + (wave * LOADS_PER_WAVE + i) * 1024);
        }
    };

    v4i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < ksteps) issue(s);

    const int frag_row = lane & 15;
    const int frag_c = lane >> 4;  // logical chunk within a 64-byte k step
    for (int ks = 0; ks < ksteps; ++ks) {
        // stage ks has landed once only the loads of the stages after it are
        // outstanding
        // loads complete in order: after stage ks only the stages issued
        // after it (at most STAGES - 2 of them) may still be in flight
        const int later = min(STAGES - 2, ksteps - 1 - ks);
        if (later >= 2) {
            DAV2_WAIT_VMCNT(2 * LOADS_PER_WAVE);
        } else if (later == 1) {
            DAV2_WAIT_VMCNT(LOADS_PER_WAVE);
        } else {
            DAV2_WAIT_VMCNT(0);
        }
        // Plain barrier: the wait above already covers this wave's copies of
        // stage ks, and the slot refilled next was last read by operands the
        // MFMAs of the previous stage consumed. (__syncthreads would also
        // drain the copies of stage ks + 1.)
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if (ks + STAGES - 1 < ksteps) issue(ks + STAGES - 1);
        const int8_t* st = smem + (ks % STAGES) * STAGE_BYTES;
        const int ksub = min(static_cast<int>((g.k - static_cast<uint32_t>(ks) * kBK) / 64), BK / 64);
#pragma unroll
        for (int kk = 0; kk < BK / 64; ++kk) {
            if (kk < ksub) {
                v4i af[TM], bf[TN];
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const uint32_t r = wm * WM + i * 16 + frag_row;
                    af[i] = *reinterpret_cast<const v4i*>(st + swz<BK>(r, kk * 4 + frag_c));
                }
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const uint32_t r = BM + wn * WN + j * 16 + frag_row;
                    bf[j] = *reinterpret_cast<const v4i*>(st + swz<BK>(r, kk * 4 + frag_c));
                }
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
        }
    }

    // 16x16 MFMA result layout: lane l holds rows 4*(l/16)+r (r = 0..3) of
    // column l%16.
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint32_t qcol = col0 + wn * WN + j * 16 + (lane & 15);
            if (qcol >= g.rows_q) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t prow = row0 + wm * WM + i * 16 + 4 * (lane >> 4) + r;
                if (prow < g.rows_p) store_one<EPI>(g, prow, qcol, acc[i][j][r]);
            }
        }
    }
}

template <int BM, int BN, int WMW, int WNW, int BK, int STAGES, int EPI>
void launch_cfg(const GemmParams& g, hipStream_t s) {
    constexpr size_t lds = static_cast<size_t>(STAGES) * (BM + BN) * BK;
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(gemm_i8_kernel<BM, BN, WMW, WNW, BK, STAGES, EPI>),
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    (void)attr;
    const dim3 grid(ceil_div(g.rows_p, BM), ceil_div(g.rows_q, BN));
    hipLaunchKernelGGL((gemm_i8_kernel<BM, BN, WMW, WNW, BK, STAGES, EPI>), grid, dim3(64 * WMW * WNW), lds, s, g);
}

template <int EPI>
void launch_epi(const GemmParams& g, hipStream_t s) {
    // Measured on MI355X for the ViT-L encoder shapes (M = 1370, K = 1024 /
    // 4096): 64x64 tiles with four waves, 128-byte stages and a three-stage
    // ring beat every larger tile (more workgroups in flight hide the load
    // latency better) and match the vendor int8 GEMM. Channel-major GEMMs
    // with few output channels use 32-row tiles.
    if (g.rows_p <= 32) launch_cfg<32, 64, 1, 2, 128, 3, EPI>(g, s);
    else launch_cfg<64, 64, 2, 2, 128, 3, EPI>(g, s);
}

}  // namespace

extern "C" int dav2_hip_gemm_i8(const dav2_gemm_i8_args* a, void* stream) {
    if (!a) return hipErrorInvalidValue;
    if (a->m == 0 || a->n == 0) return hipSuccess;
    if (!a->a || !a->b || a->k == 0 || a->k % 64 || a->lda < a->k || a->ldb < a->k ||
        a->lda % 16 || a->ldb % 16 || (reinterpret_cast<uintptr_t>(a->a) & 15) ||
        (reinterpret_cast<uintptr_t>(a->b) & 15))
        return hipErrorInvalidValue;
    const uint32_t e = a->epilogue;
    if (e == DAV2_GEMM_EPI_RAW_I32 ? !a->out_i32 : (!a->out || !a->a_scales || !a->b_scales))
        return hipErrorInvalidValue;
    if (e == DAV2_GEMM_EPI_ROW_LAYERSCALE && (!a->residual || !a->gamma)) return hipErrorInvalidValue;
    if (e == DAV2_GEMM_EPI_CONVT &&
        (!a->bias || a->convt_kernel == 0 || a->convt_channels == 0 || a->convt_width == 0 || a->convt_height == 0 ||
         static_cast<uint64_t>(a->convt_width) * a->convt_height != a->m ||
         static_cast<uint64_t>(a->convt_kernel) * a->convt_kernel * a->convt_channels != a->n))
        return hipErrorInvalidValue;
    if (e > DAV2_GEMM_EPI_CONVT) return hipErrorInvalidValue;

    GemmParams g{};
    const bool swapped = e == DAV2_GEMM_EPI_TRANSPOSED || e == DAV2_GEMM_EPI_CONVT;
    g.p = swapped ? a->b : a->a;
    g.ldp = swapped ? a->ldb : a->lda;
    g.rows_p = swapped ? a->n : a->m;
    g.q = swapped ? a->a : a->b;
    g.ldq = swapped ? a->lda : a->ldb;
    g.rows_q = swapped ? a->m : a->n;
    g.k = a->k;
    g.n = a->n;
    g.a_scales = a->a_scales;
    g.b_scales = a->b_scales;
    g.bias = a->bias;
    g.out_i32 = a->out_i32;
    g.out = a->out;
    g.out_row_offset = a->out_row_offset;
    g.out_row_stride = a->out_row_stride;
    g.residual = a->residual;
    g.gamma = a->gamma;
    g.convt_k = a->convt_kernel;
    g.convt_w = a->convt_width;
    g.convt_h = a->convt_height;
    g.convt_c = a->convt_channels;
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (e) {
        case DAV2_GEMM_EPI_RAW_I32: launch_epi<DAV2_GEMM_EPI_RAW_I32>(g, s); break;
        case DAV2_GEMM_EPI_ROW: launch_epi<DAV2_GEMM_EPI_ROW>(g, s); break;
        case DAV2_GEMM_EPI_ROW_GELU: launch_epi<DAV2_GEMM_EPI_ROW_GELU>(g, s); break;
        case DAV2_GEMM_EPI_ROW_LAYERSCALE: launch_epi<DAV2_GEMM_EPI_ROW_LAYERSCALE>(g, s); break;
        case DAV2_GEMM_EPI_TRANSPOSED: launch_epi<DAV2_GEMM_EPI_TRANSPOSED>(g, s); break;
        case DAV2_GEMM_EPI_CONVT: launch_epi<DAV2_GEMM_EPI_CONVT>(g, s); break;
    }
    return hipGetLastError();
}
