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

#include <type_traits>

#include "common.h"
#include <hip/hip_ext.h>
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
    uint32_t coalesced_out;  // row-major output rows 16-byte aligned (n % 4 == 0, out aligned)
    uint32_t nontemporal_out;  // coalesced row-major stores bypass the caches (see the store)
    float* col_absmax;       // ROW_COLMAX partial maxima [row tile][n - col_absmax_begin]
    uint32_t col_absmax_begin;
    uint32_t relu_output;    // TRANSPOSED: max(out, 0) after the residual
    uint32_t k_split;        // K bytes per blockIdx.z slice (multiple of 128; == k without split-K)
};

// Split-K slices of a channel-major GEMM store their int32 sums here:
// out_i32[(slice * rows_p + prow) * rows_q + qcol]; a second kernel adds the
// slices (exact) and applies the TRANSPOSED epilogue.
constexpr int kEpiSplitPartial = 100;

template <int EPI>
constexpr bool row_major_epi() {
    return EPI == DAV2_GEMM_EPI_ROW || EPI == DAV2_GEMM_EPI_ROW_GELU || EPI == DAV2_GEMM_EPI_ROW_LAYERSCALE ||
           EPI == DAV2_GEMM_EPI_ROW_COLMAX;
}

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
    static constexpr bool swapped =
        EPI == DAV2_GEMM_EPI_TRANSPOSED || EPI == DAV2_GEMM_EPI_CONVT || EPI == kEpiSplitPartial;
};

// Epilogue operands of one lane, loaded before the K loop so that no global
// load latency falls between the last MFMA and the stores. "p" values follow
// the lane's output rows of operand P (16i + 4(l/16) + r), "q" values its
// columns (16j + l%16); rows and columns past the matrix load a valid element
// whose result is never stored.
template <int EPI, int TM, int TN>
struct EpilogueOperands {
    static constexpr bool kSwapped = Orientation<EPI>::swapped;
    static constexpr bool kScales = EPI != DAV2_GEMM_EPI_RAW_I32 && EPI != kEpiSplitPartial;
    static constexpr bool kLayerScale = EPI == DAV2_GEMM_EPI_ROW_LAYERSCALE;
    float ps[TM][4];  // scale of the P row: a_scales[m] (row-major) or b_scales[n] (swapped)
    float pb[TM][4];  // bias of the P row (swapped)
    float qs[TN];     // scale of the Q column: b_scales[n] (row-major) or a_scales[m] (swapped)
    float qb[TN];     // bias of the Q column (row-major)
    float qg[TN];     // LayerScale gamma
    float res[kLayerScale ? TM : 1][kLayerScale ? TN : 1][4];

    DAV2_DEV void load(const GemmParams& g, uint32_t prow0, uint32_t qcol0, int lane) {
        if (!kScales) return;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint32_t qc = min(qcol0 + j * 16 + (lane & 15), g.rows_q - 1);
            qs[j] = kSwapped ? g.a_scales[qc] : g.b_scales[qc];
            if (!kSwapped) {
                qb[j] = g.bias ? g.bias[qc] : 0.0f;
                if (kLayerScale) qg[j] = g.gamma[qc];
            }
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t pr = min(prow0 + i * 16 + 4 * (lane >> 4) + r, g.rows_p - 1);
                ps[i][r] = kSwapped ? g.b_scales[pr] : g.a_scales[pr];
                if (EPI == DAV2_GEMM_EPI_CONVT) {
                    const uint32_t kidx = pr / g.convt_c;
                    pb[i][r] = g.bias[pr - kidx * g.convt_c];
                } else if (kSwapped) {
                    pb[i][r] = g.bias ? g.bias[pr] : 0.0f;
                }
                if (kLayerScale) {
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        const uint32_t qc = min(qcol0 + j * 16 + (lane & 15), g.rows_q - 1);
                        res[i][j][r] = g.residual[(static_cast<uint64_t>(pr) + g.out_row_offset) * g.n + qc];
                    }
                }
            }
    }
};

// Final value of a row-major epilogue from the dequantized v.
template <int EPI, int TM, int TN>
DAV2_DEV float row_value(const EpilogueOperands<EPI, TM, TN>& e, int i, int j, int r, float v) {
    if (EPI == DAV2_GEMM_EPI_ROW_GELU) return gelu_erf(v);
    if (EPI == DAV2_GEMM_EPI_ROW_LAYERSCALE) {
        // add_scaled.glsl:26-30: residual + (addend * gamma), no contraction.
        constexpr bool ls = EpilogueOperands<EPI, TM, TN>::kLayerScale;
        const float scaled = v * e.qg[j];
        return e.res[ls ? i : 0][ls ? j : 0][r] + scaled;
    }
    return v;
}

// One output element (row prow of P, column qcol of Q) of block (i, j),
// accumulator r: dequant ((acc * s_in) * s_w) + bias, then the epilogue;
// TRANSPOSED adds the residual at the same index (RES, add.glsl) and then
// takes max(., 0) (RELU, relu.glsl).
template <int EPI, int TM, int TN, bool RES = false, bool RELU = false>
DAV2_DEV void store_one(const GemmParams& g, const EpilogueOperands<EPI, TM, TN>& e, int i, int j, int r,
                        uint32_t prow, uint32_t qcol, int32_t acc) {
    constexpr bool sw = Orientation<EPI>::swapped;
    const uint32_t m = sw ? qcol : prow;
    const uint32_t n = sw ? prow : qcol;
    if (EPI == DAV2_GEMM_EPI_RAW_I32) {
        g.out_i32[static_cast<uint64_t>(m) * g.n + n] = acc;
        return;
    }
    if (EPI == kEpiSplitPartial) {
        g.out_i32[(static_cast<uint64_t>(blockIdx.z) * g.rows_p + prow) * g.rows_q + qcol] = acc;
        return;
    }
    const float s_in = sw ? e.qs[j] : e.ps[i][r];
    const float s_w = sw ? e.ps[i][r] : e.qs[j];
    const float b = sw ? e.pb[i][r] : e.qb[j];
    const float v = dequant(acc, s_in, s_w, b);
    if (EPI == DAV2_GEMM_EPI_CONVT) {
        const uint32_t k = g.convt_k;
        const uint32_t iy = m / g.convt_w, ix = m - iy * g.convt_w;
        const uint32_t kidx = n / g.convt_c, oc = n - kidx * g.convt_c;
        const uint32_t ky = kidx / k, kx = kidx - ky * k;
        const uint32_t ow = g.convt_w * k, oh = g.convt_h * k;
        const uint64_t idx = (static_cast<uint64_t>(oc) * oh + iy * k + ky) * ow + ix * k + kx;
        g.out[idx] = v;
        return;
    }
    if (EPI == DAV2_GEMM_EPI_TRANSPOSED) {
        const uint64_t idx = static_cast<uint64_t>(n) * g.out_row_stride + m + g.out_row_offset;
        float o = v;
        if (RES) o = o + g.residual[idx];
        if (RELU) o = fmaxf(o, 0.0f);
        g.out[idx] = o;
        return;
    }
    const uint64_t idx = (static_cast<uint64_t>(m) + g.out_row_offset) * g.n + n;
    g.out[idx] = row_value<EPI, TM, TN>(e, i, j, r, v);
}

// Waits until at most `later` stages' copies (LPW per stage and wave) are
// outstanding; later <= MAX (the counts must be immediates).
template <int MAX, int LPW>
DAV2_DEV void wait_stages(int later) {
    if constexpr (MAX <= 0) {
        DAV2_WAIT_VMCNT(0);
    } else {
        if (later >= MAX) DAV2_WAIT_VMCNT(MAX * LPW);
        else wait_stages<MAX - 1, LPW>(later);
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


// LDS byte offset of logical 16-byte chunk c of row r in a stage of BK-byte
// rows: chunks are XOR-swizzled with the row's 256-byte period index, so the
// 16 rows that one MFMA operand load reads at the same logical chunk hit 16
// distinct bank groups (256 bytes = all banks once).
template <int BK>
DAV2_DEV uint32_t swz(uint32_t r, uint32_t c) {
    constexpr uint32_t cpr = BK / 16, rows_per_period = 256 / BK;
    return r * BK + ((c ^ ((r / rows_per_period) & (cpr - 1))) << 4);
}


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
    static_assert(STAGES >= 2 && STAGES <= 8 && (STAGES - 2) * LOADS_PER_WAVE < 64, "pipeline depth / vmcnt range");
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
    // This workgroup's K slice (all of K without split-K): kbase is a
    // multiple of 128, klen a multiple of 64 -- full stages, then possibly a
    // partial one.
    const uint32_t kbase = blockIdx.z * g.k_split;
    const uint32_t klen = min(g.k_split, g.k - kbase);
    const int ksteps = static_cast<int>((klen + kBK - 1) / kBK);

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
            src[i] = g.p + r * g.ldp + kbase + chunk_bytes[i];
        } else {
            const uint32_t r = min(col0 + srow - BM, g.rows_q - 1);
            src[i] = g.q + r * g.ldq + kbase + chunk_bytes[i];
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
            while (off + chunk_bytes[i] >= klen) off -= 64;
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
    // Epilogue operands: issued after the first stages' copies, waited for
    // only at the stores.
    EpilogueOperands<EPI, TM, TN> epi;
    epi.load(g, row0 + wm * WM, col0 + wn * WN, lane);

    const int frag_row = lane & 15;
    const int frag_c = lane >> 4;  // logical chunk within a 64-byte k step
    for (int ks = 0; ks < ksteps; ++ks) {
        // stage ks has landed once only the loads of the stages after it are
        // outstanding
        // loads complete in order: after stage ks only the stages issued
        // after it (at most STAGES - 2 of them) may still be in flight
        wait_stages<STAGES - 2, LOADS_PER_WAVE>(min(STAGES - 2, ksteps - 1 - ks));
        // Plain barrier: the wait above already covers this wave's copies of
        // stage ks, and the slot refilled next was last read by operands the
        // MFMAs of the previous stage consumed. (__syncthreads would also
        // drain the copies of stage ks + 1.)
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if (ks + STAGES - 1 < ksteps) issue(ks + STAGES - 1);
        const int8_t* st = smem + (ks % STAGES) * STAGE_BYTES;
        const int ksub = min(static_cast<int>((klen - static_cast<uint32_t>(ks) * kBK) / 64), BK / 64);
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

    // Row-major epilogues: the final values go through LDS so that each
    // store writes whole 256-byte row segments (16 lanes x float4) instead
    // of 64-byte pieces of four rows.
    constexpr bool kRowMajor = row_major_epi<EPI>();
    constexpr bool kColMax = EPI == DAV2_GEMM_EPI_ROW_COLMAX;
    constexpr int kOutStride = BN + 4;  // floats; rows 4 apart start 16 banks apart (launch_cfg sizes LDS for it)
    if (kRowMajor && (kColMax || g.coalesced_out)) {
        float* tile = reinterpret_cast<float*>(smem);
        __syncthreads();  // every wave is done with the last stage's operands
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int lr = wm * WM + i * 16 + 4 * (lane >> 4) + r, lc = wn * WN + j * 16 + (lane & 15);
                    const float v = dequant(acc[i][j][r], epi.ps[i][r], epi.qs[j], epi.qb[j]);
                    tile[lr * kOutStride + lc] = row_value<EPI, TM, TN>(epi, i, j, r, v);
                }
        __syncthreads();
        constexpr int kLanesPerRow = BN / 4, kRowsPerPass = 64 * NW / kLanesPerRow;
        const int c4 = (tid % kLanesPerRow) * 4;
        const uint32_t col = col0 + c4;
        float4 cmax = make_float4(0.f, 0.f, 0.f, 0.f);  // column maxima over this thread's rows
#pragma unroll
        for (int rr = tid / kLanesPerRow; rr < BM; rr += kRowsPerPass) {
            const uint32_t row = row0 + rr;
            if (row >= g.rows_p) break;
            const float4 v = *reinterpret_cast<const float4*>(tile + rr * kOutStride + c4);
            if (kColMax) {
                cmax.x = fmaxf(cmax.x, fabsf(v.x));
                cmax.y = fmaxf(cmax.y, fabsf(v.y));
                cmax.z = fmaxf(cmax.z, fabsf(v.z));
                cmax.w = fmaxf(cmax.w, fabsf(v.w));
            }
            float* dst = g.out + (static_cast<uint64_t>(row) + g.out_row_offset) * g.n + col;
            if (col + 3 < g.rows_q) {
                if (g.nontemporal_out)
                    store_nt(dst, v);
                else
                    *reinterpret_cast<float4*>(dst) = v;
            } else {
                if (col < g.rows_q) dst[0] = v.x;
                if (col + 1 < g.rows_q) dst[1] = v.y;
                if (col + 2 < g.rows_q) dst[2] = v.z;
            }
        }
        if constexpr (kColMax) if (col0 >= g.col_absmax_begin) {
            // lanes l, l ^ 16, l ^ 32, l ^ 48 of a wave hold the same columns
            static_assert(kLanesPerRow == 16 && BM * kOutStride * 4 + NW * BN * 4 <=
                          (BM * kOutStride * 4 > STAGES * (BM + BN) * BK ? BM * kOutStride * 4 : STAGES * (BM + BN) * BK),
                          "column maxima: 16 lanes per row, partials fit behind the output tile");
#pragma unroll
            for (int o = 16; o < 64; o <<= 1) {
                cmax.x = fmaxf(cmax.x, __shfl_xor(cmax.x, o, kWave));
                cmax.y = fmaxf(cmax.y, __shfl_xor(cmax.y, o, kWave));
                cmax.z = fmaxf(cmax.z, __shfl_xor(cmax.z, o, kWave));
                cmax.w = fmaxf(cmax.w, __shfl_xor(cmax.w, o, kWave));
            }
            float* part = tile + BM * kOutStride;  // [wave][BN]
            if (lane < 16) *reinterpret_cast<float4*>(part + wave * BN + c4) = cmax;
            __syncthreads();
            if (tid < BN && col0 + tid < g.rows_q) {
                float m = part[tid];
#pragma unroll
                for (int w = 1; w < NW; ++w) m = fmaxf(m, part[w * BN + tid]);
                const uint64_t ld = g.rows_q - g.col_absmax_begin;
                g.col_absmax[static_cast<uint64_t>(tm) * ld + (col0 - g.col_absmax_begin) + tid] = m;
            }
        }
        return;
    }
    // 16x16 MFMA result layout: lane l holds rows 4*(l/16)+r (r = 0..3) of
    // column l%16. The TRANSPOSED residual / ReLU choice is made once, outside
    // the unrolled stores.
    auto store_all = [&](auto res_tag, auto relu_tag) {
        constexpr bool kRes = decltype(res_tag)::value, kRelu = decltype(relu_tag)::value;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const uint32_t qcol = col0 + wn * WN + j * 16 + (lane & 15);
                if (qcol >= g.rows_q) continue;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t prow = row0 + wm * WM + i * 16 + 4 * (lane >> 4) + r;
                    if (prow < g.rows_p)
                        store_one<EPI, TM, TN, kRes, kRelu>(g, epi, i, j, r, prow, qcol, acc[i][j][r]);
                }
            }
        }
    };
    if constexpr (EPI == DAV2_GEMM_EPI_TRANSPOSED) {
        if (g.residual) {
            if (g.relu_output) store_all(std::true_type{}, std::true_type{});
            else store_all(std::true_type{}, std::false_type{});
        } else {
            if (g.relu_output) store_all(std::false_type{}, std::true_type{});
            else store_all(std::false_type{}, std::false_type{});
        }
    } else {
        store_all(std::false_type{}, std::false_type{});
    }
}

// dav2_hip_gemm_i8_events: the dispatch hook (dispatch() in common.h) set for
// one dav2_hip_gemm_i8 call, cleared when that call returns.
thread_local bool t_events_for_one_gemm = false;

// Long-K row-major GEMMs of many rows (fc2 at batch 8: 10960 x 1024 x 4096)
// on v_mfma_i32_32x32x32_i8, whose operand fragments carry half the LDS bytes
// per operation of the 16x16x64 form. Lane l holds row l % 32 of each operand
// with K bytes 16 (l / 32) .. + 15; result register r is row 8 (r / 4) +
// 4 (l / 32) + r % 4 of column l % 32 (checked on gfx950 with a one-wave
// probe). BM x 256 tiles (BM 256 or 192) on BM / 16 waves (BM / 64 x 4,
// each 64 x 64 as 2 x 2 blocks of 32 x 32), the same XCD-banded tile order
// and global -> LDS stage ring (two 128-byte stages) as gemm_i8_kernel; K a
// multiple of 128.
// Epilogues ROW and ROW_LAYERSCALE with gemm_i8_kernel's arithmetic. Each
// wave stages its int32 sums in LDS, 32 rows at a time, and reads them back
// row-major, so that one a_scale per row and float4 column operands
// dequantize them and the residual loads and stores are 256-byte row pieces
// (16 lanes x float4): output rows (and the residual's) 16-byte aligned.
typedef int v16i __attribute__((ext_vector_type(16)));
constexpr int kWideBN = 256;
constexpr int kWideOutStride = 72;  // int32 per staged row: rows 4 apart start 32 banks apart

template <int BM>
constexpr size_t wide_lds() {
    constexpr size_t ring = 2u * (BM + kWideBN) * 128u;
    constexpr size_t out = static_cast<size_t>(BM / 16) * 32u * kWideOutStride * 4u;
    return ring > out ? ring : out;
}

template <int BM, int EPI>
__global__ __launch_bounds__(4 * BM) void gemm_i8_wide_kernel(GemmParams g) {
    static_assert(EPI == DAV2_GEMM_EPI_ROW || EPI == DAV2_GEMM_EPI_ROW_LAYERSCALE, "row-major epilogues");
    static_assert(BM % 64 == 0 && wide_lds<BM>() <= 160u * 1024u, "64-row waves, LDS per CU");
    constexpr int BK = 128, CPR = BK / 16, RPL = 1024 / BK, STAGES = 2;
    constexpr int NW = BM / 16, WAVES_N = 4, WM = 64, WN = 64, TM = WM / 32, TN = WN / 32;
    constexpr int COPIES = (BM + kWideBN) / RPL;  // 1 KiB global -> LDS copies per stage
    constexpr int LPW = (COPIES + NW - 1) / NW;  // copy i * NW + wave of each stage, if < COPIES
    constexpr int STAGE_BYTES = (BM + kWideBN) * BK;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    uint32_t tm, tn;
    tile_of(tm, tn);
    const uint32_t row0 = tm * BM, col0 = tn * kWideBN;
    const int ksteps = static_cast<int>(g.k / BK);
    const int8_t* src[LPW];
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
        const int copy = min(i * NW + wave, COPIES - 1);  // uniform per wave
        const uint32_t srow = RPL * copy + lane / CPR;  // stage row
        const uint32_t chunk = ((lane % CPR) ^ ((srow / (256 / BK)) & (CPR - 1))) * 16u;
        if (srow < static_cast<uint32_t>(BM))  // uniform per instruction
            src[i] = g.p + min(row0 + srow, g.rows_p - 1) * g.ldp + chunk;
        else
            src[i] = g.q + min(col0 + srow - BM, g.rows_q - 1) * g.ldq + chunk;
    }
    auto issue = [&](int ks) {
#pragma unroll
        for (int i = 0; i < LPW; ++i)
            if (i * NW + wave < COPIES)
                copy16_to_lds(src[i] + static_cast<uint32_t>(ks) * BK,
                              smem + (ks % STAGES) * STAGE_BYTES + (i * NW + wave) * 1024);
    };
    v16i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = v16i{};
    issue(0);
    const int fr = lane & 31, fc = lane >> 5;
    for (int ks = 0; ks < ksteps; ++ks) {
        DAV2_WAIT_VMCNT(0);  // stage ks (the only one in flight)
        __builtin_amdgcn_s_barrier();  // every wave's copies of it have landed; the other slot is free
        __builtin_amdgcn_sched_barrier(0);
        if (ks + 1 < ksteps) issue(ks + 1);
        const int8_t* st = smem + (ks % STAGES) * STAGE_BYTES;
#pragma unroll
        for (int kk = 0; kk < BK / 32; ++kk) {
            v4i af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
                af[i] = *reinterpret_cast<const v4i*>(st + swz<BK>(wm * WM + i * 32 + fr, kk * 2 + fc));
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bf[j] = *reinterpret_cast<const v4i*>(st + swz<BK>(BM + wn * WN + j * 32 + fr, kk * 2 + fc));
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    }
    __syncthreads();  // every wave is done with the last stage's operands
    int32_t* stage = reinterpret_cast<int32_t*>(smem) + wave * (32 * kWideOutStride);
    const int c4 = (lane & 15) * 4;
    const uint32_t col = col0 + wn * WN + c4;
    float s_w[4], b[4], gam[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t c = min(col + e, g.rows_q - 1);
        s_w[e] = g.b_scales[c];
        b[e] = g.bias ? g.bias[c] : 0.0f;
        gam[e] = EPI == DAV2_GEMM_EPI_ROW_LAYERSCALE ? g.gamma[c] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                stage[(8 * (r / 4) + 4 * fc + (r % 4)) * kWideOutStride + j * 32 + fr] = acc[i][j][r];
        __syncthreads();  // this wave's rows are staged (waves share no rows)
#pragma unroll
        for (int it = 0; it < 8; ++it) {
            const int lr = it * 4 + (lane >> 4);
            const uint32_t row = row0 + wm * WM + i * 32 + lr;
            if (row >= g.rows_p || col >= g.rows_q) break;  // n % 4 == 0: col + 3 < n as well
            const int4 a = *reinterpret_cast<const int4*>(stage + lr * kWideOutStride + c4);
            const float s_in = g.a_scales[row];
            const int32_t av[4] = {a.x, a.y, a.z, a.w};
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = dequant(av[e], s_in, s_w[e], b[e]);
            const uint64_t idx = (static_cast<uint64_t>(row) + g.out_row_offset) * g.n + col;
            if (EPI == DAV2_GEMM_EPI_ROW_LAYERSCALE) {
                // add_scaled.glsl:26-30: residual + (addend * gamma)
                const float4 res = *reinterpret_cast<const float4*>(g.residual + idx);
                const float rv[4] = {res.x, res.y, res.z, res.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float scaled = v[e] * gam[e];
                    v[e] = rv[e] + scaled;
                }
            }
            *reinterpret_cast<float4*>(g.out + idx) = make_float4(v[0], v[1], v[2], v[3]);
        }
        if (i + 1 < TM) __syncthreads();  // the reads are done before the next block overwrites the stage
    }
}

template <int BM, int EPI>
void launch_wide_bm(const GemmParams& g, hipStream_t s) {
    constexpr size_t lds = wide_lds<BM>();
    static const hipError_t attr =
        hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_i8_wide_kernel<BM, EPI>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    (void)attr;
    const dim3 grid(ceil_div(g.rows_p, BM), ceil_div(g.rows_q, kWideBN), 1);
    dispatch(gemm_i8_wide_kernel<BM, EPI>, grid, dim3(4 * BM), lds, s, g);
}

// One workgroup per CU (MI355X: 256 CUs), so the time goes as the rounds of
// workgroups times the tile height: 192-row tiles unless 256 takes no longer.
// fc2 (N = 1024, K = 4096, LayerScale), us for gemm_i8_kernel / 256-row /
// 192-row tiles on one box: 10960 rows (one round of 172 or 232 tiles)
// 84.3 / 75.0 / 69.8; 21908 rows (two rounds either way) 162.6 / 150.6 / 137.1.
template <int EPI>
void launch_wide(const GemmParams& g, hipStream_t s) {
    constexpr uint32_t kCus = 256;
    const uint32_t tn = ceil_div(g.rows_q, kWideBN);
    auto cost = [&](uint32_t bm) { return ceil_div(static_cast<uint64_t>(ceil_div(g.rows_p, bm)) * tn, kCus) * bm; };
    if (cost(192) < cost(256))
        launch_wide_bm<192, EPI>(g, s);
    else
        launch_wide_bm<256, EPI>(g, s);
}

template <int BM, int BN, int WMW, int WNW, int BK, int STAGES, int EPI>
void launch_cfg(const GemmParams& g, hipStream_t s, bool last = true) {
    // LDS: the stage ring, or the row-major output tile if that is larger.
    constexpr size_t ring = static_cast<size_t>(STAGES) * (BM + BN) * BK;
    constexpr size_t out_tile = static_cast<size_t>(BM) * (BN + 4) * 4;
    constexpr size_t lds = row_major_epi<EPI>() && out_tile > ring ? out_tile : ring;
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(gemm_i8_kernel<BM, BN, WMW, WNW, BK, STAGES, EPI>),
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    (void)attr;
    const dim3 grid(ceil_div(g.rows_p, BM), ceil_div(g.rows_q, BN), ceil_div(g.k, g.k_split));
    (void)last;
    dispatch(gemm_i8_kernel<BM, BN, WMW, WNW, BK, STAGES, EPI>, grid, dim3(64 * WMW * WNW), lds, s, g);
}

// Rows of P from which launch_epi picks 64x128 tiles for the row-major
// epilogues other than the column-maxima one.
constexpr uint32_t kWideTileRows = 4096;

// Columns of Q from which those GEMMs take 128x128 tiles on eight waves.
constexpr uint32_t kWideTileCols = 3072;

// Rows of P per tile of the configuration launch_epi picks: 128 / 64 for the
// 128x128 / 64x128 tiles of the large row-major GEMMs without column maxima
// (rows_p >= kWideTileRows), else 32, 96 or 64 as in the switch below.
// Columns of Q from which the smaller row-major GEMMs without column maxima
// (fc1 at batch 1) take 128x64 tiles on eight waves.
constexpr uint32_t kTallTileCols = 4096;

inline uint32_t tile_rows(uint32_t rows_p, uint32_t rows_q, bool row_major, bool col_max) {
    if (row_major && !col_max && rows_p >= kWideTileRows) return rows_q >= kWideTileCols ? 128 : 64;
    if (row_major && !col_max && rows_q >= kTallTileCols && rows_p >= 512) return 128;
    if (rows_p <= 32) return 32;
    if (row_major && rows_q >= 2048 && rows_p >= 512) return 96;
    return 64;
}

template <int EPI>
void launch_epi(const GemmParams& g, hipStream_t s, bool last = true) {
    // Measured on MI355X for the ViT-L encoder shapes (M = 1370, K = 1024 /
    // 4096, 128-byte stages): for N = 1024 64x64 tiles with a three-stage
    // ring are fastest; for N >= 2048 96x64 tiles with a two-stage ring are
    // (720 workgroups for N = 3072, one round at three per CU, against 1056
    // 64x64 ones). Channel-major GEMMs with few output channels use 32-row
    // tiles.
    // From M = 4096 rows on (ViT-L 518 batch 8: M = 10960) 64x128 tiles
    // with a two-stage ring are fastest for the row-major GEMMs without
    // column maxima (proj / fc1 / fc2: 35 / 126 / 106 us with the tiles
    // below, 29 / 97 / 73 us with these), and from N = 3072 on 128x128 tiles
    // on eight waves of 32x64 (qkv / fc1 at batch 8: 68 -> 64 / 125 -> 115
    // us; fewer columns measured slower); the column-maxima epilogue needs
    // 64-column tiles.
    // Below that, from N = 4096 on (fc1 at batch 1), 128x64 tiles on eight
    // waves of 32x32 (20.4 -> 18.3 us at M = 1370): twice the waves of the
    // 96x64 tiles on the same CUs to hide the operand waits.
    if constexpr (EPI == DAV2_GEMM_EPI_ROW || EPI == DAV2_GEMM_EPI_ROW_LAYERSCALE) {
        // many rows and long K (fc2 from batch 8): the 32x32x32 kernel, whose
        // float4 epilogue needs 16-byte aligned output and residual rows
        if (g.rows_p >= kWideTileRows && g.k >= 4096 && g.k % 128 == 0 && g.k_split == g.k && g.coalesced_out &&
            (EPI != DAV2_GEMM_EPI_ROW_LAYERSCALE || (reinterpret_cast<uintptr_t>(g.residual) & 15) == 0)) {
            launch_wide<EPI>(g, s);
            return;
        }
    }
    if constexpr (row_major_epi<EPI>() && EPI != DAV2_GEMM_EPI_ROW_COLMAX) {
        if (g.rows_p >= kWideTileRows) {
            if (g.rows_q >= kWideTileCols)
                launch_cfg<128, 128, 4, 2, 128, 2, EPI>(g, s, last);
            else
                launch_cfg<64, 128, 2, 2, 128, 2, EPI>(g, s, last);
            return;
        }
        if (g.rows_q >= kTallTileCols && g.rows_p >= 512) {
            launch_cfg<128, 64, 4, 2, 128, 2, EPI>(g, s, last);
            return;
        }
    }
    switch (tile_rows(g.rows_p, g.rows_q, row_major_epi<EPI>(), EPI == DAV2_GEMM_EPI_ROW_COLMAX)) {
        case 32: launch_cfg<32, 64, 1, 2, 128, 3, EPI>(g, s, last); break;
        case 96: launch_cfg<96, 64, 2, 2, 128, 2, EPI>(g, s, last); break;
        default: launch_cfg<64, 64, 2, 2, 128, 3, EPI>(g, s, last); break;
    }
}

// Adds the split-K slices (exact int32 sums) and applies the TRANSPOSED
// epilogue: out[n * stride + m + off] = ((acc * a_scale[m]) * b_scale[n]) +
// bias[n], + residual (add.glsl), max(., 0) (relu.glsl). One thread per
// output, m fastest.
__global__ __launch_bounds__(256) void split_reduce_transposed_kernel(
    const int32_t* __restrict__ partial, uint32_t slices, uint32_t n, uint32_t m, const float* __restrict__ a_scales,
    const float* __restrict__ b_scales, const float* __restrict__ bias, const float* __restrict__ residual,
    uint32_t relu, float* __restrict__ out, uint64_t out_row_stride, uint64_t out_row_offset) {
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    const uint64_t total = static_cast<uint64_t>(n) * m;
    if (idx >= total) return;
    const uint32_t nn = static_cast<uint32_t>(idx / m), mm = static_cast<uint32_t>(idx - static_cast<uint64_t>(nn) * m);
    int32_t acc = 0;
    for (uint32_t z = 0; z < slices; ++z) acc += partial[static_cast<uint64_t>(z) * total + idx];
    float v = dequant(acc, a_scales[mm], b_scales[nn], bias ? bias[nn] : 0.0f);
    const uint64_t o = static_cast<uint64_t>(nn) * out_row_stride + mm + out_row_offset;
    if (residual) v = v + residual[o];
    if (relu) v = fmaxf(v, 0.0f);
    out[o] = v;
}

}  // namespace

extern "C" uint64_t dav2_hip_gemm_i8_split_scratch_bytes(uint32_t m, uint32_t n, uint32_t split_k) {
    return static_cast<uint64_t>(split_k) * m * n * sizeof(int32_t);
}

namespace {

int gemm_i8(const dav2_gemm_i8_args* a, void* stream) {
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
    if (e == DAV2_GEMM_EPI_ROW_COLMAX &&
        (!a->col_absmax || a->col_absmax_begin % 64 || a->col_absmax_begin >= a->n || a->n % 4 ||
         (reinterpret_cast<uintptr_t>(a->out) & 15)))
        return hipErrorInvalidValue;
    if (e > DAV2_GEMM_EPI_ROW_COLMAX) return hipErrorInvalidValue;
    if (a->relu_output && e != DAV2_GEMM_EPI_TRANSPOSED) return hipErrorInvalidValue;
    const bool split = a->split_k > 1;
    if (split && (e != DAV2_GEMM_EPI_TRANSPOSED || a->split_k > 64 || !a->split_scratch ||
                  (reinterpret_cast<uintptr_t>(a->split_scratch) & 3u)))
        return hipErrorInvalidValue;

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
    g.coalesced_out = !swapped && a->n % 4 == 0 && (reinterpret_cast<uintptr_t>(a->out) & 15) == 0;
    // The next kernel reads a row-major output straight back (LayerNorm the
    // LayerScale residual stream, the digit packing qkv, the row quantizer
    // fc1's GELU output), and finding it in the caches gains it more than
    // the GEMM's own nontemporal stores would (nothing left in L2 to write
    // back at the kernel's end). Measured, same-process A/Bs: batch 1,
    // LayerScale +0.2% and qkv with column maxima +0.5% per pass; batch 8,
    // every row-major output +1.0% (digit packing + attention -11 us, row
    // quantizer -1.8 us); except fc1's GELU output below 4096 rows (batch
    // 1: fc1 +1.5 us against -0.7 us for the row quantizer), kept
    // nontemporal.
    g.nontemporal_out = e == DAV2_GEMM_EPI_ROW_GELU && a->m < 4096u;
    g.col_absmax = a->col_absmax;
    g.col_absmax_begin = a->col_absmax_begin;
    g.relu_output = a->relu_output;
    g.k_split = a->k;
    uint32_t slices = 1;
    if (split) {
        // slices of whole 128-byte stages; the last one may be shorter
        g.k_split = ceil_div(ceil_div(a->k, a->split_k), 128) * 128u;
        slices = ceil_div(a->k, g.k_split);
        g.out_i32 = a->split_scratch;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (split && slices > 1) {
        launch_epi<kEpiSplitPartial>(g, s, false);
        const uint64_t total = static_cast<uint64_t>(a->m) * a->n;
        dispatch(split_reduce_transposed_kernel, dim3(ceil_div(total, 256)), dim3(256), 0, s,
                     a->split_scratch, slices, a->n, a->m, a->a_scales, a->b_scales, a->bias, a->residual,
                     a->relu_output, a->out, a->out_row_stride, a->out_row_offset);
        return hipGetLastError();
    }
    if (split) g.out_i32 = a->out_i32;
    switch (e) {
        case DAV2_GEMM_EPI_RAW_I32: launch_epi<DAV2_GEMM_EPI_RAW_I32>(g, s); break;
        case DAV2_GEMM_EPI_ROW: launch_epi<DAV2_GEMM_EPI_ROW>(g, s); break;
        case DAV2_GEMM_EPI_ROW_GELU: launch_epi<DAV2_GEMM_EPI_ROW_GELU>(g, s); break;
        case DAV2_GEMM_EPI_ROW_LAYERSCALE: launch_epi<DAV2_GEMM_EPI_ROW_LAYERSCALE>(g, s); break;
        case DAV2_GEMM_EPI_TRANSPOSED: launch_epi<DAV2_GEMM_EPI_TRANSPOSED>(g, s); break;
        case DAV2_GEMM_EPI_CONVT: launch_epi<DAV2_GEMM_EPI_CONVT>(g, s); break;
        case DAV2_GEMM_EPI_ROW_COLMAX: launch_epi<DAV2_GEMM_EPI_ROW_COLMAX>(g, s); break;
    }
    return hipGetLastError();
}

}  // namespace

extern "C" int dav2_hip_gemm_i8(const dav2_gemm_i8_args* a, void* stream) {
    const int status = gemm_i8(a, stream);
    if (t_events_for_one_gemm) {
        launch_events() = LaunchEvents{nullptr, nullptr};
        t_events_for_one_gemm = false;
    }
    return status;
}

extern "C" void dav2_hip_gemm_i8_events(void* start, void* stop) {
    launch_events() = LaunchEvents{static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)};
    t_events_for_one_gemm = start || stop;
}

extern "C" uint32_t dav2_hip_gemm_i8_row_tiles(uint32_t m, uint32_t n, uint32_t epilogue) {
    const bool swapped = epilogue == DAV2_GEMM_EPI_TRANSPOSED || epilogue == DAV2_GEMM_EPI_CONVT;
    const bool row_major = epilogue == DAV2_GEMM_EPI_ROW || epilogue == DAV2_GEMM_EPI_ROW_GELU ||
                           epilogue == DAV2_GEMM_EPI_ROW_LAYERSCALE || epilogue == DAV2_GEMM_EPI_ROW_COLMAX;
    const uint32_t rows_p = swapped ? n : m, rows_q = swapped ? m : n;
    return ceil_div(rows_p, tile_rows(rows_p, rows_q, row_major, epilogue == DAV2_GEMM_EPI_ROW_COLMAX));
}
