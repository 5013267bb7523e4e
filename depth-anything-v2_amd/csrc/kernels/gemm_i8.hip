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
// (BN/WAVES_N) sub-tile of 16x16 MFMA blocks. Each 64-byte K step is staged
// global -> VGPR -> LDS, double-buffered so the loads of step s+1 overlap the
// MFMAs of step s, with one workgroup barrier per step.

#include "common.h"
#include "dav2_hip.h"

using namespace dav2k;

namespace {

constexpr int kBK = 64;              // K bytes per pipeline step
constexpr int kLdsStride = kBK + 16;  // padded LDS row (bytes): spreads 16 rows over all banks

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

template <int BM, int BN, int WAVES_M, int WAVES_N, int EPI>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void gemm_i8_kernel(GemmParams g) {
    constexpr int NT = 64 * WAVES_M * WAVES_N;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int TM = WM / 16, TN = WN / 16;
    constexpr int P_CHUNKS = BM * (kBK / 16);  // 16-byte chunks per stage
    constexpr int Q_CHUNKS = BN * (kBK / 16);
    constexpr int P_PER_T = (P_CHUNKS + NT - 1) / NT;
    constexpr int Q_PER_T = (Q_CHUNKS + NT - 1) / NT;
    static_assert(TM >= 1 && TN >= 1, "wave tile must hold at least one MFMA block");

    __shared__ __attribute__((aligned(16))) int8_t smem[2][(BM + BN) * kLdsStride];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const uint32_t row0 = blockIdx.y * BM;
    const uint32_t col0 = blockIdx.x * BN;
    const int ksteps = static_cast<int>(g.k / kBK);

    v4i rp[P_PER_T], rq[Q_PER_T];

    auto load_global = [&](int ks) {
        const uint64_t kofs = static_cast<uint64_t>(ks) * kBK;
#pragma unroll
        for (int i = 0; i < P_PER_T; ++i) {
            const int c = tid + i * NT;
            const uint32_t r = row0 + (c >> 2);
            v4i v = {0, 0, 0, 0};
            if (c < P_CHUNKS && r < g.rows_p)
                v = *reinterpret_cast<const v4i*>(g.p + r * g.ldp + kofs + (c & 3) * 16);
            rp[i] = v;
        }
#pragma unroll
        for (int i = 0; i < Q_PER_T; ++i) {
            const int c = tid + i * NT;
            const uint32_t r = col0 + (c >> 2);
            v4i v = {0, 0, 0, 0};
            if (c < Q_CHUNKS && r < g.rows_q)
                v = *reinterpret_cast<const v4i*>(g.q + r * g.ldq + kofs + (c & 3) * 16);
            rq[i] = v;
        }
    };
    auto store_lds = [&](int buf) {
#pragma unroll
        for (int i = 0; i < P_PER_T; ++i) {
            const int c = tid + i * NT;
            if (c < P_CHUNKS)
                *reinterpret_cast<v4i*>(&smem[buf][(c >> 2) * kLdsStride + (c & 3) * 16]) = rp[i];
        }
#pragma unroll
        for (int i = 0; i < Q_PER_T; ++i) {
            const int c = tid + i * NT;
            if (c < Q_CHUNKS)
                *reinterpret_cast<v4i*>(&smem[buf][(BM + (c >> 2)) * kLdsStride + (c & 3) * 16]) = rq[i];
        }
    };

    v4i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    load_global(0);
    store_lds(0);
    __syncthreads();

    const int frag_row = lane & 15;
    const int frag_k = (lane >> 4) * 16;
    for (int ks = 0; ks < ksteps; ++ks) {
        const int cur = ks & 1;
        if (ks + 1 < ksteps) load_global(ks + 1);
        v4i af[TM], bf[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
            af[i] = *reinterpret_cast<const v4i*>(
                &smem[cur][(wm * WM + i * 16 + frag_row) * kLdsStride + frag_k]);
#pragma unroll
        for (int j = 0; j < TN; ++j)
            bf[j] = *reinterpret_cast<const v4i*>(
                &smem[cur][(BM + wn * WN + j * 16 + frag_row) * kLdsStride + frag_k]);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        if (ks + 1 < ksteps) store_lds(cur ^ 1);
        __syncthreads();
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

int device_cu_count() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    return cus;
}

template <int BM, int BN, int WMW, int WNW, int EPI>
void launch_cfg(const GemmParams& g, hipStream_t s) {
    const dim3 grid(ceil_div(g.rows_q, BN), ceil_div(g.rows_p, BM));
    hipLaunchKernelGGL((gemm_i8_kernel<BM, BN, WMW, WNW, EPI>), grid, dim3(64 * WMW * WNW), 0, s, g);
}

template <int EPI>
void launch_epi(const GemmParams& g, hipStream_t s) {
    const uint64_t cus = static_cast<uint64_t>(device_cu_count());
    const uint64_t tiles_l = static_cast<uint64_t>(ceil_div(g.rows_p, 128)) * ceil_div(g.rows_q, 128);
    const uint64_t tiles_m = static_cast<uint64_t>(ceil_div(g.rows_p, 128)) * ceil_div(g.rows_q, 64);
    if (tiles_l >= 2 * cus) launch_cfg<128, 128, 2, 2, EPI>(g, s);
    else if (tiles_m >= cus) launch_cfg<128, 64, 2, 2, EPI>(g, s);
    else launch_cfg<64, 64, 2, 2, EPI>(g, s);
}

}  // namespace

extern "C" int dav2_hip_gemm_i8(const dav2_gemm_i8_args* a, void* stream) {
    if (!a) return hipErrorInvalidValue;
    if (a->m == 0 || a->n == 0) return hipSuccess;
    if (!a->a || !a->b || a->k == 0 || a->k % kBK || a->lda < a->k || a->ldb < a->k ||
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
