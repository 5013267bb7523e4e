// fp32 and fp16 paths of the precision modes (DAV2_CREATE_FORCE_FP32 /
// FORCE_FP16): the linear and convolution GEMMs in float32 on the MFMA
// (v_mfma_f32_16x16x4_f32), with the epilogues of the int8 GEMM, and the
// fp32 im2col that feeds convolutions.
//
// fp16 arithmetic comes in the reference's two forms. Cooperative-matrix
// linears (linear_coop_fp16.glsl via linear_fp16* with cooperative_matrix_fp16,
// src/operators.cpp:540-768): operands rounded to binary16, exact products,
// fp32 accumulation. The fp32 GEMM does this with half_operands: both tiles
// are rounded to binary16 as they are staged, and the product of two binary16
// values is exact in fp32. Native binary16 shaders (prepare_tokens_fp16,
// project_tokens_fp16, conv_transpose_nonoverlap_fp16): every product is a
// binary16 multiplication, widened and added to an fp32 sum in k order;
// gemm_h16p_kernel does exactly that on the VALU, so its results match the
// oracle bit for bit.
//
// Reference: linear_tiled.glsl / linear_vec*.glsl (src/operators.cpp:882-955),
// conv2d (:1528-1676), conv_transpose_nonoverlap (:1807-1861),
// project_tokens (:1408-1452), gelu.glsl, add_scaled.glsl. The reference sums
// each dot product in its own tile order; fp32 results are compared within a
// tolerance, not bit for bit.
//
// Tiles: 64x64 outputs per 256-thread workgroup, 2x2 waves of 32x32; K in
// steps of 32 floats through a two-stage LDS ring filled from registers
// (the next step's loads are in flight while the current one multiplies).
// A lane's 16-byte fragment holds 4 consecutive k of its row; the 4 MFMAs of
// a fragment take element e of every lane, so each MFMA sums k = 4g + e over
// the lane groups g and the four together cover 16 k.

#include "common.h"
#include "dav2_hip.h"

namespace {

using namespace dav2k;

constexpr int kBM = 64, kBN = 64, kBK = 32;  // tile rows, tile columns, floats per K step
constexpr int kLdsRow = kBK + 4;             // padded LDS row (floats)

struct F32Params {
    const float* a;
    uint64_t lda;
    const float* b;
    uint64_t ldb;
    uint32_t m, n, k;
    const float* bias;
    float* out;
    uint64_t out_row_offset, out_row_stride;
    const float* residual;
    const float* gamma;
    uint32_t relu_output;
    uint32_t convt_k, convt_w, convt_h, convt_c;
    uint32_t half_operands;  // round both operands to binary16 when staged
};

template <int EPI>
DAV2_DEV void store_f32(const F32Params& g, uint32_t m, uint32_t n, float acc) {
    if (EPI == DAV2_GEMM_EPI_CONVT) {
        const uint32_t kidx = n / g.convt_c, oc = n - kidx * g.convt_c;
        const float v = acc + (g.bias ? g.bias[oc] : 0.0f);
        const uint32_t k = g.convt_k;
        const uint32_t iy = m / g.convt_w, ix = m - iy * g.convt_w;
        const uint32_t ky = kidx / k, kx = kidx - ky * k;
        const uint32_t ow = g.convt_w * k, oh = g.convt_h * k;
        g.out[(static_cast<uint64_t>(oc) * oh + iy * k + ky) * ow + ix * k + kx] = v;
        return;
    }
    const float v = acc + (g.bias ? g.bias[n] : 0.0f);
    if (EPI == DAV2_GEMM_EPI_TRANSPOSED) {
        const uint64_t idx = static_cast<uint64_t>(n) * g.out_row_stride + m + g.out_row_offset;
        float o = v;
        if (g.residual) o = o + g.residual[idx];
        if (g.relu_output) o = fmaxf(o, 0.0f);
        g.out[idx] = o;
        return;
    }
    const uint64_t idx = (static_cast<uint64_t>(m) + g.out_row_offset) * g.n + n;
    if (EPI == DAV2_GEMM_EPI_ROW_GELU) {
        g.out[idx] = gelu_erfcc(v);
    } else if (EPI == DAV2_GEMM_EPI_ROW_LAYERSCALE) {
        const float scaled = v * g.gamma[n];  // add_scaled.glsl:26-30, no contraction
        g.out[idx] = g.residual[idx] + scaled;
    } else {
        g.out[idx] = v;
    }
}

template <int EPI>
__global__ __launch_bounds__(256) void gemm_f32_kernel(F32Params g) {
    __shared__ __attribute__((aligned(16))) float as[2][kBM * kLdsRow];
    __shared__ __attribute__((aligned(16))) float bs[2][kBN * kLdsRow];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const uint32_t row0 = blockIdx.x * kBM, col0 = blockIdx.y * kBN;
    const int steps = static_cast<int>((g.k + kBK - 1) / kBK);

    // Thread t moves float4 t and t + 256 of each 64 x 32 operand tile:
    // tile row idx / 8, floats 4 (idx % 8) .. +3. Rows past the matrix and
    // k past K read zeros (K is a multiple of 4, so a float4 is all in or out).
    float4 ra[2], rb[2];
    auto fetch = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            const uint32_t r = static_cast<uint32_t>(idx >> 3), kk = k0 + 4u * (idx & 7);
            const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
            ra[i] = row0 + r < g.m && kk < g.k
                        ? *reinterpret_cast<const float4*>(g.a + static_cast<uint64_t>(row0 + r) * g.lda + kk)
                        : zero;
            rb[i] = col0 + r < g.n && kk < g.k
                        ? *reinterpret_cast<const float4*>(g.b + static_cast<uint64_t>(col0 + r) * g.ldb + kk)
                        : zero;
        }
    };
    auto stash = [&](int s) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            const int off = (idx >> 3) * kLdsRow + 4 * (idx & 7);
            float4 va = ra[i], vb = rb[i];
            if (g.half_operands) {
                va = make_float4(round_half(va.x), round_half(va.y), round_half(va.z), round_half(va.w));
                vb = make_float4(round_half(vb.x), round_half(vb.y), round_half(vb.z), round_half(vb.w));
            }
            *reinterpret_cast<float4*>(&as[s][off]) = va;
            *reinterpret_cast<float4*>(&bs[s][off]) = vb;
        }
    };

    v4f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    fetch(0);
    stash(0);
    __syncthreads();
    const int frag = (lane & 15) * kLdsRow + 4 * (lane >> 4);
    for (int step = 0; step < steps; ++step) {
        const int s = step & 1;
        if (step + 1 < steps) fetch(static_cast<uint32_t>(step + 1) * kBK);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            float4 fa[2], fb[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                fa[i] = *reinterpret_cast<const float4*>(&as[s][(wm * 32 + i * 16) * kLdsRow + frag + 16 * half]);
                fb[i] = *reinterpret_cast<const float4*>(&bs[s][(wn * 32 + i * 16) * kLdsRow + frag + 16 * half]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i].x, fb[j].x, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i].y, fb[j].y, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i].z, fb[j].z, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i].w, fb[j].w, acc[i][j], 0, 0, 0);
                }
        }
        // the other stage was last read before the previous barrier
        if (step + 1 < steps) stash(s ^ 1);
        __syncthreads();
    }

    // 16x16 result layout: lane l holds rows 4 (l / 16) + r of column l % 16.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t n = col0 + wn * 32 + j * 16 + (lane & 15);
            if (n >= g.n) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t m = row0 + wm * 32 + i * 16 + 4 * (lane >> 4) + r;
                if (m < g.m) store_f32<EPI>(g, m, n, acc[i][j][r]);
            }
        }
}

// Native binary16 products: out[m][n] = sum over k = 0, 1, .. K-1 of
// float(fp16(h(a[m][k]) * h(b[n][k]))) in fp32, h = round to binary16, then
// the epilogue (+ bias): prepare_tokens_fp16.glsl:37-52,
// project_tokens_common.glsl (NATIVE_FP16) and
// conv_transpose_nonoverlap_common.glsl (NATIVE_FP16), whose sums run over
// the inner index in ascending order. Thread (tx, ty) of 16 x 16 owns rows
// 4 ty .. +3 and columns 4 tx .. +3 of a 64 x 64 tile; K goes in chunks of
// 32, staged k-major in LDS as binary16 values held in floats (exact).
template <int EPI>
__global__ __launch_bounds__(256) void gemm_h16p_kernel(F32Params g) {
    __shared__ __attribute__((aligned(16))) float as[kBK][kBM + 4];
    __shared__ __attribute__((aligned(16))) float bs[kBK][kBN + 4];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const uint32_t row0 = blockIdx.x * kBM, col0 = blockIdx.y * kBN;
    float s[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) s[r][c] = 0.0f;
    for (uint32_t k0 = 0; k0 < g.k; k0 += kBK) {
        // float4 idx = tid + 256 i of each 64 x 32 operand tile: row idx / 8,
        // k 4 (idx % 8) .. +3 (K is a multiple of 4)
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            const uint32_t r = static_cast<uint32_t>(idx >> 3), kq = 4u * (idx & 7), kk = k0 + kq;
            const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
            const float4 va = row0 + r < g.m && kk < g.k
                                  ? *reinterpret_cast<const float4*>(g.a + static_cast<uint64_t>(row0 + r) * g.lda + kk)
                                  : zero;
            const float4 vb = col0 + r < g.n && kk < g.k
                                  ? *reinterpret_cast<const float4*>(g.b + static_cast<uint64_t>(col0 + r) * g.ldb + kk)
                                  : zero;
            as[kq + 0][r] = round_half(va.x);
            as[kq + 1][r] = round_half(va.y);
            as[kq + 2][r] = round_half(va.z);
            as[kq + 3][r] = round_half(va.w);
            bs[kq + 0][r] = round_half(vb.x);
            bs[kq + 1][r] = round_half(vb.y);
            bs[kq + 2][r] = round_half(vb.z);
            bs[kq + 3][r] = round_half(vb.w);
        }
        __syncthreads();
        const uint32_t kc = min(static_cast<uint32_t>(kBK), g.k - k0);  // no terms past K
#pragma unroll 4
        for (uint32_t k = 0; k < kc; ++k) {
            const float4 av = *reinterpret_cast<const float4*>(&as[k][ty * 4]);
            const float4 bv = *reinterpret_cast<const float4*>(&bs[k][tx * 4]);
            const h2 b01 = {static_cast<_Float16>(bv.x), static_cast<_Float16>(bv.y)};
            const h2 b23 = {static_cast<_Float16>(bv.z), static_cast<_Float16>(bv.w)};
            const float a[4] = {av.x, av.y, av.z, av.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const _Float16 ah = static_cast<_Float16>(a[r]);
                const h2 aa = {ah, ah};
                add_half_products(s[r][0], s[r][1], aa, b01);
                add_half_products(s[r][2], s[r][3], aa, b23);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t m = row0 + 4u * ty + r;
        if (m >= g.m) continue;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t n = col0 + 4u * tx + c;
            if (n < g.n) store_f32<EPI>(g, m, n, s[r][c]);
        }
    }
}

// out[p][c] = input[ic][iy][ix] of tap c = ic k^2 + ky k + kx of output pixel
// p (zero outside the image, max(., 0) first with relu); columns K .. ld-1 zero.
__global__ __launch_bounds__(256) void im2col_f32_kernel(const float* __restrict__ input, uint32_t width,
                                                         uint32_t height, uint32_t channels, uint32_t out_width,
                                                         uint32_t kernel, uint32_t stride, int32_t padding,
                                                         uint32_t relu, uint64_t rows, uint32_t columns, uint32_t ld,
                                                         float* __restrict__ out) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    if (i >= rows * ld) return;
    const uint64_t p = i / ld;
    const uint32_t c = static_cast<uint32_t>(i - p * ld);
    float v = 0.0f;
    if (c < columns) {
        const uint32_t kk = kernel * kernel;
        const uint32_t ic = c / kk, t = c - ic * kk, ky = t / kernel, kx = t - ky * kernel;
        const uint32_t oy = static_cast<uint32_t>(p / out_width), ox = static_cast<uint32_t>(p - uint64_t(oy) * out_width);
        const int32_t iy = static_cast<int32_t>(oy * stride + ky) - padding;
        const int32_t ix = static_cast<int32_t>(ox * stride + kx) - padding;
        if (iy >= 0 && ix >= 0 && iy < static_cast<int32_t>(height) && ix < static_cast<int32_t>(width)) {
            v = input[(static_cast<uint64_t>(ic) * height + iy) * width + ix];
            if (relu) v = fmaxf(v, 0.0f);
        }
    }
    out[i] = v;
}

template <int EPI>
void launch(const F32Params& g, hipStream_t s) {
    dispatch(gemm_f32_kernel<EPI>, dim3(ceil_div(g.m, kBM), ceil_div(g.n, kBN)), dim3(256), 0, s, g);
}

template <int EPI>
void launch_h16p(const F32Params& g, hipStream_t s) {
    dispatch(gemm_h16p_kernel<EPI>, dim3(ceil_div(g.m, kBM), ceil_div(g.n, kBN)), dim3(256), 0, s, g);
}

// Checks a dav2_gemm_f32_args and fills the kernel parameters; false if the
// call is invalid.
bool f32_params(const dav2_gemm_f32_args* a, F32Params& g) {
    if (!a || !a->a || !a->b || !a->out || a->m == 0 || a->n == 0 || a->k == 0 || a->k % 4u || a->lda < a->k ||
        a->ldb < a->k || a->lda % 4u || a->ldb % 4u || (reinterpret_cast<uintptr_t>(a->a) & 15u) ||
        (reinterpret_cast<uintptr_t>(a->b) & 15u) || ceil_div(a->n, kBN) > 65535u || a->half_operands > 1u)
        return false;
    const uint32_t e = a->epilogue;
    if (e != DAV2_GEMM_EPI_ROW && e != DAV2_GEMM_EPI_ROW_GELU && e != DAV2_GEMM_EPI_ROW_LAYERSCALE &&
        e != DAV2_GEMM_EPI_TRANSPOSED && e != DAV2_GEMM_EPI_CONVT)
        return false;
    if (e == DAV2_GEMM_EPI_ROW_LAYERSCALE && (!a->residual || !a->gamma)) return false;
    if (e == DAV2_GEMM_EPI_TRANSPOSED && a->out_row_stride < a->m + a->out_row_offset) return false;
    if (e == DAV2_GEMM_EPI_CONVT &&
        (a->convt_kernel == 0 || a->convt_channels == 0 || a->n != a->convt_kernel * a->convt_kernel * a->convt_channels ||
         a->m != a->convt_width * a->convt_height))
        return false;
    if ((a->relu_output || (a->residual && e != DAV2_GEMM_EPI_ROW_LAYERSCALE)) && e != DAV2_GEMM_EPI_TRANSPOSED)
        return false;
    g = F32Params{};
    g.a = a->a;
    g.lda = a->lda;
    g.b = a->b;
    g.ldb = a->ldb;
    g.m = a->m;
    g.n = a->n;
    g.k = a->k;
    g.bias = a->bias;
    g.out = a->out;
    g.out_row_offset = a->out_row_offset;
    g.out_row_stride = a->out_row_stride;
    g.residual = a->residual;
    g.gamma = a->gamma;
    g.relu_output = a->relu_output;
    g.convt_k = a->convt_kernel;
    g.convt_w = a->convt_width;
    g.convt_h = a->convt_height;
    g.convt_c = a->convt_channels;
    g.half_operands = a->half_operands;
    return true;
}

}  // namespace

extern "C" {

int dav2_hip_gemm_f32(const dav2_gemm_f32_args* a, void* stream) {
    F32Params g;
    if (!f32_params(a, g)) return hipErrorInvalidValue;
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (a->epilogue) {
        case DAV2_GEMM_EPI_ROW: launch<DAV2_GEMM_EPI_ROW>(g, s); break;
        case DAV2_GEMM_EPI_ROW_GELU: launch<DAV2_GEMM_EPI_ROW_GELU>(g, s); break;
        case DAV2_GEMM_EPI_ROW_LAYERSCALE: launch<DAV2_GEMM_EPI_ROW_LAYERSCALE>(g, s); break;
        case DAV2_GEMM_EPI_TRANSPOSED: launch<DAV2_GEMM_EPI_TRANSPOSED>(g, s); break;
        default: launch<DAV2_GEMM_EPI_CONVT>(g, s); break;
    }
    return hipGetLastError();
}

int dav2_hip_gemm_h16_products(const dav2_gemm_f32_args* a, void* stream) {
    F32Params g;
    if (!f32_params(a, g)) return hipErrorInvalidValue;
    const uint32_t e = a->epilogue;
    if ((e != DAV2_GEMM_EPI_ROW && e != DAV2_GEMM_EPI_TRANSPOSED && e != DAV2_GEMM_EPI_CONVT) || a->residual ||
        a->relu_output)
        return hipErrorInvalidValue;
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (e) {
        case DAV2_GEMM_EPI_ROW: launch_h16p<DAV2_GEMM_EPI_ROW>(g, s); break;
        case DAV2_GEMM_EPI_TRANSPOSED: launch_h16p<DAV2_GEMM_EPI_TRANSPOSED>(g, s); break;
        default: launch_h16p<DAV2_GEMM_EPI_CONVT>(g, s); break;
    }
    return hipGetLastError();
}

int dav2_hip_im2col_f32(const float* input, uint32_t input_width, uint32_t input_height, uint32_t input_channels,
                        uint32_t output_width, uint32_t output_height, uint32_t kernel, uint32_t stride,
                        int32_t padding, uint32_t relu, float* out, uint32_t ld, void* stream) {
    const uint64_t rows = static_cast<uint64_t>(output_width) * output_height;
    const uint64_t columns = static_cast<uint64_t>(input_channels) * kernel * kernel;
    if (rows == 0) return hipSuccess;
    if (!input || !out || kernel == 0 || stride == 0 || padding < 0 || ld < columns || columns >= (1u << 24) ||
        rows * ld >= (1ull << 38))
        return hipErrorInvalidValue;
    dispatch(im2col_f32_kernel, dim3(ceil_div(rows * ld, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), input, input_width, input_height, input_channels,
                       output_width, kernel, stride, padding, relu, rows, static_cast<uint32_t>(columns), ld, out);
    return hipGetLastError();
}

}  // extern "C"
