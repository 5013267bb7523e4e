// Shared device helpers for the gfx950 kernels. Wave size is 64 throughout.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#define DAV2_DEV __device__ __forceinline__

namespace dav2k {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Wave reductions as the halving tree partial[l] = op(partial[l],
// partial[l + w]) for w = 32, 16, ..., 1, the order of a shared-memory tree
// reduction; lane 0 ends with the result and every lane receives it. The
// moves stay in the VALU: lanes 32-63 reach lanes 0-31 through
// v_permlane32_swap, lanes 16-31 reach 0-15 through v_permlane16_swap, and
// the steps within a row of 16 lanes are DPP row shifts (lanes that would
// read past their row get 0, and only lanes whose results feed lane 0 are
// meaningful). Every lane of the wave must be active.
template <typename Op>
DAV2_DEV float wave_tree(float v, Op op) {
    const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = op(v, __uint_as_float(p32[1]));
    const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = op(v, __uint_as_float(p16[1]));
    v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x108, 0xF, 0xF, true)));  // row_shl:8
    v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x104, 0xF, 0xF, true)));  // row_shl:4
    v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x102, 0xF, 0xF, true)));  // row_shl:2
    v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x101, 0xF, 0xF, true)));  // row_shl:1
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
}

DAV2_DEV float wave_sum_tree(float v) {
    return wave_tree(v, [](float a, float b) { return a + b; });
}

DAV2_DEV float wave_max(float v) {
    return wave_tree(v, [](float a, float b) { return fmaxf(a, b); });
}

DAV2_DEV float wave_min(float v) {
    return wave_tree(v, [](float a, float b) { return fminf(a, b); });
}

// Reference quantization step (quantize_rows_int8_fused.glsl:46-50 and
// gpu_model.cpp:251-254): clamp to [-127, 127], round half to even.
DAV2_DEV int quantize_rne(float v) {
    v = fminf(fmaxf(v, -127.0f), 127.0f);
    return static_cast<int>(__builtin_rintf(v));
}

DAV2_DEV uint32_t pack4(int a, int b, int c, int d) {
    return (static_cast<uint32_t>(a) & 0xffu) | ((static_cast<uint32_t>(b) & 0xffu) << 8) |
           ((static_cast<uint32_t>(c) & 0xffu) << 16) | ((static_cast<uint32_t>(d) & 0xffu) << 24);
}

// IEEE division and square root, correctly rounded (the build never enables
// fast-math; these spell the intent out at the call sites that must match the
// CPU oracle bit for bit).
DAV2_DEV float div_rn(float a, float b) { return __fdiv_rn(a, b); }

// v exactly as computed: a rounded fp32 value the compiler may not fuse
// into the operation that consumes it. Needed where an fp32 result is then
// rounded to binary16: fp16(a * b) would otherwise become one
// v_fma_mixlo_f16, which rounds the exact product once instead of rounding
// it to fp32 first (the two differ when the fp32 rounding lands on a
// binary16 tie).
DAV2_DEV float keep_fp32(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// s + float(fp16(a * b)) for two pairs: one binary16 multiplication of each
// pair (v_pk_mul_f16), each product widened and added in fp32 (the native
// binary16 shaders' sum += float(x16 * y16); no contraction under
// -ffp-contract=off).
DAV2_DEV void add_half_products(float& s0, float& s1, h2 a, h2 b) {
    const h2 p = a * b;
    s0 = s0 + static_cast<float>(p.x);
    s1 = s1 + static_cast<float>(p.y);
}

// The binary16 value nearest v (round to nearest even), as a float.
DAV2_DEV float round_half(float v) { return static_cast<float>(static_cast<_Float16>(keep_fp32(v))); }

inline unsigned ceil_div(uint64_t a, uint64_t b) { return static_cast<unsigned>((a + b - 1) / b); }

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 16 bytes per lane from global memory straight into LDS
// (global_load_lds_dwordx4): lane l's bytes land at lds_base + 16*l; the
// base must be the same for the whole wave. The copies count in vmcnt.
DAV2_DEV void copy16_to_lds(const void* src, void* lds_base) {
    __builtin_amdgcn_global_load_lds(src, (lds_ptr_t)lds_base, 16, 0, 0);
}

// 4 bytes per lane (global_load_lds_dword): lane l's bytes land at
// lds_base + 4*l.
DAV2_DEV void copy4_to_lds(const void* src, void* lds_base) {
    __builtin_amdgcn_global_load_lds(src, (lds_ptr_t)lds_base, 4, 0, 0);
}

// s_waitcnt with vmcnt = n (expcnt, lgkmcnt not waited on), n < 64.
#define DAV2_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

// Scale rule shared by every activation quantizer:
// quantize_rows_int8_fused.glsl:37 and im2col_quantize_int8.glsl:63.
DAV2_DEV float row_scale(float absmax) { return fmaxf(absmax / 127.0f, 1.0e-8f); }

// quantize_rne(x / s) (the IEEE quotient) for a row scale s from row_scale
// (so |x / s| <= 127 (1 + 2^-23)), inv = div_rn(1, s). The product x * inv
// is within 127 x (2^-23 + 2^-24 + 2^-47) < 2^-15.4 of the rounded quotient,
// so both round to the same integer whenever the product is more than 2^-14
// from a half-integer; the other lanes (about 1 in 8000) divide. NaN and
// infinite x or s give the quotient's result as well (clamped NaN is -127).
// quantize_product is the first step alone: q = the clamped rint(x * inv),
// and true where the product lies within 2^-14 of a half-integer, so that
// only quantize_div's quotient may decide.
DAV2_DEV bool quantize_product(float x, float inv, int& q) {
    const float y = x * inv;
    const float n = __builtin_rintf(y);
    q = static_cast<int>(fminf(fmaxf(n, -127.0f), 127.0f));
    return fabsf(y - n) > 0.5f - 0x1p-14f;
}

DAV2_DEV int quantize_div(float x, float s, float inv) {
    int q;
    if (__builtin_expect(quantize_product(x, inv, q), 0)) return quantize_rne(div_rn(x, s));
    return q;
}

// Per-pixel |x| maxima of a CHW map over groups of kGroupChannels channels:
// partial[g][p] = max over c in group g of |x[c][p]| (quantize.hip). The
// window maximum of these is the absmax of an im2col row.
constexpr uint32_t kGroupChannels = 32;
inline uint32_t channel_groups(uint32_t channels) { return (channels + kGroupChannels - 1) / kGroupChannels; }
hipError_t launch_channel_group_absmax(const float* x, uint32_t channels, uint64_t plane, float* partial,
                                       bool relu, hipStream_t stream);

// e^a by Cody-Waite range reduction (a = n ln2 + r, |r| <= ln2/2, ln2 split
// into a 16-bit head and a tail) and the degree-7 Taylor polynomial of e^r in
// Horner form with explicit fmaf; error below 1 ulp of float over the range.
// Every step is a correctly rounded IEEE operation, so the CPU oracle's
// restatement of the same sequence returns the same bits. Results below
// e^-86 (about 2^-124) are flushed to zero, above FLT_MAX they are +inf.
DAV2_DEV float exp_cw(float a) {
    if (!(a > -86.0f)) return a != a ? a : 0.0f;
    if (a > 88.72f) return __builtin_inff();
    const float n = __builtin_rintf(a * 1.44269504f);
    float r = fmaf(-n, 0.693145751953125f, a);  // ln2 head, exact product
    r = fmaf(-n, 1.42860677e-6f, r);             // ln2 - head
    float p = 1.98412698e-4f;                    // 1/7!
    p = fmaf(p, r, 1.38888889e-3f);              // 1/6!
    p = fmaf(p, r, 8.33333333e-3f);              // 1/5!
    p = fmaf(p, r, 4.16666667e-2f);              // 1/4!
    p = fmaf(p, r, 1.66666667e-1f);              // 1/3!
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, static_cast<int>(n));
}

// gelu.glsl:29-48: 0.5 x (1 + erf(x / sqrt 2)) with erf from the
// Numerical Recipes erfc fit, the shader's operation order and exp_cw.
DAV2_DEV float gelu_erfcc(float value) {
    const float x = value * 0.70710678118654752440f;
    const float magnitude = fabsf(x);
    // t = 1 / (1 + m/2) correctly rounded: the hardware reciprocal refined by
    // one Newton step with fma (Markstein's reciprocal iteration), which
    // returns the correctly rounded quotient for every float d in [1, 16)
    // (checked exhaustively on gfx950). For d >= 16 (m >= 30) or NaN,
    // exp_cw(-m*m + poly) below is 0 or NaN whatever finite t is, so t = 0
    // gives the same result as the IEEE quotient.
    const float d = 1.0f + 0.5f * magnitude;
    float t = 0.0f;
    if (d < 16.0f) {
        const float r = __builtin_amdgcn_rcpf(d);
        t = fmaf(fmaf(-d, r, 1.0f), r, r);
    }
    float poly = t * 0.17087277f;
    poly = t * (-0.82215223f + poly);
    poly = t * (1.48851587f + poly);
    poly = t * (-1.13520398f + poly);
    poly = t * (0.27886807f + poly);
    poly = t * (-0.18628806f + poly);
    poly = t * (0.09678418f + poly);
    poly = t * (0.37409196f + poly);
    poly = t * (1.00002368f + poly);
    poly = -1.26551223f + poly;
    const float erfc_magnitude = t * exp_cw(-magnitude * magnitude + poly);
    const float erf_value = x >= 0.0f ? 1.0f - erfc_magnitude : erfc_magnitude - 1.0f;
    return 0.5f * value * (1.0f + erf_value);
}

// Nontemporal store: the data goes straight to memory instead of waiting in
// this XCD's L2 for the write-back at the kernel's end. It speeds up the
// storing kernel and slows a consumer that would have found the data in the
// caches; measured per use, it pays only for fc1's GELU output at batch 1
// (the GEMM's other row-major outputs, the convolutions and the resize keep
// plain stores).
DAV2_DEV void store_nt(float* dst, float4 v) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(f4{v.x, v.y, v.z, v.w}, reinterpret_cast<f4*>(dst));
}

// Timing hook for profiling (dav2_hip_launch_events): the calling thread's
// next kernel launch records `start` when it begins, and every launch until
// the hook is cleared records `stop` when it ends (an event keeps its last
// record), so the pair spans all kernels of one operation. The dispatches
// record them themselves (hipExtLaunchKernelGGL), so they time the kernels
// and not the host's launch gaps before the first one.
struct LaunchEvents {
    hipEvent_t start, stop;
    bool launched;  // a kernel recorded the pair since it was set
};
LaunchEvents& launch_events();

template <typename Kernel, typename... Args>
void dispatch(Kernel kernel, dim3 grid, dim3 block, size_t lds, hipStream_t stream, Args... args) {
    LaunchEvents& e = launch_events();
    if (e.start || e.stop) {
        hipExtLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(lds), stream, e.start, e.stop, 0, args...);
        e.start = nullptr;
        e.launched = true;
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
    }
}

}  // namespace dav2k
