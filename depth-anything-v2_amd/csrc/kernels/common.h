// Shared device helpers for the gfx950 kernels. Wave size is 64 throughout.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define DAV2_DEV __device__ __forceinline__

namespace dav2k {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Butterfly reductions. After the xor butterfly every lane holds the full
// result, but each lane's association order differs; lane 0's order equals a
// shared-memory tree reduction over widths 32,16,...,1 (partial[l] +=
// partial[l+w]). Broadcasting lane 0 therefore reproduces the tree bit for bit.
DAV2_DEV float wave_sum_tree(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = v + __shfl_xor(v, o, kWave);
    return __shfl(v, 0, kWave);
}

DAV2_DEV float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

DAV2_DEV float wave_min(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, kWave));
    return v;
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

inline unsigned ceil_div(uint64_t a, uint64_t b) { return static_cast<unsigned>((a + b - 1) / b); }

}  // namespace dav2k
