// Device-resident weights. Every tensor's CRC-32 is verified on load
// (reference src/gpu_model.cpp:127-146). Tensors the reference quantizes for
// its int8 mode (selection rule: src/gpu_model.cpp:16-44) are stored only as
// per-output-row int8 + fp32 scales (quantizer: src/gpu_model.cpp:241-264),
// everything else as fp32. The fp32 precision mode keeps every tensor fp32;
// the fp16 mode keeps them fp32 too, with the reference's half-weight family
// (src/gpu_model.cpp:15-33) rounded to binary16 values.
//
// int8 layout: [rows][ld] bytes, ld = columns rounded up to 64, zero padding.
// Conv weights [OC][IC][k][k] flatten to rows = OC, column ic*k*k + ky*k + kx
// (the im2col column order); ConvTranspose weights [IC][OC][k][k] are
// reordered to rows (ky*k + kx)*OC + oc, columns = IC (src/gpu_model.cpp:226-240).
#pragma once

#include "model.h"
#include "operators.h"
#include "runtime.h"

#include <array>
#include <cstdint>
#include <string>
#include <string_view>
#include <unordered_map>

namespace dav2 {

struct GpuTensor {
    // fp32 copy: tensors not stored as int8; in the fp32 precision mode every
    // tensor, weights in the GEMM layout [f32_rows][f32_columns] (the int8
    // row layout unpadded: ConvTranspose reordered, everything else as stored)
    DeviceBuffer buffer;
    std::uint32_t f32_rows = 0, f32_columns = 0;
    DeviceBuffer int8_buffer;  // [int8_rows][int8_ld]
    DeviceBuffer int8_scales;  // [int8_rows]
    // Conv weights the implicit-GEMM convolution takes (kernel 1 or 3,
    // IC % 64 == 0, OC % 32 == 0): the same int8 rows with K walked tap-major
    // ((ky*k + kx)*IC + ic) and cut into the kernels' 16 x 64-byte operand
    // fragments (dav2_hip_conv_weights_pack). Empty otherwise.
    DeviceBuffer int8_packed;
    std::uint32_t int8_rows = 0;
    std::uint32_t int8_columns = 0;
    std::uint32_t int8_ld = 0;
    std::array<std::uint64_t, 4> dimensions{};
    std::uint32_t rank = 0;
    std::uint64_t elements = 0;
};

bool use_int8_weight(std::string_view name, const WeightRecord& tensor);
bool transposed_convolution_weight(std::string_view name);
inline std::uint32_t padded_k(std::uint64_t columns) { return static_cast<std::uint32_t>((columns + 63) & ~63ull); }

class GpuModel {
public:
    // precision: int8 (int8 copies of the quantized family), fp32 or fp16
    // (no int8 copies; fp16 rounds the half family to binary16).
    GpuModel(const MappedModel& model, HipContext& context, Precision precision = Precision::int8);
    const GpuTensor& tensor(std::string_view name) const;
    bool contains(std::string_view name) const { return tensors_.count(std::string(name)) != 0; }
    std::size_t tensor_count() const { return tensors_.size(); }
    std::uint64_t device_bytes() const { return device_bytes_; }

private:
    std::unordered_map<std::string, GpuTensor> tensors_;
    std::uint64_t device_bytes_ = 0;
};

}  // namespace dav2
