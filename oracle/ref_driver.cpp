// Test-only C shim over reference sources that compile on their own
// (src/model.cpp: .dav2 loader and validation; src/image.cpp: network_shape
// and the two host image preprocessors).
// Built by `make -C oracle ref` straight from the reference tree into
// oracle/_ref/; used by tests to check this build's .dav2 writer, loader
// verdicts and network-shape rule against the reference implementation.

#include "model.h"
#include "image.h"

#include <cstdio>
#include <cstring>
#include <exception>
#include <vector>

extern "C" {

// Returns 0 and fills width/height, or 1 with the exception text in error.
int ref_network_shape(int width, int height, int input_size, int* out_width, int* out_height, char* error,
                      size_t error_bytes) {
    try {
        const dav2::ImageShape s = dav2::network_shape(width, height, input_size);
        *out_width = s.width;
        *out_height = s.height;
        return 0;
    } catch (const std::exception& e) {
        std::snprintf(error, error_bytes, "%s", e.what());
        return 1;
    }
}

// Opens a .dav2 file with the reference loader. Returns 0 if accepted (and
// reports tensor count, derivation presence and metric max depth), 1 if the
// loader threw (message in error).
int ref_model_open(const char* path, int encoder, unsigned* tensor_count, int* derivation_present,
                   float* metric_max_depth, char* error, size_t error_bytes) {
    try {
        dav2::ModelFile model(path, static_cast<dav2_encoder>(encoder));
        *tensor_count = static_cast<unsigned>(model.tensor_count());
        *derivation_present = model.derivation().present ? 1 : 0;
        *metric_max_depth = model.derivation().metric_max_depth;
        return 0;
    } catch (const std::exception& e) {
        std::snprintf(error, error_bytes, "%s", e.what());
        return 1;
    }
}

// Copies tensor `name` (float32) into out (capacity in floats); returns the
// element count, or -1 if missing.
long long ref_model_tensor(const char* path, int encoder, const char* name, float* out, size_t capacity) {
    try {
        dav2::ModelFile model(path, static_cast<dav2_encoder>(encoder));
        const dav2::TensorView& t = model.tensor(name);
        const size_t n = static_cast<size_t>(t.elements);
        std::memcpy(out, t.data, (n < capacity ? n : capacity) * sizeof(float));
        return static_cast<long long>(n);
    } catch (const std::exception&) {
        return -1;
    }
}

// src/image.cpp:163-270 (reference's own BGR8 preprocessing). Returns 0 and
// fills out [3][dst_height][dst_width], or 1 with the exception text.
int ref_preprocess_bgr8(const unsigned char* bgr, int width, int height, long long stride, int dst_width,
                        int dst_height, float* out, char* error, size_t error_bytes) {
    try {
        std::vector<float> chw;
        dav2::preprocess_bgr8(bgr, width, height, static_cast<std::ptrdiff_t>(stride), {dst_width, dst_height}, chw);
        std::memcpy(out, chw.data(), chw.size() * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        std::snprintf(error, error_bytes, "%s", e.what());
        return 1;
    }
}

// src/image.cpp:289-339 (InferBridge BGRA nearest preprocessing).
int ref_preprocess_inferbridge_bgra8(const unsigned char* bgra, int width, int height, long long stride,
                                     int dst_width, int dst_height, float* out, char* error, size_t error_bytes) {
    try {
        std::vector<float> chw;
        dav2::preprocess_inferbridge_bgra8(bgra, width, height, static_cast<std::ptrdiff_t>(stride),
                                           {dst_width, dst_height}, chw);
        std::memcpy(out, chw.data(), chw.size() * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        std::snprintf(error, error_bytes, "%s", e.what());
        return 1;
    }
}

}  // extern "C"
