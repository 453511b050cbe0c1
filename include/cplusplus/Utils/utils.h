// Common utilities for the flash-GQA C++ operator API (MI355X / gfx950 build).
//
// Counterpart of the reference's include/cplusplus/Utils/utils.cuh:14-44.
// The index helpers are 64-bit here: the reference's `int` versions overflow
// once a tensor holds 2^31 elements (a [64, 32768, 8, 128] KV cache does).
#pragma once

#include <cstdint>

// A bfloat16 value: the upper 16 bits of an IEEE-754 binary32, bit-identical to
// the reference's __nv_bfloat16 and to HIP's __hip_bfloat16, so device buffers
// of either type can be passed through a reinterpret_cast.
struct bf16_t {
    uint16_t bits;
};
static_assert(sizeof(bf16_t) == 2, "bf16_t must be 2 bytes");

// Ceiling of a / b for b > 0.
constexpr int64_t CEIL_DIV(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Row-major flattening of a 3-D index (i1, i2, i3) in a [*, D2, D3] tensor.
constexpr int64_t GET_1D_INDEX_FROM_3D(int64_t i1, int64_t i2, int64_t i3, int64_t D2, int64_t D3) {
    return (i1 * D2 + i2) * D3 + i3;
}

// Row-major flattening of a 4-D index (i1, i2, i3, i4) in a [*, D2, D3, D4] tensor.
constexpr int64_t GET_1D_INDEX_FROM_4D(int64_t i1, int64_t i2, int64_t i3, int64_t i4, int64_t D2, int64_t D3,
                                       int64_t D4) {
    return ((i1 * D2 + i2) * D3 + i3) * D4 + i4;
}
