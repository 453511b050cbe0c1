// Device-side helpers shared by the flash-GQA HIP kernels (gfx950 only).
//
// MFMA operand layouts used throughout (wave64, lane l, l16 = l % 16, l32 = l % 32):
//   v_mfma_f32_16x16x32_bf16  A[m][k]: lane m + 16*(k/8) holds k%8 of 8 bf16
//                             B[k][n]: lane n + 16*(k/8) holds k%8 of 8 bf16
//                             C[m][n]: lane n + 16*(m/4), register m%4
//   v_mfma_f32_32x32x16_bf16  A[m][k]: lane m + 32*(k/8), element k%8
//                             B[k][n]: lane n + 32*(k/8), element k%8
//                             C[m][n]: lane n + 32*((m/4)%2), register (m%4) + 4*(m/8)
// The GPU parity tests check every kernel built on these layouts against the CPU oracle.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fgqa {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// Division by a runtime divisor d >= 1 of numerators 0 <= x < 2^31 with a
// multiplier the host computes once (Granlund & Montgomery, "Division by
// invariant integers using multiplication", PLDI 1994, Theorem 4.2 with
// N = 31): l = ceil(log2 d), m = ceil(2^(31 + l) / d) < 2^32, and
// x / d = (x * m) >> (31 + l), i.e. mulhi(x, m) >> (l - 1) for d >= 2.
// Two scalar instructions instead of the ~25 of a general division, which
// kernels pay per work unit when they map a rank to its unit.
struct FastDiv {
    int d;          // the divisor
    uint32_t mul;   // m (unused when d == 1)
    int shift;      // l - 1 (unused when d == 1)
};

inline FastDiv make_fast_div(int d) {
    FastDiv f{d, 0u, 0};
    if (d <= 1) return f;
    int l = 0;
    while ((1ll << l) < d) ++l;
    f.mul = (uint32_t)(((1ull << (31 + l)) + (uint64_t)d - 1) / (uint64_t)d);
    f.shift = l - 1;
    return f;
}

__host__ __device__ __forceinline__ int fast_div(int x, FastDiv f) {
    const uint32_t hi = (uint32_t)(((uint64_t)(uint32_t)x * f.mul) >> 32);   // a scalar mul_hi on the device
    return f.d == 1 ? x : (int)(hi >> f.shift);
}

constexpr int kWave = 64;
constexpr int kHeadDim = 128;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Raw (stride 0) buffer resource over [base, base + bytes).  A load whose
// offset is at or past `bytes` returns zeros instead of touching memory, which
// is how the kernels read ragged tails without a branch per load.
// Third descriptor word 0x00020000: 32-bit data format, as used for raw
// buffers on the gfx9 family (gfx90a/gfx94x/gfx950).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ u32x4_t buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
}

// Streaming variant: the `nt` (non-temporal) cache policy, for data read
// exactly once (the decode KV stream).  On MI355X a read-only stream reaches
// ~7.0 TB/s with nt against ~6.3 TB/s without.
constexpr int kCachePolicyNT = 2;
__device__ __forceinline__ u32x4_t buf_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCachePolicyNT);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16_t mfma32(bf16x8_t a, bf16x8_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Transposed LDS read (ds_read_b64_tr_b16).  Within each group of 16 lanes,
// lane i receives 4 b16 values: value j is element (i % 4) of the 8-byte
// chunk addressed by lane 4*j + i/4 of the same group.  So if lane s of the
// group points at row R(s/4), columns C + 4*(s%4) .. +3 of a row-major b16
// matrix, lane i receives rows R(0..3) of column C + i.
__device__ __forceinline__ bf16x4_t lds_read_tr16(const __bf16* p) {
    typedef short s16x4_t __attribute__((ext_vector_type(4)));
    const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4_t*)(__attribute__((address_space(3))) void*)(p));
    return __builtin_bit_cast(bf16x4_t, v);
}

// {value of lane l % 32, value of lane 32 + l % 32} for every lane l
// (v_permlane32_swap): combines the two halves of a wave in one VALU op.
__device__ __forceinline__ float half_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float xor_max(float v, int mask) { return fmaxf(v, __shfl_xor(v, mask, kWave)); }
__device__ __forceinline__ float xor_sum(float v, int mask) { return v + __shfl_xor(v, mask, kWave); }

}  // namespace fgqa
