// 32x32 MFMA tiles for gfx950: bf16 (v_mfma_f32_32x32x16_bf16) and fp32 (v_mfma_f32_32x32x2f32).
//
// Operand layout (both types): lane l supplies A[row = l % 32][k0 + (l / 32) * kKL .. + kKL)
// and B[k0 + (l / 32) * kKL .. + kKL)[col = l % 32]; accumulator element i of lane l is
// C[mfma32_row(i, l)][l % 32].
#pragma once

#include "ethos_common.hpp"

namespace ethos {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <typename T> struct Mfma;
template <> struct Mfma<uint16_t> {
    static constexpr int kK = 16;     // reduction depth per instruction
    static constexpr int kKL = 8;     // consecutive k per lane; lanes 32..63 hold the upper half
    typedef bf16x8_t frag;
    __device__ __forceinline__ static frag load(const uint16_t* p) { return *reinterpret_cast<const frag*>(p); }
    __device__ __forceinline__ static frag zero() { return frag{}; }
    __device__ __forceinline__ static f32x16_t mma(frag a, frag b, f32x16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mfma<float> {
    static constexpr int kK = 2;
    static constexpr int kKL = 1;
    typedef float frag;
    __device__ __forceinline__ static frag load(const float* p) { return *p; }
    __device__ __forceinline__ static frag zero() { return 0.0f; }
    __device__ __forceinline__ static f32x16_t mma(frag a, frag b, f32x16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
};

// Row of accumulator element i of a 32x32 MFMA tile held by `lane`; column = lane % 32.
__device__ __forceinline__ int mfma32_row(int i, int lane) { return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3); }

__device__ __forceinline__ f32x16_t f32x16_zero() {
    f32x16_t z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.0f;
    return z;
}

}  // namespace ethos
