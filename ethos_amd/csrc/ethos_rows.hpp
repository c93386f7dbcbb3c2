// Row slices held across a wave: 16-byte pieces of a row per lane, element
// e = c*64*N + lane*N + v for chunk c (N = 8 bf16 or 4 float values per piece).
#pragma once
#include "ethos_common.hpp"

namespace ethos {

template <typename T> struct Vec16;
template <> struct Vec16<uint16_t> {
    static constexpr int kN = 8;
    typedef uint4 raw;
    __device__ __forceinline__ static void unpack(const raw& r, float* f) {
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = __uint_as_float(w[i] << 16);
            f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
    __device__ __forceinline__ static raw pack(const float* f) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = (uint32_t)f32_to_bf16_bits(f[2 * i]) | ((uint32_t)f32_to_bf16_bits(f[2 * i + 1]) << 16);
        return make_uint4(w[0], w[1], w[2], w[3]);
    }
};
template <> struct Vec16<float> {
    static constexpr int kN = 4;
    typedef float4 raw;
    __device__ __forceinline__ static void unpack(const raw& r, float* f) {
        f[0] = r.x;
        f[1] = r.y;
        f[2] = r.z;
        f[3] = r.w;
    }
    __device__ __forceinline__ static raw pack(const float* f) { return make_float4(f[0], f[1], f[2], f[3]); }
};

// Load a d-long row into per-lane registers: element e = c*64*N + lane*N + v.
template <typename T, int CH>
__device__ __forceinline__ void load_row(const T* __restrict__ row, int d, int lane, float (&f)[CH * Vec16<T>::kN]) {
    constexpr int N = Vec16<T>::kN;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int e = c * 64 * N + lane * N;
        if (e < d) {
            const typename Vec16<T>::raw r = *reinterpret_cast<const typename Vec16<T>::raw*>(row + e);
            Vec16<T>::unpack(r, f + c * N);
        } else {
#pragma unroll
            for (int v = 0; v < N; ++v) f[c * N + v] = 0.0f;
        }
    }
}

// Raw (undecoded) row slices of one lane: element e = c*64*N + lane*N + v.
template <typename T, int CH>
__device__ __forceinline__ void load_raw(const T* __restrict__ row, int d, int lane,
                                         typename Vec16<T>::raw (&r)[CH]) {
    constexpr int N = Vec16<T>::kN;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int e = c * 64 * N + lane * N;
        r[c] = e < d ? *reinterpret_cast<const typename Vec16<T>::raw*>(row + e) : typename Vec16<T>::raw{};
    }
}

}  // namespace ethos
