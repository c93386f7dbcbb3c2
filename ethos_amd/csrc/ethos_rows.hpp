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

// a . b + acc over one lane's raw slice (fp32 accumulation; bf16 pairs by v_dot2c_f32_bf16)
typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot_raw(const uint4& a, const uint4& b, float acc) {
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a.x), __builtin_bit_cast(bf16x2_v, b.x), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a.y), __builtin_bit_cast(bf16x2_v, b.y), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a.z), __builtin_bit_cast(bf16x2_v, b.z), acc, false);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a.w), __builtin_bit_cast(bf16x2_v, b.w), acc,
                                           false);
}
__device__ __forceinline__ float dot_raw(const float4& a, const float4& b, float acc) {
    acc = __builtin_fmaf(a.x, b.x, acc);
    acc = __builtin_fmaf(a.y, b.y, acc);
    acc = __builtin_fmaf(a.z, b.z, acc);
    return __builtin_fmaf(a.w, b.w, acc);
}

// Per-pair activations a_p = RN_T(RN_T(gelu(RN_T(h_s . xp_t))) g_p), the arithmetic every
// activation kernel shares: the pair's 8 lanes hold pieces part + 8 i (i < P) of both rows
// (16 bytes each), each lane sums its pieces in order with dot_raw, and the 8 lanes reduce
// by three DPP steps (xor 1, xor 2, half-row mirror).  Kernels that follow this recipe give
// bit-identical activations whatever order they visit the pairs in.
__device__ __forceinline__ float act_reduce8(float acc) {
    acc += dpp_f32<kDppXor1>(acc);
    acc += dpp_f32<kDppXor2>(acc);
    acc += dpp_f32<kDppRowHalfMirror>(acc);
    return acc;
}
template <typename T>
__device__ __forceinline__ float act_epilogue(float dot, float gate) {
    const float a = Elem<T>::round32(gelu_erf(Elem<T>::round32(dot)));
    return Elem<T>::round32(a * gate);
}

// Token order for the activations, taken when the hidden rows of all unique experts fit
// in a cache (at most this many bytes): one wave per token holds the token's projection in
// registers and reads the hidden rows of its H*k pairs, which stay cache-resident, instead
// of gathering one projection row per pair.  Same lanes, same per-lane dot products and
// same reduction as the expert-order walk, so the results are bit-identical.
constexpr int64_t kActTokenOrderMaxHBytes = 8 << 20;

// Activations inside the bf16 hidden-row kernel: when the expert order applies (more
// hidden-row bytes than kActTokenOrderMaxHBytes), the hidden-row kernel computes the
// activations of every tile of kActTileRows unique experts whose pairs number at most
// kActFusedCap, from the tile's rows while they are still in LDS.  The pairs of larger
// tiles (a few hot experts) are left to the activation kernel, which spreads them over
// the whole GPU instead of one workgroup.
constexpr int kActTileRows = 64;
constexpr int64_t kActFusedCap = 2048;

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

// The same slices through a buffer descriptor over the row's d elements: lanes past the row
// read zeros without a per-lane branch, and for a wave-uniform row pointer the descriptor and
// its address arithmetic stay in scalar registers.
template <typename T, int CH>
__device__ __forceinline__ void load_raw_buf(const T* row, int d, int lane, typename Vec16<T>::raw (&r)[CH]) {
    constexpr int N = Vec16<T>::kN;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(row), (short)0, d * (int)sizeof(T), 0x00020000);
#pragma unroll
    for (int c = 0; c < CH; ++c)
        r[c] = __builtin_bit_cast(typename Vec16<T>::raw,
                                  __builtin_amdgcn_raw_buffer_load_b128(rs, (c * 64 * N + lane * N) * (int)sizeof(T), 0, 0));
}

}  // namespace ethos
