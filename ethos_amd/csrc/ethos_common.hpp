// Shared device helpers for the ETHOS expert-layer kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ethos {

enum DType : int { kF32 = 0, kBF16 = 1 };

constexpr int kWave = 64;

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// float -> bf16 bits, round to nearest even (NaN stays a quiet NaN); branch-free.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    const uint32_t b = __float_as_uint(f);
    const uint32_t r = (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
    const uint32_t n = (b >> 16) | 0x40u;
    return (uint16_t)(((b & 0x7fffffffu) > 0x7f800000u) ? n : r);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Two floats -> packed bf16 pair (a in the low half), round to nearest even, one
// v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    const f32x2_t f = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}

// double -> float with round-to-odd: truncate, then force the last bit to 1 if inexact.
// Rounding that float to bf16 (8 significant bits <= 24 - 2) gives the correctly rounded
// bf16 of the double.
__device__ __forceinline__ float f64_to_f32_odd(double d) {
    float f = (float)d;
    if ((double)f == d) return f;
    uint32_t b = __float_as_uint(f);
    if ((b & 1u) == 0u) b = (fabs((double)f) > fabs(d)) ? b - 1u : b + 1u;
    return __uint_as_float(b);
}

// Storage-type traits: T is float (fp32) or uint16_t (bf16 bits).
template <typename T> struct Elem;
template <> struct Elem<float> {
    static constexpr DType kDType = kF32;
    __device__ __forceinline__ static float to_f32(float v) { return v; }
    __device__ __forceinline__ static double to_f64(float v) { return (double)v; }
    __device__ __forceinline__ static float from_f32(float v) { return v; }
    __device__ __forceinline__ static float from_f64(double v) { return (float)v; }
    __device__ __forceinline__ static float from_f32_rne(float v) { return v; }
    // round a float to T and return the T value as float
    __device__ __forceinline__ static float round32(float v) { return v; }
    __device__ __forceinline__ static void round32x2(float& a, float& b) {}
    __device__ __forceinline__ static float round64(double v) { return (float)v; }
    // a float c <= every x with RN_T(x) >= t, for t a T value: the spacing below t is at
    // most |t| 2^-23, so RN(t - |t| 2^-23) <= t - ulp is below the midpoint between t and
    // its predecessor; 2^-126 covers t = 0 and subnormal t
    __device__ __forceinline__ static float round_down_cut(float t) { return (t - fabsf(t) * 0x1p-23f) - 0x1p-126f; }
};
template <> struct Elem<uint16_t> {
    static constexpr DType kDType = kBF16;
    __device__ __forceinline__ static float to_f32(uint16_t v) { return bf16_bits_to_f32(v); }
    __device__ __forceinline__ static double to_f64(uint16_t v) { return (double)bf16_bits_to_f32(v); }
    __device__ __forceinline__ static uint16_t from_f32(float v) { return f32_to_bf16_bits(v); }
    __device__ __forceinline__ static uint16_t from_f64(double v) { return f32_to_bf16_bits(f64_to_f32_odd(v)); }
    // from_f32 through the hardware conversion (round to nearest even; the same bits for
    // every non-NaN input)
    __device__ __forceinline__ static uint16_t from_f32_rne(float v) { return (uint16_t)(pack_bf16x2(v, v) & 0xffffu); }
    // through the hardware conversion (round to nearest even), as round32x2
    __device__ __forceinline__ static float round32(float v) { return __uint_as_float(pack_bf16x2(v, v) << 16); }
    // two values at once through the hardware conversion (round to nearest even)
    __device__ __forceinline__ static void round32x2(float& a, float& b);
    __device__ __forceinline__ static float round64(double v) { return bf16_bits_to_f32(from_f64(v)); }
    // a float c <= every x with RN_T(x) >= t, for t a bf16 value: the bf16 spacing below
    // t is at most |t| 2^-7, so t - |t| 2^-7 (exact in fp32) is at most the midpoint
    // between t and its predecessor; 2^-126 covers t = 0 and subnormal t
    __device__ __forceinline__ static float round_down_cut(float t) { return (t - fabsf(t) * 0x1p-7f) - 0x1p-126f; }
};

__device__ __forceinline__ void Elem<uint16_t>::round32x2(float& a, float& b) {
    const uint32_t pk = pack_bf16x2(a, b);
    a = __uint_as_float(pk << 16);
    b = __uint_as_float(pk & 0xffff0000u);
}

// Exact GELU (erf form), fp32.
__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

// erf-form GELU of two packed bf16 values (low and high half), correctly rounded to
// bf16, from a table of the 3328 inputs that are not a closed form (gelu_bf16_lut.inc,
// written by gelu_lut.py): table entry d for x = +bf16(0x3a80 + d), d < 1536
// (2^-10 <= x < 4), and entry 1536 + d for x = -bf16(0x3a80 + d), d < 1792
// (2^-10 <= |x| < 16).  Elsewhere RN(GELU(x)) = x for x >= 4, -0 for -inf < x <= -16,
// NaN for -inf and NaN, and RN(x / 2) for |x| < 2^-10.  The lane arithmetic works on
// both 16-bit halves at once; the per-half masks (all ones where a condition holds) come
// from arithmetic shifts, written as inline asm so that the compiler keeps them packed
// instead of splitting them into per-half compares and selects.  `lut_bytes` is the
// table's LDS byte address.
constexpr int kGeluLutSize = 3328;

// each half: v < 0 (as i16) ? 0xffff : 0.  The shift count is the packed pair (15, 15):
// an inline constant would give the high half a count of 0.
__device__ __forceinline__ uint32_t pk_sign_mask(uint32_t v) {
    uint32_t r;
    asm("v_pk_ashrrev_i16 %0, %1, %2" : "=v"(r) : "s"(0x000f000fu), "v"(v));
    return r;
}
// b is wave-uniform (a constant): held in an SGPR, since packed instructions take no
// literal operands
__device__ __forceinline__ uint32_t pk_add_u16(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_pk_add_u16 %0, %1, %2" : "=v"(r) : "v"(a), "s"(b));
    return r;
}
__device__ __forceinline__ uint32_t pk_add_u16_vv(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_pk_add_u16 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ uint32_t pk_sub_u16(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_pk_sub_u16 %0, %1, %2" : "=v"(r) : "v"(a), "s"(b));
    return r;
}
__device__ __forceinline__ uint32_t pk_rsub_u16(uint32_t a, uint32_t b) {  // b - a per half
    uint32_t r;
    asm("v_pk_sub_u16 %0, %2, %1" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ uint32_t pk_min_u16(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_pk_min_u16 %0, %1, %2" : "=v"(r) : "v"(a), "s"(b));
    return r;
}
__device__ __forceinline__ uint32_t bit_select(uint32_t m, uint32_t a, uint32_t b) {  // (m & a) | (~m & b)
    return (m & a) | (~m & b);
}

__device__ __forceinline__ uint32_t pk_max_i16(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_pk_max_i16 %0, %1, %2" : "=v"(r) : "v"(a), "s"(b));
    return r;
}
__device__ __forceinline__ uint32_t pk_min_i16_vv(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_pk_min_i16 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ uint32_t pk_lshl_b16(uint32_t a, uint32_t sh) {  // sh: wave-uniform (SGPR)
    uint32_t r;
    asm("v_pk_lshlrev_b16 %0, %1, %2" : "=v"(r) : "s"(sh), "v"(a));
    return r;
}

// The same function as gelu_bf16x2_lut from a table of float32 pairs (M, C) with
// RN(GELU(x)) = RN_bf16(fma(x, M, C)) for every input, so that no per-case selection is
// needed: entries 0 .. kGeluMcSize / 2 - 1 serve x >= +0, the rest x <= -0, each half
// ordered as (|x| < 2^-10: M = 0.5, C = +-0), (the table inputs: M = 0, C = the table
// value), (x >= 4: M = 1, C = 0 / x <= -16: M = 0, C = -0).  The index is
// clamp(|x|bits - 0x3a7f, 0, hi) + base with hi = 1537 / 1793 and base = 0 / 1538.
constexpr int kGeluMcPos = 1538;               // entries for x >= +0
constexpr int kGeluMcSize = kGeluMcPos + 1794;  // and for x <= -0
// Entry i in two steps, so that a caller can request every table value it needs before
// building any entry: the table index entry i reads (a valid index for every i below
// kGeluMcSize; entries that are a closed form ignore the value), then the entry from it.
__device__ __forceinline__ int gelu_mc_lut_index(int i) {
    if (i < kGeluMcPos) return i == 0 || i == kGeluMcPos - 1 ? 0 : i - 1;
    const int j = i - kGeluMcPos;
    return j == 0 || j == 1793 ? 0 : 1536 + j - 1;
}
__device__ __forceinline__ f32x2_t gelu_mc_entry_from(int i, uint16_t v) {
    if (i < kGeluMcPos) {
        if (i == 0) return f32x2_t{0.5f, 0.0f};
        if (i == kGeluMcPos - 1) return f32x2_t{1.0f, 0.0f};
        return f32x2_t{0.0f, __uint_as_float((uint32_t)v << 16)};
    }
    const int j = i - kGeluMcPos;
    if (j == 0) return f32x2_t{0.5f, -0.0f};
    if (j == 1793) return f32x2_t{0.0f, -0.0f};
    return f32x2_t{0.0f, __uint_as_float((uint32_t)v << 16)};
}
__device__ __forceinline__ uint32_t gelu_bf16x2_mc(uint32_t pk, uint32_t mc_bytes) {
    const uint32_t a = pk & 0x7fff7fffu;
    const uint32_t negm = pk_sign_mask(pk);
    // |x|bits - 0x3a7f as a signed 16-bit value: <= 0 below the table, 1 + d inside it
    const uint32_t d = pk_max_i16(pk_sub_u16(a, 0x3a7f3a7fu), 0u);
    const uint32_t hi = 0x06010601u + (negm & 0x01000100u);  // 1537 or 1793
    const uint32_t idx = pk_min_i16_vv(d, hi) + (negm & 0x06020602u);  // + 1538 for x <= -0
    const uint32_t off = pk_lshl_b16(idx, 0x00030003u);  // 8-byte entries (max offset 26.6 KB)
    typedef const __attribute__((address_space(3))) f32x2_t* lds_f2_ptr;
    const f32x2_t e0 = *(lds_f2_ptr)(size_t)(mc_bytes + (off & 0xffffu));
    const f32x2_t e1 = *(lds_f2_ptr)(size_t)(mc_bytes + (off >> 16));
    const float r0 = __builtin_fmaf(__uint_as_float(pk << 16), e0[0], e0[1]);
    const float r1 = __builtin_fmaf(__uint_as_float(pk & 0xffff0000u), e1[0], e1[1]);
    return pack_bf16x2(r0, r1);
}

__device__ __forceinline__ uint32_t gelu_bf16x2_lut(uint32_t pk, uint32_t lut_bytes) {
    const uint32_t a = pk & 0x7fff7fffu;
    const uint32_t negm = pk_sign_mask(pk);
    const uint32_t d = pk_sub_u16(a, 0x3a803a80u);  // wraps below the table: |x| < 2^-10
    const uint32_t smallm = pk_sign_mask(d);
    // table index: d (+ 1536 for negative x), clamped; lanes outside the table are
    // replaced below
    const uint32_t idx = pk_min_u16(pk_add_u16_vv(d, negm & 0x06000600u), 0x0cff0cffu);
    // big: d >= 0x600 (x >= 4) or d >= 0x700 (x <= -16), i.e. thr - d < 0 with
    // thr = 0x5ff or 0x6ff
    const uint32_t bigm = pk_sign_mask(pk_rsub_u16(d, pk_add_u16(negm & 0x01000100u, 0x05ff05ffu)));
    // big result: x itself for x > 0; -0 for negative x, or a NaN for -inf / NaN (a >= 0x7f80)
    const uint32_t bigneg = 0x80008000u | (pk_sign_mask(pk_add_u16(a, 0x00800080u)) & 0x7fc07fc0u);
    const uint32_t bigv = bit_select(negm, bigneg, pk);
    const uint32_t off = pk_add_u16_vv(idx, idx);  // byte offsets
    typedef const __attribute__((address_space(3))) uint16_t* lds_u16_ptr;
    const uint32_t tlo = *(lds_u16_ptr)(size_t)(lut_bytes + (off & 0xffffu));
    const uint32_t thi = *(lds_u16_ptr)(size_t)(lut_bytes + (off >> 16));
    const uint32_t tv = tlo | (thi << 16);
    // small result: RN(x / 2), exact arithmetic in fp32 (also for bf16 subnormals)
    const uint32_t half = pack_bf16x2(__uint_as_float(pk << 16) * 0.5f, __uint_as_float(pk & 0xffff0000u) * 0.5f);
    return bit_select(smallm, half, bit_select(bigm, bigv, tv));
}

// ---------------------------------------------------------------- wave reductions (DPP)
// dpp_ctrl encodings (GCN/CDNA DPP): quad_perm, row_half_mirror, row_mirror.
// Lane mask of a predicate: the compare writes the scalar mask directly (HIP's __ballot
// takes an int and adds a select and a second compare).
__device__ __forceinline__ uint64_t ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }
// Number of set bits of m below the calling lane (v_mbcnt).
__device__ __forceinline__ int count_below(uint64_t m) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

constexpr int kDppXor1 = 0xb1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4e;        // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kCtrl, 0xf, 0xf, false);
}
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
    return __uint_as_float(dpp_u32<kCtrl>(__float_as_uint(v)));
}

// Sum over the 64 lanes; every lane receives the same value (fixed association order).
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<kDppXor1>(v);
    v += dpp_f32<kDppXor2>(v);
    v += dpp_f32<kDppRowHalfMirror>(v);
    v += dpp_f32<kDppRowMirror>(v);
    float r0 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 0));
    float r1 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 16));
    float r2 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 32));
    float r3 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 48));
    return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ uint64_t u64_max(uint64_t a, uint64_t b) { return a > b ? a : b; }

template <int kCtrl>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
    uint32_t lo = dpp_u32<kCtrl>((uint32_t)v);
    uint32_t hi = dpp_u32<kCtrl>((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int lane) {
    uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, lane);
    uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), lane);
    return ((uint64_t)hi << 32) | lo;
}

// Max over the 64 lanes; every lane receives it.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    v = u64_max(v, dpp_u64<kDppXor1>(v));
    v = u64_max(v, dpp_u64<kDppXor2>(v));
    v = u64_max(v, dpp_u64<kDppRowHalfMirror>(v));
    v = u64_max(v, dpp_u64<kDppRowMirror>(v));
    uint64_t a = u64_max(readlane_u64(v, 0), readlane_u64(v, 16));
    uint64_t b = u64_max(readlane_u64(v, 32), readlane_u64(v, 48));
    return u64_max(a, b);
}

typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));

// Raw buffer resource (byte-addressed, stride 0, 32-bit num_records) for a global array.
__device__ __forceinline__ i32x4_t buffer_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t)base;
    return i32x4_t{(int32_t)(uint32_t)a, (int32_t)(uint32_t)((a >> 32) & 0xffffu), (int32_t)bytes, 0x00020000};
}

// 16 bytes per lane from a buffer straight into LDS at lds + 16 * lane (lds is the
// wave-uniform LDS byte address).  Issued as inline asm so that the compiler does not
// make later LDS reads of other buffers wait for the copy; the caller waits (vmcnt)
// and synchronises before the copied data is read.
__device__ __forceinline__ void lds_dma16(i32x4_t rsrc, int voff, int soff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds), "v"(voff), "s"(rsrc),
                 "s"(soff)
                 : "memory");
}
// The same with the non-temporal hint, for data read once (it then displaces less of what
// other loads reuse from L2).
__device__ __forceinline__ void lds_dma16_nt(i32x4_t rsrc, int voff, int soff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds" ::"s"(lds), "v"(voff), "s"(rsrc),
                 "s"(soff)
                 : "memory");
}

template <typename P>
__device__ __forceinline__ uint32_t lds_addr(P* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(__attribute__((address_space(3))) P*)p);
}

// ---------------------------------------------------------------- canonical keys
// Order-preserving image of a float (-0 == +0), and a 64-bit selection key whose
// natural order is (score descending, index ascending).
__device__ __forceinline__ uint32_t ord32(float f) {
    uint32_t b = __float_as_uint(f);
    if (b == 0x80000000u) b = 0u;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ uint64_t make_key(float score, uint32_t idx) {
    return ((uint64_t)ord32(score) << 32) | (uint64_t)(~idx);
}
__device__ __forceinline__ uint32_t key_idx(uint64_t k) { return ~(uint32_t)(k & 0xffffffffu); }
__device__ __forceinline__ float key_score(uint64_t k) {
    uint32_t o = (uint32_t)(k >> 32);
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

}  // namespace ethos
