// Expert apply and weighted scatter-back (reference: model.py:326-341).
//
// Per pair p = (t, h, j) with expert slot s:
//   a_p = RN_T( RN_T(gelu_erf( RN_T(u_s . x_t) )) * g_p )                  (phase 1)
//   y_t = RN_T( sum_h^T RN_T( sum_j RN_T(a_p * v_s) ) / H )                (phase 2)
// where the inner sum is fp32 in j order, the head sum is taken in T one head at a
// time, and RN_T is rounding to the layer dtype -- the reference's rounding points
// (fp32 token accumulator model.py:312,334, per-head cast :336, dtype head sum :338,
// dtype divide :341).
//
// Phase 1 walks the pairs in expert order (the sorted permutation): a wave takes 64
// consecutive sorted positions and reloads u_s only when the slot changes, so each
// expert's u row is read about once.  Phase 2 is token-major: one wave per token
// gathers the v rows of its H*k pairs and reduces them in registers; every output
// element is written by exactly one lane, so no atomics are needed and the result
// is deterministic.
#include "ethos_common.hpp"
#include "ethos_launch.hpp"

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

constexpr int kActGroup = 4;  // pairs whose loads are in flight together

template <typename T, int CH>
__global__ __launch_bounds__(256) void apply_act_kernel(const T* __restrict__ x, const T* __restrict__ uv,
                                                        const int32_t* __restrict__ perm,
                                                        const int32_t* __restrict__ sorted_slot,
                                                        const T* __restrict__ gates, int64_t n_pairs, int hk, int d,
                                                        float* __restrict__ act) {
    constexpr int N = Vec16<T>::kN;
    typedef typename Vec16<T>::raw Raw;
    const int lane = threadIdx.x & 63;
    const int64_t wave_id = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t n_waves = (int64_t)gridDim.x * 4;
    const int64_t n_chunks = (n_pairs + 63) / 64;
    const int64_t d2 = 2 * (int64_t)d;
    for (int64_t chunk = wave_id; chunk < n_chunks; chunk += n_waves) {
        const int64_t i0 = chunk * 64;
        const int cnt = (int)min((int64_t)64, n_pairs - i0);
        const int my_p = lane < cnt ? perm[i0 + lane] : 0;
        const int my_s = lane < cnt ? sorted_slot[i0 + lane] : 0;
        // Groups of kActGroup consecutive sorted pairs: every u and x row of a group is
        // requested before the first dot product (repeated u rows of one expert hit in
        // the cache), then the group's wave reductions run interleaved.
        for (int j0 = 0; j0 < cnt; j0 += kActGroup) {
            Raw ur[kActGroup][CH], xr[kActGroup][CH];
            int pq[kActGroup];
#pragma unroll
            for (int q = 0; q < kActGroup; ++q) {
                const int j = j0 + q < cnt ? j0 + q : cnt - 1;  // a tail group repeats the last pair
                const int s = __builtin_amdgcn_readlane(my_s, j);
                pq[q] = __builtin_amdgcn_readlane(my_p, j);
                load_raw<T, CH>(uv + (int64_t)s * d2, d, lane, ur[q]);
                load_raw<T, CH>(x + (int64_t)(pq[q] / hk) * d, d, lane, xr[q]);
            }
            float part[kActGroup];
#pragma unroll
            for (int q = 0; q < kActGroup; ++q) {
                part[q] = 0.0f;
#pragma unroll
                for (int c = 0; c < CH; ++c) {
                    float uf[N], xf[N];
                    Vec16<T>::unpack(ur[q][c], uf);
                    Vec16<T>::unpack(xr[q][c], xf);
#pragma unroll
                    for (int v = 0; v < N; ++v) part[q] = __builtin_fmaf(uf[v], xf[v], part[q]);
                }
            }
#pragma unroll
            for (int q = 0; q < kActGroup; ++q) {
                const float dot = wave_sum(part[q]);
                if (lane == q && j0 + q < cnt) {
                    const float g = Elem<T>::to_f32(gates[pq[q]]);
                    const float a = Elem<T>::round32(gelu_erf(Elem<T>::round32(dot)));
                    act[pq[q]] = Elem<T>::round32(a * g);
                }
            }
        }
    }
}

constexpr int kScatterUnroll = 8;  // v rows in flight per wave

template <typename T, int CH>
__global__ __launch_bounds__(256) void apply_scatter_kernel(const T* __restrict__ uv,
                                                            const int32_t* __restrict__ pair_slot,
                                                            const float* __restrict__ act, int64_t n_tok, int H,
                                                            int k, int d, T* __restrict__ out) {
    constexpr int N = Vec16<T>::kN;
    typedef typename Vec16<T>::raw Raw;
    const int lane = threadIdx.x & 63;
    const int64_t wave_id = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t n_waves = (int64_t)gridDim.x * 4;
    const int64_t d2 = 2 * (int64_t)d;
    const float inv_h_div = (float)H;
    for (int64_t t = wave_id; t < n_tok; t += n_waves) {
        float o[CH * N];
#pragma unroll
        for (int e = 0; e < CH * N; ++e) o[e] = 0.0f;
        for (int h = 0; h < H; ++h) {
            float hacc[CH * N];
#pragma unroll
            for (int e = 0; e < CH * N; ++e) hacc[e] = 0.0f;
            const int64_t pbase = (t * H + h) * k;
            for (int j0 = 0; j0 < k; j0 += kScatterUnroll) {
                Raw vr[kScatterUnroll][CH];
                float a[kScatterUnroll];
#pragma unroll
                for (int q = 0; q < kScatterUnroll; ++q) {
                    if (j0 + q < k) {
                        const int s = pair_slot[pbase + j0 + q];
                        a[q] = act[pbase + j0 + q];
                        load_raw<T, CH>(uv + (int64_t)s * d2 + d, d, lane, vr[q]);
                    }
                }
#pragma unroll
                for (int q = 0; q < kScatterUnroll; ++q) {
                    if (j0 + q < k) {
#pragma unroll
                        for (int c = 0; c < CH; ++c) {
                            float vf[N];
                            Vec16<T>::unpack(vr[q][c], vf);
#pragma unroll
                            for (int v = 0; v < N; ++v) hacc[c * N + v] += Elem<T>::round32(a[q] * vf[v]);
                        }
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < CH * N; ++e) o[e] = Elem<T>::round32(o[e] + Elem<T>::round32(hacc[e]));
        }
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int e = c * 64 * N + lane * N;
            if (e < d) {
                float r[N];
#pragma unroll
                for (int v = 0; v < N; ++v) r[v] = o[c * N + v] / inv_h_div;
                *reinterpret_cast<typename Vec16<T>::raw*>(out + t * d + e) = Vec16<T>::pack(r);
            }
        }
    }
}

template <typename T, int CH>
static int launch_apply_t(const void* x, const void* uv, const int32_t* perm, const int32_t* sorted_slot,
                          const int32_t* pair_slot, const void* gates, int64_t n_tok, int H, int k, int d, float* act,
                          void* out, int num_cus, hipStream_t stream) {
    const int64_t n_pairs = n_tok * H * k;
    const int64_t chunks = (n_pairs + 63) / 64;
    int64_t g1 = (chunks + 3) / 4;
    const int64_t cap = (int64_t)num_cus * 16;
    if (g1 > cap) g1 = cap;
    if (g1 < 1) g1 = 1;
    hipLaunchKernelGGL((apply_act_kernel<T, CH>), dim3((unsigned)g1), dim3(256), 0, stream, (const T*)x,
                       (const T*)uv, perm, sorted_slot, (const T*)gates, n_pairs, H * k, d, act);
    int64_t g2 = (n_tok + 3) / 4;
    if (g2 > cap) g2 = cap;
    if (g2 < 1) g2 = 1;
    hipLaunchKernelGGL((apply_scatter_kernel<T, CH>), dim3((unsigned)g2), dim3(256), 0, stream, (const T*)uv,
                       pair_slot, (const float*)act, n_tok, H, k, d, (T*)out);
    return (int)hipGetLastError();
}

int apply_chunks(int d, int dtype) {
    const int per = 64 * (dtype == kBF16 ? 8 : 4);
    return (d + per - 1) / per;
}

int launch_apply(const void* x, const void* uv, const int32_t* perm, const int32_t* sorted_slot,
                 const int32_t* pair_slot, const void* gates, int64_t n_tok, int H, int k, int d, int dtype, float* act,
                 void* out, int num_cus, hipStream_t stream) {
    const int ch = apply_chunks(d, dtype);
#define ETHOS_APPLY_CASE(TT, C)                                                                                   \
    if (ch <= C)                                                                                                  \
        return launch_apply_t<TT, C>(x, uv, perm, sorted_slot, pair_slot, gates, n_tok, H, k, d, act, out, num_cus, \
                                     stream);
    if (dtype == kBF16) {
        ETHOS_APPLY_CASE(uint16_t, 1)
        ETHOS_APPLY_CASE(uint16_t, 2)
        ETHOS_APPLY_CASE(uint16_t, 4)
        ETHOS_APPLY_CASE(uint16_t, 8)
    } else {
        ETHOS_APPLY_CASE(float, 1)
        ETHOS_APPLY_CASE(float, 2)
        ETHOS_APPLY_CASE(float, 4)
        ETHOS_APPLY_CASE(float, 8)
    }
#undef ETHOS_APPLY_CASE
    return -1;
}

}  // namespace ethos
