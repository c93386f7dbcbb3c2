// Product-key routing: sub-key scoring, canonical top-(k_cand) per query half,
// k_cand x k_cand combination, canonical top-k, fp32 softmax gates, expert-id decode.
// (reference: model.py:217-245 per head; heads stacked as rows = token * H + head,
// model.py:250-252).
//
// Numeric contract (identical to the CPU oracle's, written independently):
//   s[j]   = RN_T(fp64 FMA chain over the half-query and sub-key j, index order)
//   order  = (score descending, index ascending), -0 == +0; the index is the sub-key
//            index for the per-half lists and the expert id e = i1*K + i2 for the
//            combined list -- "ties broken to the lowest index".
//   c[a,b] = RN_T(fp32(v1[a] + v2[b]))
//   gate_i = RN_T(expf(c_i - c_0) / sum_i expf(c_i - c_0)), sum in list order.
//
// Layout: one workgroup (4 waves) owns 32 consecutive rows.  For each half, the
// sub-key table is staged into LDS transposed ([dim][key], <= 64 KiB per tile) and
// every wave scores its 8 rows against it; lane l owns keys l, l+64, ....  A
// running canonical top-k_cand per (row, half) is merged tile by tile with a
// DPP wave-max extraction over canonical 64-bit keys (score image << 32 | ~index).
#pragma clang fp contract(off)

#include "ethos_common.hpp"
#include "ethos_launch.hpp"

namespace ethos {

constexpr int kRtWaves = 4;
constexpr int kRtRowsPerWave = 8;
constexpr int kRtRows = kRtWaves * kRtRowsPerWave;
constexpr int kRtMaxKc = 32;      // k_cand <= 32  (top_k <= 16)
constexpr int kRtMaxNk = 8;       // keys per lane per tile (tile <= 512 keys)
constexpr int kRtCombSlots = 16;  // combined pairs per lane (k_cand^2 <= 1024)
constexpr int kRtTileBytes = 64 * 1024;

// Descending compare-exchange sort of a small per-lane array (fully unrolled).
template <int N>
__device__ __forceinline__ void sort_desc(uint64_t (&c)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i)
#pragma unroll
        for (int j = N - 1; j > i; --j) {
            const uint64_t a = c[j - 1], b = c[j];
            const bool sw = b > a;
            c[j - 1] = sw ? b : a;
            c[j] = sw ? a : b;
        }
}

// Extract the `count` largest keys over the wave (each lane's array sorted
// descending, 0 = empty) into out[0..count), descending.  Keys are distinct.
template <int N>
__device__ __forceinline__ void wave_extract(uint64_t (&c)[N], int count, uint64_t* out, int lane) {
    for (int r = 0; r < count; ++r) {
        const uint64_t m = wave_max_u64(c[0]);
        if (m != 0 && c[0] == m) {
#pragma unroll
            for (int i = 0; i < N - 1; ++i) c[i] = c[i + 1];
            c[N - 1] = 0;
        }
        if (lane == 0) out[r] = m;
    }
}

template <typename T>
__global__ __launch_bounds__(256) void route_kernel(const T* __restrict__ q, const T* __restrict__ keys1,
                                                    const T* __restrict__ keys2, int64_t rows, int dq, int K,
                                                    int top_k, int kc, int KT, T* __restrict__ out_gates,
                                                    int32_t* __restrict__ out_ids) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int dh2 = dq / 2;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    T* keyt = reinterpret_cast<T*>(smem);
    size_t off = ((size_t)dh2 * KT * sizeof(T) + 15) & ~(size_t)15;
    double* qs = reinterpret_cast<double*>(smem + off) + (size_t)wave * dh2;
    off += (size_t)kRtWaves * dh2 * sizeof(double);
    uint64_t* lists = reinterpret_cast<uint64_t*>(smem + off);  // [kRtRows][2][kRtMaxKc]
    off += (size_t)kRtRows * 2 * kRtMaxKc * sizeof(uint64_t);
    uint64_t* topk = reinterpret_cast<uint64_t*>(smem + off) + wave * kRtMaxKc;

    const int64_t row0 = (int64_t)blockIdx.x * kRtRows;
    const int nk = KT / kWave;

    for (int half = 0; half < 2; ++half) {
        const T* keys = half ? keys2 : keys1;
        for (int j0 = 0; j0 < K; j0 += KT) {
            const int kt = min(KT, K - j0);
            __syncthreads();
            for (int e = tid; e < kt * dh2; e += 256) {
                const int j = e / dh2, i = e - j * dh2;
                keyt[i * KT + j] = keys[(int64_t)(j0 + j) * dh2 + i];
            }
            __syncthreads();
            for (int rr = 0; rr < kRtRowsPerWave; ++rr) {
                const int lr = wave * kRtRowsPerWave + rr;
                const int64_t r = row0 + lr;
                if (r >= rows) break;
                for (int i = lane; i < dh2; i += kWave) qs[i] = Elem<T>::to_f64(q[r * dq + half * dh2 + i]);
                __builtin_amdgcn_wave_barrier();
                double acc[kRtMaxNk];
#pragma unroll
                for (int m = 0; m < kRtMaxNk; ++m) acc[m] = 0.0;
                for (int i = 0; i < dh2; ++i) {
                    const double qi = qs[i];
                    const T* kr = keyt + i * KT + lane;
#pragma unroll
                    for (int m = 0; m < kRtMaxNk; ++m)
                        if (m < nk) acc[m] = fma(qi, Elem<T>::to_f64(kr[m * kWave]), acc[m]);
                }
                __builtin_amdgcn_wave_barrier();
                uint64_t c[kRtMaxNk + 1];
#pragma unroll
                for (int m = 0; m < kRtMaxNk; ++m) {
                    const int j = lane + m * kWave;
                    c[m] = (m < nk && j < kt) ? make_key(Elem<T>::round64(acc[m]), (uint32_t)(j0 + j)) : 0ull;
                }
                uint64_t* lst = lists + ((size_t)lr * 2 + half) * kRtMaxKc;
                c[kRtMaxNk] = (j0 > 0 && lane < kc) ? lst[lane] : 0ull;
                __builtin_amdgcn_wave_barrier();
                sort_desc(c);
                wave_extract(c, kc, lst, lane);
                __builtin_amdgcn_wave_barrier();
            }
        }
    }

    // Combine the two candidate lists of each row and take the canonical top-k.
    for (int rr = 0; rr < kRtRowsPerWave; ++rr) {
        const int lr = wave * kRtRowsPerWave + rr;
        const int64_t r = row0 + lr;
        if (r >= rows) break;
        const uint64_t* l1 = lists + ((size_t)lr * 2 + 0) * kRtMaxKc;
        const uint64_t* l2 = lists + ((size_t)lr * 2 + 1) * kRtMaxKc;
        uint64_t c[kRtCombSlots];
#pragma unroll
        for (int s = 0; s < kRtCombSlots; ++s) {
            const int p = lane * kRtCombSlots + s;
            const int a = p / kc, b = p - a * kc;
            if (p < kc * kc) {
                const uint64_t ka = l1[a], kb = l2[b];
                const float v = Elem<T>::round32(key_score(ka) + key_score(kb));
                c[s] = make_key(v, key_idx(ka) * (uint32_t)K + key_idx(kb));
            } else {
                c[s] = 0ull;
            }
        }
        sort_desc(c);
        wave_extract(c, top_k, topk, lane);
        __builtin_amdgcn_wave_barrier();
        const float m = key_score(topk[0]);
        float sum = 0.0f;
        for (int i = 0; i < top_k; ++i) sum += expf(key_score(topk[i]) - m);
        if (lane < top_k) {
            const uint64_t k = topk[lane];
            const float ex = expf(key_score(k) - m);
            out_ids[r * top_k + lane] = (int32_t)key_idx(k);
            out_gates[r * top_k + lane] = Elem<T>::from_f32(ex / sum);
        }
        __builtin_amdgcn_wave_barrier();
    }
}

// Keys per LDS tile for a sub-key width and element size (multiple of 64, <= 512).
int route_tile_keys(int K, int dh2, int elem_bytes) {
    int kt = kRtTileBytes / (dh2 * elem_bytes);
    kt = (kt / kWave) * kWave;
    if (kt > kRtMaxNk * kWave) kt = kRtMaxNk * kWave;
    const int kround = ((K + kWave - 1) / kWave) * kWave;
    if (kt > kround) kt = kround;
    return kt;
}

size_t route_smem_bytes(int dh2, int KT, int elem_bytes) {
    size_t off = ((size_t)dh2 * KT * elem_bytes + 15) & ~(size_t)15;
    off += (size_t)kRtWaves * dh2 * sizeof(double);
    off += (size_t)kRtRows * 2 * kRtMaxKc * sizeof(uint64_t);
    off += (size_t)kRtWaves * kRtMaxKc * sizeof(uint64_t);
    return off;
}

int launch_route(const void* q, const void* k1, const void* k2, int64_t rows, int dq, int K, int top_k, int kc,
                 int dtype, void* gates, int32_t* ids, hipStream_t stream) {
    const int eb = dtype == kBF16 ? 2 : 4;
    const int dh2 = dq / 2;
    const int KT = route_tile_keys(K, dh2, eb);
    const size_t smem = route_smem_bytes(dh2, KT, eb);
    dim3 grid((unsigned)((rows + kRtRows - 1) / kRtRows));
    if (dtype == kBF16)
        hipLaunchKernelGGL(route_kernel<uint16_t>, grid, dim3(256), smem, stream, (const uint16_t*)q,
                           (const uint16_t*)k1, (const uint16_t*)k2, rows, dq, K, top_k, kc, KT,
                           (uint16_t*)gates, ids);
    else
        hipLaunchKernelGGL(route_kernel<float>, grid, dim3(256), smem, stream, (const float*)q, (const float*)k1,
                           (const float*)k2, rows, dq, K, top_k, kc, KT, (float*)gates, ids);
    return (int)hipGetLastError();
}

}  // namespace ethos
