// Query projection + eval-mode Query BatchNorm for all routing heads
// (reference: model.py:195-202,215-216, nn.Linear(d_model, d_query) then BatchNorm1d).
//
//   q[t, h, o] = RN_T( fmaf( RN_T( sum_i x[t,i] * Wq[h,o,i]  +  b[h,o] ), alpha[h,o], beta[h,o] ) )
//
// The dot product is an fp64 fused-multiply-add chain taken in index order i = 0..d-1.
// For bf16 operands every product and every partial sum is exact in fp64, so the
// result is the correctly rounded dot product whatever the order; for fp32 operands
// the fixed order makes it reproducible.  alpha/beta are the fp32 BatchNorm eval
// coefficients (w / sqrt(var + eps), b - mean * alpha) computed once on the host.
#pragma clang fp contract(off)

#include "ethos_common.hpp"
#include "ethos_launch.hpp"
#include "ethos_mfma.hpp"

namespace ethos {

constexpr int kQpTM = 64;   // tokens per tile
constexpr int kQpTN = 64;   // output columns (h*dq + o) per tile
constexpr int kQpKC = 32;   // reduction chunk staged in LDS

template <typename T>
__global__ __launch_bounds__(256) void qproj_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                    const T* __restrict__ bias, const float* __restrict__ alpha,
                                                    const float* __restrict__ beta, int n_tok, int d, int ncols,
                                                    T* __restrict__ q) {
    __shared__ double xs[kQpKC][kQpTM];
    __shared__ double ws[kQpKC][kQpTN];
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    const int c0 = blockIdx.x * kQpTN;
    const int t0 = blockIdx.y * kQpTM;

    double acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0;

    for (int k0 = 0; k0 < d; k0 += kQpKC) {
        const int kc = min(kQpKC, d - k0);
        for (int e = tid; e < kQpTM * kQpKC; e += 256) {
            const int r = e / kQpKC, kk = e % kQpKC;
            const bool kin = kk < kc;
            xs[kk][r] = (kin && t0 + r < n_tok) ? Elem<T>::to_f64(x[(int64_t)(t0 + r) * d + k0 + kk]) : 0.0;
            ws[kk][r] = (kin && c0 + r < ncols) ? Elem<T>::to_f64(w[(int64_t)(c0 + r) * d + k0 + kk]) : 0.0;
        }
        __syncthreads();
        for (int kk = 0; kk < kc; ++kk) {
            double a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = xs[kk][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = ws[kk][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fma(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = t0 + ty * 4 + i;
        if (t >= n_tok) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = c0 + tx * 4 + j;
            if (c >= ncols) continue;
            const double lin = acc[i][j] + Elem<T>::to_f64(bias[c]);
            const float ql = Elem<T>::round64(lin);
            const float qb = __builtin_fmaf(ql, alpha[c], beta[c]);
            q[(int64_t)t * ncols + c] = Elem<T>::from_f32(qb);
        }
    }
}

// ---------------------------------------------------------------------------------
// bf16: certified MFMA projection with exact refinement.
//
// Every 16-term slice of the dot product is one 32x32x16 MFMA on a zero accumulator;
// bf16 x bf16 products are exact in fp32, so however the MFMA orders its 15
// additions, each rounded at worst like a truncating fp32 add, the slice is within
// 15 * 2^-23 of the sum of its |x_i w_i|.  Slices are added in fp64 (error <= 2^-46 of
// the same sum over 1024 terms), and A = sum |x_i w_i| itself comes from a second MFMA
// on sign-cleared operands (fp32, relative error < 2^-12).  Hence
//     |S~ - S| <= E = (15 * 2^-23 + 2^-46) * 1.001 * A * (1 + 2^-12) + 2^-50 (|S~| + |b|),
// and when RN_T(S~ + b - E) == RN_T(S~ + b + E) the correctly rounded projection is
// known; the rest (about 1% on random data) is queued and recomputed exactly.
// ---------------------------------------------------------------------------------
constexpr int kQmRows = 64;    // tokens per workgroup tile (2 waves x 32)
constexpr int kQmCols = 128;   // output columns per workgroup tile (2 waves x 64)
constexpr int kQmKC = 64;      // reduction chunk staged in LDS
constexpr int kQmPitch = kQmKC + 8;

struct QprojWs {
    int32_t* count;   // [1]   uncertain elements
    int32_t* list;    // [n_tok * ncols]
};

__host__ __device__ inline size_t qproj_ws_bytes(int64_t n_tok, int ncols) {
    return 256 + 4 * (size_t)n_tok * ncols + 64;
}

__host__ __device__ inline QprojWs qproj_ws(void* ws, int64_t n_tok, int ncols) {
    (void)n_tok;
    (void)ncols;
    unsigned char* p = reinterpret_cast<unsigned char*>(ws);
    QprojWs w;
    w.count = reinterpret_cast<int32_t*>(p);
    w.list = reinterpret_cast<int32_t*>(p + 256);
    return w;
}

__global__ void qproj_clear_kernel(int32_t* __restrict__ count) { *count = 0; }

__device__ __forceinline__ bf16x8_t abs_bf16x8(bf16x8_t v) {
    uint4 u = __builtin_bit_cast(uint4, v);
    u.x &= 0x7fff7fffu;
    u.y &= 0x7fff7fffu;
    u.z &= 0x7fff7fffu;
    u.w &= 0x7fff7fffu;
    return __builtin_bit_cast(bf16x8_t, u);
}

constexpr int kQmLocal = 1024;  // uncertain elements a workgroup resolves itself (4 per thread)

__global__ __launch_bounds__(256) void qproj_mfma_kernel(const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ w,
                                                         const uint16_t* __restrict__ bias,
                                                         const float* __restrict__ alpha,
                                                         const float* __restrict__ beta, int n_tok, int d, int ncols,
                                                         int32_t* __restrict__ count, int32_t* __restrict__ list,
                                                         uint16_t* __restrict__ q) {
    __shared__ __align__(16) uint16_t xs[kQmRows * kQmPitch];
    __shared__ __align__(16) uint16_t ws[kQmCols * kQmPitch];
    __shared__ uint32_t local[kQmLocal];  // (row << 16) | column within the tile
    __shared__ int n_local;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int h = lane >> 5, l32 = lane & 31;
    const int wr = wave >> 1, wc = wave & 1;
    const int t0 = blockIdx.y * kQmRows, c0 = blockIdx.x * kQmCols;
    if (tid == 0) n_local = 0;

    // x [64 x 64] and w [128 x 64] chunks in 16-byte pieces (rows past the end are zero):
    // piece e = tid + 256 j is row e / 8, k offset 8 (e % 8); rows < 64 are x, the rest w
    constexpr int kPieces = (kQmRows + kQmCols) * (kQmKC / 8) / 256;
    static_assert((kQmRows + kQmCols) * (kQmKC / 8) % 256 == 0 && kQmRows * (kQmKC / 8) % 256 == 0,
                  "staging shape");
    auto fetch = [&](int k0, uint4 (&v)[kPieces]) {
#pragma unroll
        for (int j = 0; j < kPieces; ++j) {
            const int e = tid + 256 * j;
            const int r = e / (kQmKC / 8), kq = (e % (kQmKC / 8)) * 8;
            v[j] = make_uint4(0, 0, 0, 0);
            if (r < kQmRows) {
                if (t0 + r < n_tok) v[j] = *reinterpret_cast<const uint4*>(x + (int64_t)(t0 + r) * d + k0 + kq);
            } else {
                const int rc = r - kQmRows;
                if (c0 + rc < ncols) v[j] = *reinterpret_cast<const uint4*>(w + (int64_t)(c0 + rc) * d + k0 + kq);
            }
        }
    };
    auto put = [&](const uint4 (&v)[kPieces]) {
#pragma unroll
        for (int j = 0; j < kPieces; ++j) {
            const int e = tid + 256 * j;
            const int r = e / (kQmKC / 8), kq = (e % (kQmKC / 8)) * 8;
            if (r < kQmRows)
                *reinterpret_cast<uint4*>(&xs[r * kQmPitch + kq]) = v[j];
            else
                *reinterpret_cast<uint4*>(&ws[(r - kQmRows) * kQmPitch + kq]) = v[j];
        }
    };
    auto stage = [&](int k0) {
        uint4 v[kPieces];
        fetch(k0, v);
        put(v);
    };

    double acc64[2][16];
    f32x16_t accA[2] = {f32x16_zero(), f32x16_zero()};
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc64[cb][i] = 0.0;

    // the next chunk is fetched into registers while this one is multiplied
    uint4 nxt[kPieces];
    fetch(0, nxt);
    for (int k0 = 0; k0 < d; k0 += kQmKC) {
        __syncthreads();
        put(nxt);
        __syncthreads();
        if (k0 + kQmKC < d) fetch(k0 + kQmKC, nxt);
#pragma unroll
        for (int kk = 0; kk < kQmKC; kk += 16) {
            const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(&xs[(wr * 32 + l32) * kQmPitch + kk + 8 * h]);
            const bf16x8_t aa = abs_bf16x8(a);
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
                const bf16x8_t b =
                    *reinterpret_cast<const bf16x8_t*>(&ws[(wc * 64 + cb * 32 + l32) * kQmPitch + kk + 8 * h]);
                const f32x16_t c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, f32x16_zero(), 0, 0, 0);
                accA[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aa, abs_bf16x8(b), accA[cb], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 16; ++i) acc64[cb][i] += (double)c[i];
            }
        }
    }

    // certify each element; store it, or queue it: first in LDS, past kQmLocal globally
    const double kBound = (15.0 * 0x1p-23 + 0x1p-46) * 1.001 * (1.0 + 0x1p-12);
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        const int cl = wc * 64 + cb * 32 + l32;
        const int c = c0 + cl;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int tl = wr * 32 + mfma32_row(i, lane);
            const int t = t0 + tl;
            const bool live = t < n_tok && c < ncols;
            bool sure = true;
            if (live) {
                const double s = acc64[cb][i];
                const double b = (double)bf16_bits_to_f32(bias[c]);
                const double e = kBound * (double)accA[cb][i] + 0x1p-50 * (fabs(s) + fabs(b)) + 0x1p-1000;
                const uint16_t lo = Elem<uint16_t>::from_f64((s - e) + b);
                const uint16_t hi = Elem<uint16_t>::from_f64((s + e) + b);
                sure = lo == hi;
                if (sure) {
                    const float qb = __builtin_fmaf(bf16_bits_to_f32(lo), alpha[c], beta[c]);
                    q[(int64_t)t * ncols + c] = f32_to_bf16_bits(qb);
                }
            }
            const bool queue = live && !sure;
            const uint64_t bal = __ballot(queue);
            if (bal) {
                const int leader = __builtin_ctzll(bal);
                const int rank = (int)__popcll(bal & ((1ull << lane) - 1ull));
                int base = 0;
                if (lane == leader) base = atomicAdd(&n_local, (int)__popcll(bal));
                base = __shfl(base, leader, 64);
                if (queue) {
                    const int slot = base + rank;
                    if (slot < kQmLocal) {
                        local[slot] = ((uint32_t)tl << 16) | (uint32_t)cl;
                    } else {
                        const int g = atomicAdd(count, 1);
                        list[g] = t * ncols + c;
                    }
                }
            }
        }
    }
    __syncthreads();
    const int nl = n_local < kQmLocal ? n_local : kQmLocal;

    // Exact fp64 chains for the queued elements, re-streaming the same K tiles: each
    // thread runs two elements' chains side by side (each in index order, 16-byte LDS
    // reads of eight terms), 512 elements per pass.
    for (int g0 = 0; g0 < nl; g0 += 512) {
        int er[2], ec[2];
        bool ok[2];
        double ex[2] = {0.0, 0.0};
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int j = g0 + 256 * r + tid;
            ok[r] = j < nl;
            const uint32_t v = ok[r] ? local[j] : 0u;
            er[r] = (int)(v >> 16);
            ec[r] = (int)(v & 0xffffu);
        }
        for (int k0 = 0; k0 < d; k0 += kQmKC) {
            __syncthreads();
            stage(k0);
            __syncthreads();
#pragma unroll 2
            for (int kk = 0; kk < kQmKC; kk += 8) {
                uint4 xa[2], wa[2];
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    xa[r] = *reinterpret_cast<const uint4*>(&xs[er[r] * kQmPitch + kk]);
                    wa[r] = *reinterpret_cast<const uint4*>(&ws[ec[r] * kQmPitch + kk]);
                }
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                        for (int r = 0; r < 2; ++r) {
                            const uint32_t xv = (&xa[r].x)[q], wv = (&wa[r].x)[q];
                            const float xf = __uint_as_float(hf ? (xv & 0xffff0000u) : (xv << 16));
                            const float wf = __uint_as_float(hf ? (wv & 0xffff0000u) : (wv << 16));
                            ex[r] = fma((double)xf, (double)wf, ex[r]);
                        }
            }
        }
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            if (ok[r]) {
                const int t = t0 + er[r], c = c0 + ec[r];
                const float ql = Elem<uint16_t>::round64(ex[r] + (double)bf16_bits_to_f32(bias[c]));
                q[(int64_t)t * ncols + c] = f32_to_bf16_bits(__builtin_fmaf(ql, alpha[c], beta[c]));
            }
        }
    }
}

// Exact fp64 chain for the queued elements (index order, as the contract defines).
__global__ __launch_bounds__(256) void qproj_fixup_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ w,
                                                          const uint16_t* __restrict__ bias,
                                                          const float* __restrict__ alpha,
                                                          const float* __restrict__ beta, int d, int ncols,
                                                          const int32_t* __restrict__ count,
                                                          const int32_t* __restrict__ list, uint16_t* __restrict__ q) {
    const int n = *count;
    for (int idx = blockIdx.x * 256 + threadIdx.x; idx < n; idx += gridDim.x * 256) {
        const int e = list[idx];
        const int t = e / ncols, c = e - t * ncols;
        const uint16_t* xr = x + (int64_t)t * d;
        const uint16_t* wr = w + (int64_t)c * d;
        double acc = 0.0;
        for (int i = 0; i < d; i += 8) {
            const uint4 xa = *reinterpret_cast<const uint4*>(xr + i);
            const uint4 wa = *reinterpret_cast<const uint4*>(wr + i);
            const uint32_t xv[4] = {xa.x, xa.y, xa.z, xa.w};
            const uint32_t wv[4] = {wa.x, wa.y, wa.z, wa.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc = fma((double)__uint_as_float(xv[j] << 16), (double)__uint_as_float(wv[j] << 16), acc);
                acc = fma((double)__uint_as_float(xv[j] & 0xffff0000u), (double)__uint_as_float(wv[j] & 0xffff0000u),
                          acc);
            }
        }
        const float ql = Elem<uint16_t>::round64(acc + (double)bf16_bits_to_f32(bias[c]));
        q[e] = f32_to_bf16_bits(__builtin_fmaf(ql, alpha[c], beta[c]));
    }
}

size_t qproj_workspace_bytes(int64_t n_tok, int ncols, int dtype) {
    return dtype == kBF16 ? qproj_ws_bytes(n_tok, ncols) : 0;
}

int launch_qproj(const void* x, const void* w, const void* b, const float* alpha, const float* beta, int64_t n_tok,
                 int d, int ncols, int dtype, void* ws, void* q, int num_cus, hipStream_t stream) {
    if (dtype == kBF16 && d % kQmKC == 0) {
        const QprojWs W = qproj_ws(ws, n_tok, ncols);
        hipLaunchKernelGGL(qproj_clear_kernel, dim3(1), dim3(1), 0, stream, W.count);
        dim3 grid((ncols + kQmCols - 1) / kQmCols, (unsigned)((n_tok + kQmRows - 1) / kQmRows));
        hipLaunchKernelGGL(qproj_mfma_kernel, grid, dim3(256), 0, stream, (const uint16_t*)x, (const uint16_t*)w,
                           (const uint16_t*)b, alpha, beta, (int)n_tok, d, ncols, W.count, W.list, (uint16_t*)q);
        hipLaunchKernelGGL(qproj_fixup_kernel, dim3((unsigned)num_cus * 4), dim3(256), 0, stream, (const uint16_t*)x,
                           (const uint16_t*)w, (const uint16_t*)b, alpha, beta, d, ncols, W.count, W.list,
                           (uint16_t*)q);
        return (int)hipGetLastError();
    }
    dim3 grid((ncols + kQpTN - 1) / kQpTN, (unsigned)((n_tok + kQpTM - 1) / kQpTM));
    if (dtype == kBF16)
        hipLaunchKernelGGL(qproj_kernel<uint16_t>, grid, dim3(256), 0, stream, (const uint16_t*)x,
                           (const uint16_t*)w, (const uint16_t*)b, alpha, beta, (int)n_tok, d, ncols, (uint16_t*)q);
    else
        hipLaunchKernelGGL(qproj_kernel<float>, grid, dim3(256), 0, stream, (const float*)x, (const float*)w,
                           (const float*)b, alpha, beta, (int)n_tok, d, ncols, (float*)q);
    return (int)hipGetLastError();
}

}  // namespace ethos
