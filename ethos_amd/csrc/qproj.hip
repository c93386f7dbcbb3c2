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

int launch_qproj(const void* x, const void* w, const void* b, const float* alpha, const float* beta, int64_t n_tok,
                 int d, int ncols, int dtype, void* q, hipStream_t stream) {
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
