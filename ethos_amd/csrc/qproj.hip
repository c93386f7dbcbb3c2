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
// bf16: exact integer MFMA projection on three int8 digit planes per operand.
//
// Every row r of x and of Wq gets a fixed-point format of its own:
//     v_i = 2^(E_r - 21) F_i + res_i,   F_i = trunc(v_i 2^(21 - E_r)),   |v_i| < 2^E_r,
// so |F_i| < 2^21 and F_i = 2^14 D0_i + 2^7 D1_i + D2_i with D0 in [-128, 127] and D1, D2
// in [0, 127]: three int8 digit planes.  Elements within 14 binades of 2^E_r are exact
// (res_i = 0); each of the n_r others has |res_i| < 2^(E_r - 21).  i8 MFMAs add the 9
// digit-pair products in int32 without rounding (|C_k| < 3 d 2^14 < 2^31 for d <= 16384):
//     P = sum_i F^x_i F^w_i = sum_k 2^(7 (4 - k)) C_k,   C_k = sum_{a+b=k} sum_i Da^x_i Db^w_i,
// an exact int64, so V = 2^(E_x + E_w - 42) P is the exact dot product of the truncated
// operands, and
//     |x.w - V| <= n_x 2^(E_x - 21) max|w| + n_w 2^(E_w - 21) max|x|.
// The fp64 FMA chain the contract defines is within d 2^-53 sum_i |x_i w_i| <=
// d 2^-53 min(max|x| |w|_1, max|w| |x|_1) of x.w.  With those bounds (1% slack), 2^-50 of
// the magnitudes for the fp64 evaluation and one subnormal ulp (so that a zero sum keeps
// its sign undecided), RN_T(lo) == RN_T(hi) settles RN_T(fl64(chain + b)).  Rows with a
// non-finite value and sums within the bound of a rounding boundary are queued and
// recomputed with the exact chain.
// ---------------------------------------------------------------------------------
constexpr int kQiPad = 64;              // digit rows are padded to a multiple of this many bytes
constexpr int kQiMaxD = 16384;          // int32 digit-product sums cannot overflow below this

struct QRowMeta {
    int32_t e;        // E_r: every |v_i| < 2^E_r
    int32_t n_inex;   // elements not exact in the digit format; -1: the row holds inf / NaN
    float l1;         // upper bound of sum |v_i|
    float amax;       // upper bound of max |v_i|
};

// Small batches (at most kQiSplitMaxTok tokens, whose 64 x 64 output tiles would leave most
// CUs idle) split the reduction into kQiSplit ranges of chunks, one workgroup each; each
// writes its exact partial digit-product sums P (int64) and a second kernel adds the
// kQiSplit partials of every element (integers: exact, in any order) and certifies them.
constexpr int kQiSplit = 8;
constexpr int64_t kQiSplitMaxTok = 128;

struct QprojWs {
    int8_t* xdig;     // [3][n_tok][dpad]
    int8_t* wdig;     // [3][ncols][dpad]
    QRowMeta* meta;   // [n_tok + ncols]: x rows, then Wq rows
    int64_t* part;    // [kQiSplit][n_tok][ncols] partial sums (n_tok <= kQiSplitMaxTok only)
};

__host__ __device__ inline int qproj_dpad(int d) { return (d + kQiPad - 1) / kQiPad * kQiPad; }

__host__ __device__ inline size_t qproj_align(size_t b) { return (b + 255) & ~(size_t)255; }

__host__ __device__ inline size_t qproj_ws_bytes(int64_t n_tok, int ncols, int d) {
    const size_t rows = (size_t)n_tok + (size_t)ncols;
    const size_t part = n_tok <= kQiSplitMaxTok ? (size_t)kQiSplit * (size_t)n_tok * (size_t)ncols * 8 : 0;
    return qproj_align(3 * rows * (size_t)qproj_dpad(d)) + qproj_align(sizeof(QRowMeta) * rows) + qproj_align(part);
}

__host__ __device__ inline QprojWs qproj_ws(void* ws, int64_t n_tok, int ncols, int d) {
    unsigned char* p = reinterpret_cast<unsigned char*>(ws);
    const size_t dpad = (size_t)qproj_dpad(d);
    QprojWs w;
    w.xdig = reinterpret_cast<int8_t*>(p);
    w.wdig = w.xdig + 3 * (size_t)n_tok * dpad;
    p += qproj_align(3 * ((size_t)n_tok + ncols) * dpad);
    w.meta = reinterpret_cast<QRowMeta*>(p);
    p += qproj_align(sizeof(QRowMeta) * ((size_t)n_tok + ncols));
    w.part = n_tok <= kQiSplitMaxTok ? reinterpret_cast<int64_t*>(p) : nullptr;
    return w;
}

__device__ __forceinline__ uint32_t qp_wave_max_u32(uint32_t v) { return (uint32_t)wave_max_u64((uint64_t)v); }

// One wave per row of x (rows < n_tok) or Wq (the n_rows - n_tok rows after them): digit
// planes and the row's format.
__global__ __launch_bounds__(256) void qproj_digits_kernel(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ w, int n_tok, int ncols,
                                                           int64_t n_rows, int d, int8_t* __restrict__ xdig,
                                                           int8_t* __restrict__ wdig, QRowMeta* __restrict__ xmeta,
                                                           QRowMeta* __restrict__ wmeta) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (row >= n_rows) return;
    const bool is_x = row < n_tok;
    const int64_t r = is_x ? row : row - n_tok;
    const uint16_t* src = (is_x ? x : w) + r * d;
    const int dpad = qproj_dpad(d);
    const int64_t plane = (int64_t)(is_x ? n_tok : ncols) * dpad;
    int8_t* dst = (is_x ? xdig : wdig) + r * dpad;
    const int ng = d / 8, npad = dpad / 8;

    // The row's first kDigCache groups of 8 per lane (rows of up to 2048 elements entirely)
    // are loaded once, all before any is used, and serve both passes; groups past the row
    // load group 0 again, unused.
    constexpr int kDigCache = 4;
    uint4 cv[kDigCache];
#pragma unroll
    for (int c = 0; c < kDigCache; ++c) {
        const int g = lane + c * kWave;
        cv[c] = *reinterpret_cast<const uint4*>(src + 8 * (g < ng ? g : 0));
    }

    // pass 1: largest biased exponent, inf / NaN, |.|_1 and max |.|
    uint32_t emax = 0, amax_bits = 0;
    bool bad = false;
    float l1 = 0.0f;
    auto scan = [&](const uint4 v) {
        const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t bits = (wd[j >> 1] >> (16 * (j & 1))) & 0x7fffu;
            const uint32_t e = bits >> 7;
            emax = max(emax, e);
            bad |= e == 0xffu;
            amax_bits = max(amax_bits, bits);
            l1 += __uint_as_float(bits << 16);
        }
    };
#pragma unroll
    for (int c = 0; c < kDigCache; ++c)
        if (lane + c * kWave < ng) scan(cv[c]);
    for (int g = lane + kDigCache * kWave; g < ng; g += kWave) scan(*reinterpret_cast<const uint4*>(src + 8 * g));
    emax = qp_wave_max_u32(emax);
    bad = __ballot(bad) != 0;
    // subnormal floor: the bounds stay upper bounds even if fp32 arithmetic flushes them
    const float amax = __uint_as_float(qp_wave_max_u32(amax_bits) << 16) + 0x1p-126f;
    l1 = wave_sum(l1) * (1.0f + 0x1p-10f) + (float)d * 0x1p-126f;
    const int E = (int)max(emax, 1u) - 126;

    // pass 2: F = trunc(v 2^(21 - E)) from the bit fields, split into three digits
    int n_inex = 0;
    auto digits = [&](int g, const uint4 v, bool live) {
        uint32_t p0[2] = {0u, 0u}, p1[2] = {0u, 0u}, p2[2] = {0u, 0u};
        if (live) {
            const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t bits = (wd[j >> 1] >> (16 * (j & 1))) & 0xffffu;
                const uint32_t be = (bits >> 7) & 0xffu;
                const uint32_t m = be ? (0x80u | (bits & 0x7fu)) : (bits & 0x7fu);   // v = m 2^(e - 7)
                const int e = be ? (int)be - 127 : -126;
                const int sh = e + 14 - E;                                           // F = m 2^sh
                uint32_t f;
                if (sh >= 0) {
                    f = m << sh;
                } else {
                    const int rs = -sh;
                    f = rs < 8 ? (m >> rs) : 0u;
                    n_inex += (rs < 8 ? (m & ((1u << rs) - 1u)) : m) != 0u;
                }
                const int F = (bits & 0x8000u) ? -(int)f : (int)f;
                const uint32_t d0 = (uint32_t)(F >> 14) & 0xffu, d1 = ((uint32_t)F >> 7) & 0x7fu,
                               d2 = (uint32_t)F & 0x7fu;
                const int wi = j >> 2, sb = 8 * (j & 3);
                p0[wi] |= d0 << sb;
                p1[wi] |= d1 << sb;
                p2[wi] |= d2 << sb;
            }
        }
        *reinterpret_cast<uint2*>(dst + 8 * g) = make_uint2(p0[0], p0[1]);
        *reinterpret_cast<uint2*>(dst + plane + 8 * g) = make_uint2(p1[0], p1[1]);
        *reinterpret_cast<uint2*>(dst + 2 * plane + 8 * g) = make_uint2(p2[0], p2[1]);
    };
#pragma unroll
    for (int c = 0; c < kDigCache; ++c) {
        const int g = lane + c * kWave;
        if (g < npad) digits(g, cv[c], g < ng && !bad);
    }
    for (int g = lane + kDigCache * kWave; g < npad; g += kWave) {
        const bool live = g < ng && !bad;
        digits(g, live ? *reinterpret_cast<const uint4*>(src + 8 * g) : make_uint4(0u, 0u, 0u, 0u), live);
    }
    const int total_inex = (int)wave_sum((float)n_inex);
    if (lane == 0) {
        QRowMeta mt;
        mt.e = E;
        mt.n_inex = bad ? -1 : total_inex;
        mt.l1 = l1;
        mt.amax = amax;
        (is_x ? xmeta : wmeta)[r] = mt;
    }
}

typedef int32_t i32x16_t __attribute__((ext_vector_type(16)));

// An x row's format as the certification reads it: {max|x| 2^-E, |x|_1 2^-E, n_inex 2^-21}
// and {E, n_inex}.
__device__ __forceinline__ float4 qp_xf(const QRowMeta& m) {
    return make_float4(ldexpf(m.amax, -m.e), ldexpf(m.l1, -m.e), (float)m.n_inex * 0x1p-21f, 0.0f);
}
__device__ __forceinline__ int2 qp_xi(const QRowMeta& m) { return make_int2(m.e, m.n_inex); }

// An output column's format, bias and BatchNorm coefficients.
struct QColFmt {
    int ew, nw;        // E_w, n_inex of the Wq row (-1: inf / NaN)
    float aw, lw, mw;  // max|w| 2^-E_w, |w|_1 2^-E_w, n_inex 2^-21
    double b;
    float al, be;
};
__device__ __forceinline__ QColFmt qp_col(const QRowMeta& m, uint16_t bias, float alpha, float beta) {
    QColFmt f;
    f.ew = m.e;
    f.nw = m.n_inex;
    f.aw = ldexpf(m.amax, -m.e);
    f.lw = ldexpf(m.l1, -m.e);
    f.mw = (float)m.n_inex * 0x1p-21f;
    f.b = (double)bf16_bits_to_f32(bias);
    f.al = alpha;
    f.be = beta;
    return f;
}

// Certify one element from Pd, its digit-product sum P = sum_k 2^(7 (4 - k)) C_k as fp64
// (exact below 2^53, else rounded at most four times), and write its output bits to *out;
// false when the element must take the exact chain.  The error bounds are evaluated in fp32
// scaled by 2^-(E_x + E_w), where every term is O(1) (max|v| 2^-E lies in [1/2, 1), |v|_1
// 2^-E in [1/2, d]); the 1% slack covers their fp32 rounding.  P's partial sums (scaled to
// units of P) are integers of magnitude at most B = sum_i (|F_i| + 2^15)(|G_i| + 2^15) <=
// 2^42 H', where in units of 2^(E_x + E_w) H' = A' + 2^-6 (|x|_1 + |w|_1) + d 2^-12 and A'
// bounds sum |x_i w_i|.  Below 2^53 (H' < 2^11) P's fp64 form is exact; otherwise its
// roundings add at most 2^-51 H' to the error.  Branch-free: *out always receives bits,
// which are the element's value when the result is true (a provisional value otherwise).
__device__ __forceinline__ bool qp_certify_bits(double Pd, float4 xf, int2 xi, const QColFmt& cf, int d,
                                                uint16_t* out) {
    const float dscale = (float)d * 0x1p-52f;  // chain rounding: d 2^-52 A'
    const float dterm = (float)d * 0x1p-12f;
    const double V = ldexp(Pd, xi.x + cf.ew - 42);
    const float As = fminf(xf.x * cf.lw, cf.aw * xf.y);
    const float Hs = As + 0x1p-6f * (xf.y + cf.lw) + dterm;
    // Both rows exact in the digit format and H' < 2^11 (with margin for the rounding of
    // H'): V is exact, and so is every partial sum of the chain (an integer multiple of
    // 2^(E_x + E_w - 42) below 2^53 of them), so the chain never rounds and equals V (+0 for
    // a zero sum, as the chain from +0 gives); otherwise the certified interval.
    const bool exact = (xi.y | cf.nw) == 0 && Hs < 2047.0f;
    const float Es =
        1.01f * (__builtin_fmaf(dscale, As, __builtin_fmaf(xf.z, cf.aw, cf.mw * xf.x)) + 0x1p-51f * Hs);
    const double Ed = ldexp((double)Es, xi.x + cf.ew) + 0x1p-50 * (fabs(V) + fabs(cf.b)) + 0x1p-1074;
    const double E = exact ? 0.0 : Ed;
    const double sv = V + cf.b;  // the element lies in [sv - E, sv + E] (E = 0: it is sv)
    // The interval test in fp32, one paired conversion for both ends.  f = RN_f32(sv) is
    // within 2^-24 |f| of sv for 2^-100 <= |f| <= 2^100; E32 = RN_f32(E) >= E (1 - 2^-23) -
    // 2^-126 (flushed below 2^-126); so Ef, rounded twice, is >= E + |f| 2^-21 (1 - 2^-23).
    // With Ef <= |f| / 2 the ends f -+ Ef are normal and their fp32 roundings (at most
    // 1.5 |f| 2^-24 each) stay outside [sv - E, sv + E]; when RN_bf16 gives both ends the
    // same bits it is constant on the interval (rounding is monotone), so that is the
    // element's value.  An exact zero (E = 0, sv = +-0) is its own value.
    const float f = (float)sv;
    const float af = fabsf(f);
    const float Ef = __builtin_fmaf((float)E, 1.0f + 0x1p-20f, __builtin_fmaf(af, 0x1p-21f, 0x1p-125f));
    const uint32_t ends = pack_bf16x2(f - Ef, f + Ef);
    const bool zero = exact && sv == 0.0;
    const uint32_t lo = zero ? __float_as_uint(f) >> 16 : ends & 0xffffu;
    const bool sure = ((ends >> 16) == (ends & 0xffffu) && af >= 0x1p-100f && af <= 0x1p100f && Ef <= 0.5f * af) ||
                      zero;
    *out = f32_to_bf16_bits(__builtin_fmaf(bf16_bits_to_f32((uint16_t)lo), cf.al, cf.be));
    return sure && xi.y >= 0 && cf.nw >= 0;
}
// The same, writing *out only for a certified element.
__device__ __forceinline__ bool qp_certify(double Pd, float4 xf, int2 xi, const QColFmt& cf, int d, uint16_t* out) {
    uint16_t o;
    const bool sure = qp_certify_bits(Pd, xf, xi, cf, d, &o);
    if (sure) *out = o;
    return sure;
}

// The exact fp64 chain of one element e = t ncols + c (index order, as the contract defines),
// computed by the whole wave (every lane calls with the same e); lane 0 stores the element.
// A bf16 x bf16 product is exact in fp64 (16 significant bits, exponents within [-266,
// 256]), so fma(x_i, w_i, acc) == acc + x_i w_i bit for bit.  Exactness test: every product
// is an integer multiple of 2^L, L the smallest lowest-bit exponent of the non-zero products
// (a bf16 value with biased exponent b is a multiple of 2^(max(b, 1) - 134)), and so is every
// partial sum, in any order, of magnitude at most S = sum |x_i w_i|.  When S < 2^(L + 53)
// every such sum is exact in fp64: the chain never rounds and equals the wave's sum in any
// order.  (S is taken with a factor-2 margin for the rounding of its own sum; a non-finite
// product makes S non-finite and fails the test.)  Otherwise the lanes write the products of
// `chunk` indices at a time (a multiple of 8) to the wave's LDS scratch pw and lane 0 adds
// them in order.
__device__ __forceinline__ void qp_exact_element(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                              const uint16_t* __restrict__ bias, const float* __restrict__ alpha,
                                              const float* __restrict__ beta, int d, int ncols, int64_t e,
                                              double* pw, int chunk, uint16_t* __restrict__ q) {
    const int lane = threadIdx.x & 63;
    const int64_t t = e / ncols;
    const int c = (int)(e - t * ncols);
    const uint16_t* xr = x + t * d;
    const uint16_t* wr = w + (int64_t)c * d;
    double ls = 0.0, la = 0.0;
    int lmin = 0x7fffffff;
    for (int g = lane; g < d / 8; g += kWave) {
        const uint4 xa = *reinterpret_cast<const uint4*>(xr + 8 * g);
        const uint4 wa = *reinterpret_cast<const uint4*>(wr + 8 * g);
        const uint32_t xv[4] = {xa.x, xa.y, xa.z, xa.w};
        const uint32_t wv[4] = {wa.x, wa.y, wa.z, wa.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t xb = (xv[j >> 1] >> (16 * (j & 1))) & 0xffffu;
            const uint32_t wb = (wv[j >> 1] >> (16 * (j & 1))) & 0xffffu;
            const double pj = (double)__uint_as_float(xb << 16) * (double)__uint_as_float(wb << 16);
            if (pj != 0.0) {
                const int lx = max((int)((xb >> 7) & 0xffu), 1) - 134;
                const int lw = max((int)((wb >> 7) & 0xffu), 1) - 134;
                lmin = min(lmin, lx + lw);
            }
            ls += pj;
            la += fabs(pj);
        }
    }
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) {
        ls += __shfl_xor(ls, m, kWave);
        la += __shfl_xor(la, m, kWave);
        lmin = min(lmin, __shfl_xor(lmin, m, kWave));
    }
    double acc = ls;
    if (!(lmin == 0x7fffffff || la < ldexp(1.0, lmin + 52))) {
        acc = 0.0;
        for (int k0 = 0; k0 < d; k0 += chunk) {
            const int len = min(chunk, d - k0);  // a multiple of 8
            for (int g = lane; g < len / 8; g += kWave) {
                const uint4 xa = *reinterpret_cast<const uint4*>(xr + k0 + 8 * g);
                const uint4 wa = *reinterpret_cast<const uint4*>(wr + k0 + 8 * g);
                const uint32_t xv[4] = {xa.x, xa.y, xa.z, xa.w};
                const uint32_t wv[4] = {wa.x, wa.y, wa.z, wa.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    pw[8 * g + 2 * j] = (double)__uint_as_float(xv[j] << 16) * (double)__uint_as_float(wv[j] << 16);
                    pw[8 * g + 2 * j + 1] =
                        (double)__uint_as_float(xv[j] & 0xffff0000u) * (double)__uint_as_float(wv[j] & 0xffff0000u);
                }
            }
            __builtin_amdgcn_wave_barrier();
            if (lane == 0) {
#pragma unroll 8
                for (int i = 0; i < len; ++i) acc = acc + pw[i];
            }
            __builtin_amdgcn_wave_barrier();
        }
    }
    if (lane == 0) {
        const float ql = Elem<uint16_t>::round64(acc + (double)bf16_bits_to_f32(bias[c]));
        q[e] = f32_to_bf16_bits(__builtin_fmaf(ql, alpha[c], beta[c]));
    }
}

// Tile configuration: kWaves waves in kWaves / 2 rows x 2 columns, each wave 32 rows x
// 32 kCB columns; reduction chunks of kKC bytes of every digit row; kStages chunk buffers in
// LDS (kStages - 1 chunks in flight).  A chunk's copies are 1 KB blocks of kBR rows, dealt
// to the waves in turn.
template <int Waves, int CB, int Stages, int KC>
struct QiCfg {
    static constexpr int kWaves = Waves, kCB = CB, kStages = Stages, kKC = KC;
    static constexpr int kRows = 16 * kWaves;  // = 32 (kWaves / 2)
    static constexpr int kCols = 64 * kCB;
    static constexpr int kSl = kKC / 16;      // 16-byte slots per staged row
    static constexpr int kBR = 1024 / kKC;    // rows per 1 KB copy block
    static constexpr int kXBlk = kRows / kBR, kWBlk = kCols / kBR;  // blocks per x / w plane
    static constexpr int kCopies = 3 * (kXBlk + kWBlk) / kWaves;    // 1 KB copies per wave per chunk
    static constexpr int kStage = 3 * (kRows + kCols) * kKC;        // bytes of one chunk buffer
    static constexpr size_t kTiles = (size_t)kStages * kStage;
    static constexpr size_t kSmem = kTiles + kRows * (sizeof(float4) + sizeof(int2));
    static_assert((kKC == 32 || kKC == 64) && kQiPad % kKC == 0, "chunk width");
    static_assert(kRows % kBR == 0 && kCols % kBR == 0 && 3 * (kXBlk + kWBlk) % kWaves == 0, "copy blocks");
};
using QiLaunch = QiCfg<4, 1, 2, 64>;

// s_waitcnt with vmcnt(n) and no expcnt / lgkmcnt wait (gfx9 encoding: vmcnt bits [3:0]
// and [15:14], expcnt [6:4], lgkmcnt [11:8])
constexpr int vmcnt_imm(int n) { return 0x0f70 | (n & 15) | ((n >> 4) << 14); }

// LDS chunk buffer layout: x digit planes 0-2 (kRows rows of kKC bytes each), then w digit
// planes 0-2 (kCols rows each); each row's 16-byte slots XOR-swizzled (64-byte rows: with
// bits 2-3 of the row; 32-byte rows: with bit 3) so that the MFMA fragment reads (16 lanes
// on 16 consecutive rows, one slot) hit 64 distinct banks.  The chunk buffers form a ring:
// the copies of the next kStages - 1 chunks are in flight while one chunk is multiplied.
template <int KC>
__device__ __forceinline__ int qi_slot(int row, int piece) {
    if constexpr (KC == 64) return piece ^ ((row >> 2) & 3);
    else return piece ^ ((row >> 3) & 1);
}

// Tile order of the i8 product kernel, for the per-XCD L2s (workgroup b runs on XCD
// b % 8): the tiles are ordered by column group of kQiColGroup column tiles, then row
// block, then column tile, and XCD x takes the x-th eighth of that order.  So each XCD
// works on a rectangle of about as many row blocks as column tiles: a row block's x digit
// planes are read by the consecutive workgroups of its column group on one XCD, and the
// group's w digit planes (kQiColGroup * 64 columns, 3 MB at d_model 1024) stay in that
// XCD's L2, instead of every XCD reading every row block.  The grid is padded to a
// multiple of 8; false for the padding workgroups.
constexpr int kQiColGroup = 16;
template <int kRowsT, int kColsT>
__device__ __forceinline__ bool qi_tile_t(int n_tok, int ncols, int* t0, int* c0) {
    const int nct = (ncols + kColsT - 1) / kColsT, nrb = (n_tok + kRowsT - 1) / kRowsT;
    const int total = nct * nrb, per = (total + 7) / 8;
    const int i = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
    if (i >= total) return false;
    const int cg = nct < kQiColGroup ? nct : kQiColGroup;  // column tiles per group (the last may be short)
    const int grp = i / (cg * nrb), r = i - grp * cg * nrb;
    const int w = nct - grp * cg < cg ? nct - grp * cg : cg;  // this group's column tiles
    *t0 = (r / w) * kRowsT;
    *c0 = (grp * cg + r % w) * kColsT;
    return true;
}

template <int kWaves, int kCB, int kStages, int kKC, bool kSplit>
__global__ __launch_bounds__(kWaves * 64) void qproj_i8_kernel(const int8_t* __restrict__ xdig,
                                                                 const int8_t* __restrict__ wdig,
                                                                 const QRowMeta* __restrict__ xmeta,
                                                                 const QRowMeta* __restrict__ wmeta,
                                                                 const uint16_t* __restrict__ bias,
                                                                 const float* __restrict__ alpha,
                                                                 const float* __restrict__ beta, int n_tok, int d,
                                                                 int ncols, const uint16_t* __restrict__ x,
                                                                 const uint16_t* __restrict__ w,
                                                                 uint16_t* __restrict__ q, int64_t* __restrict__ part) {
    using C = QiCfg<kWaves, kCB, kStages, kKC>;
    constexpr int kQiRows = C::kRows, kQiCols = C::kCols;
    auto qi_tile = [](int n, int nc, int* t, int* c) { return qi_tile_t<kQiRows, kQiCols>(n, nc, t, c); };
    extern __shared__ __align__(16) unsigned char qsm[];
    int8_t* tiles = reinterpret_cast<int8_t*>(qsm);  // [stage][x planes, w planes][row][64 B]
    // x row formats, scaled by 2^-E_x: {max|x| 2^-E, |x|_1 2^-E, n_inex 2^-21} and {E, n_inex}
    float4* xpf = reinterpret_cast<float4*>(qsm + C::kTiles);
    int2* xpi = reinterpret_cast<int2*>(qsm + C::kTiles + kQiRows * sizeof(float4));
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int h = lane >> 5, l32 = lane & 31;
    const int wr = wave >> 1, wc = wave & 1;  // rows 32 wr .., columns 32 kCB wc ..
    int t0, c0;
    if (!qi_tile(n_tok, ncols, &t0, &c0)) return;
    const int dpad = qproj_dpad(d);
    // the chunks this workgroup reduces: all of them, or (kSplit) range blockIdx.y of
    // gridDim.y ranges (possibly empty: its partial sums are then zero)
    const int nch = dpad / kKC;
    int k_lo = 0, k_hi = nch;
    if constexpr (kSplit) {
        const int cps = (nch + (int)gridDim.y - 1) / (int)gridDim.y;
        k_lo = min(nch, (int)blockIdx.y * cps);
        k_hi = min(nch, k_lo + cps);
    }
    const int64_t xplane = (int64_t)n_tok * dpad, wplane = (int64_t)ncols * dpad;

    // Copies: the chunk's 1 KB blocks (x planes 0-2, then w planes 0-2, each plane's blocks of
    // kBR rows in order) go to the waves in turn, block b to wave b % kWaves; lane l writes
    // block bytes 16 l .. 16 l + 15 = block row l / kSl, slot l % kSl, so it loads the piece
    // that the swizzle puts in that slot.  Buffer descriptors bounded by the tile's live rows
    // return zeros past the last token / column.
    const int xrows = max(0, min(kQiRows, n_tok - t0)), wrows = max(0, min(kQiCols, ncols - c0));
    i32x4_t rs[6];
#pragma unroll
    for (int p = 0; p < 3; ++p) {
        rs[p] = buffer_rsrc(xdig + p * xplane + (int64_t)t0 * dpad, (uint32_t)(xrows * dpad));
        rs[3 + p] = buffer_rsrc(wdig + p * wplane + (int64_t)c0 * dpad, (uint32_t)(wrows * dpad));
    }
#pragma unroll
    for (int r = 0; r < 6; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) rs[r][j] = __builtin_amdgcn_readfirstlane(rs[r][j]);
    auto xplane_lds = [&](int stage, int p) { return tiles + (size_t)stage * C::kStage + p * kQiRows * kKC; };
    auto wplane_lds = [&](int stage, int p) {
        return tiles + (size_t)stage * C::kStage + (3 * kQiRows + p * kQiCols) * kKC;
    };
    // this wave's blocks: descriptor, LDS offset within a chunk buffer and lane offset
    i32x4_t brs[C::kCopies];
    int blds[C::kCopies], bvoff[C::kCopies];
#pragma unroll
    for (int j = 0; j < C::kCopies; ++j) {
        const int b = wave + kWaves * j;  // wave-uniform
        const bool isw = b >= 3 * C::kXBlk;
        const int bb = isw ? b - 3 * C::kXBlk : b, nb = isw ? C::kWBlk : C::kXBlk;
        const int p = bb / nb, rb = bb - p * nb;
        const int row = rb * C::kBR + lane / C::kSl;
        brs[j] = rs[(isw ? 3 : 0) + p];
#pragma unroll
        for (int q = 0; q < 4; ++q) brs[j][q] = __builtin_amdgcn_readfirstlane(brs[j][q]);  // (scalar operands)
        blds[j] = __builtin_amdgcn_readfirstlane((isw ? 3 * kQiRows + p * kQiCols : p * kQiRows) * kKC + rb * 1024);
        bvoff[j] = row * dpad + 16 * qi_slot<kKC>(row, lane % C::kSl);
    }
    auto issue = [&](int k0, int stage) {
#pragma unroll
        for (int j = 0; j < C::kCopies; ++j)
            lds_dma16(brs[j], bvoff[j], k0, lds_addr(tiles + (size_t)stage * C::kStage + blds[j]));
    };
    static_assert(kStages >= 2 && kStages <= 4, "waits cover at most two chunks in flight past the current one");

    // the first chunk's copies go out before the metadata loads, so that one wait covers both
    if (k_lo < k_hi) issue(k_lo * kKC, 0);
    if (!kSplit && tid < kQiRows && t0 + tid < n_tok) {
        const QRowMeta m = xmeta[t0 + tid];
        xpf[tid] = qp_xf(m);
        xpi[tid] = qp_xi(m);
    }
    // the lane's output columns' formats, bias and BatchNorm coefficients, for the epilogue
    // (loaded now so that the epilogue does not wait for them)
    QRowMeta cmeta[kCB];
    uint16_t cbias[kCB];
    float calpha[kCB], cbeta[kCB];
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb) {
        const int c = c0 + wc * 32 * kCB + cb * 32 + l32;
        const bool ok = !kSplit && c < ncols;
        cmeta[cb] = ok ? wmeta[c] : QRowMeta{0, -1, 0.0f, 0.0f};
        cbias[cb] = ok ? bias[c] : (uint16_t)0;
        calpha[cb] = ok ? alpha[c] : 0.0f;
        cbeta[cb] = ok ? beta[c] : 0.0f;
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // these loads and the first chunk's copies

    i32x16_t acc[kCB][5];
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
        for (int k = 0; k < 5; ++k)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[cb][k][i] = 0;

    const int arow = wr * 32 + l32;
#pragma unroll
    for (int j = 1; j < kStages - 1; ++j)
        if (k_lo + j < k_hi) issue((k_lo + j) * kKC, j);
    for (int kc = k_lo; kc < k_hi; ++kc) {
        const int stage = (kc - k_lo) % kStages;
        // this wave's copies of chunk kc have landed once at most those of the chunks after
        // it that are already issued (up to kStages - 2 of them, kCopies each) are pending
        const int ahead = min(kStages - 2, k_hi - 1 - kc);
        if (kStages == 2 || ahead == 0)
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        else if (ahead == 1)
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(C::kCopies));
        else
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * C::kCopies));
        __syncthreads();  // every wave's copies of chunk kc landed; chunk kc - 1 fully read
        const int kn = kc + kStages - 1;
        if (kn < k_hi) issue(kn * kKC, (kn - k_lo) % kStages);  // into chunk kc - 1's buffer
#pragma unroll
        for (int s = 0; s < kKC; s += 32) {
            const int piece = s / 16 + h;
            i32x4_t a[3], b[kCB][3];
            const int aoff = arow * kKC + 16 * qi_slot<kKC>(arow, piece);
#pragma unroll
            for (int p = 0; p < 3; ++p) a[p] = *reinterpret_cast<const i32x4_t*>(xplane_lds(stage, p) + aoff);
#pragma unroll
            for (int cb = 0; cb < kCB; ++cb) {
                const int brow = wc * 32 * kCB + cb * 32 + l32;
                const int boff = brow * kKC + 16 * qi_slot<kKC>(brow, piece);
#pragma unroll
                for (int p = 0; p < 3; ++p) b[cb][p] = *reinterpret_cast<const i32x4_t*>(wplane_lds(stage, p) + boff);
            }
#pragma unroll
            for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
                for (int pa = 0; pa < 3; ++pa)
#pragma unroll
                    for (int pb = 0; pb < 3; ++pb)
                        acc[cb][pa + pb] =
                            __builtin_amdgcn_mfma_i32_32x32x32_i8(a[pa], b[cb][pb], acc[cb][pa + pb], 0, 0, 0);
        }
    }

    if constexpr (kSplit) {
        // this range's exact partial sums P = sum_k 2^(7 (4 - k)) C_k (|P| < 2^61), one
        // int64 per live element
#pragma unroll
        for (int cb = 0; cb < kCB; ++cb) {
            const int c = c0 + wc * 32 * kCB + cb * 32 + l32;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int t = t0 + wr * 32 + mfma32_row(i, lane);
                if (c < ncols && t < n_tok) {
                    int64_t P = acc[cb][0][i];
#pragma unroll
                    for (int k = 1; k < 5; ++k) P = P * 128 + acc[cb][k][i];
                    part[((int64_t)blockIdx.y * n_tok + t) * ncols + c] = P;
                }
            }
        }
        return;
    }
    // Certify each element and store it; the uncertain ones then take the exact chain, one at
    // a time per wave (which overwrites their provisional values).  No branches per element,
    // so that the compiler can overlap the elements' dependent chains: the stores go through
    // a buffer descriptor over the tile's rows, with an out-of-range offset for the lanes past
    // the last column or token (dropped by the hardware).  The exact chains use the chunk
    // buffer of the second-to-last chunk as scratch: every wave finished reading it before the
    // barrier of the last chunk, and no copy goes into it after that barrier.
    constexpr int kPwChunk = (int)(C::kStage / (kWaves * sizeof(double))) / 8 * 8;
    static_assert(kPwChunk >= 64, "exact-chain scratch");
    const int free_stage = k_hi - k_lo >= 2 ? (k_hi - k_lo - 2) % kStages : 1;
    double* const pw = reinterpret_cast<double*>(tiles + (size_t)free_stage * C::kStage) + (size_t)wave * kPwChunk;
    const __amdgpu_buffer_rsrc_t qrs =
        __builtin_amdgcn_make_buffer_rsrc(q + (int64_t)t0 * ncols, 0, max(0, min(kQiRows, n_tok - t0)) * ncols * 2,
                                          0x00020000);
#pragma unroll
  for (int cb = 0; cb < kCB; ++cb) {
    const int c = c0 + wc * 32 * kCB + cb * 32 + l32;
    const bool col_ok = c < ncols;
    const QColFmt cf = qp_col(cmeta[cb], cbias[cb], calpha[cb], cbeta[cb]);
    uint32_t unsure = 0;  // bit i: element i is live and uncertain
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int tl = wr * 32 + mfma32_row(i, lane);
        const bool live = col_ok && t0 + tl < n_tok;
        // P by an fp64 Horner chain on the int32 sums (exact below 2^53, else four roundings)
        double Pd = (double)acc[cb][0][i];
        Pd = __builtin_fma(Pd, 128.0, (double)acc[cb][1][i]);
        Pd = __builtin_fma(Pd, 128.0, (double)acc[cb][2][i]);
        Pd = __builtin_fma(Pd, 128.0, (double)acc[cb][3][i]);
        Pd = __builtin_fma(Pd, 128.0, (double)acc[cb][4][i]);
        uint16_t o;
        const bool sure = qp_certify_bits(Pd, xpf[tl], xpi[tl], cf, d, &o);
        __builtin_amdgcn_raw_buffer_store_b16(o, qrs, live ? (tl * ncols + c) * 2 : -1, 0, 0);
        unsure |= (uint32_t)(live && !sure) << i;
    }
    // (rare) the wave's uncertain elements, lowest lane first
    for (uint64_t pend = __ballot(unsure != 0u); pend != 0; pend = __ballot(unsure != 0u)) {
        const int lead = __builtin_ctzll(pend);
        const int i = __builtin_ctz(__builtin_amdgcn_readlane(unsure, lead));
        const int tl = wr * 32 + mfma32_row(i, lead);
        const int cl = c0 + wc * 32 * kCB + cb * 32 + (lead & 31);
        qp_exact_element(x, w, bias, alpha, beta, d, ncols, (int64_t)(t0 + tl) * ncols + cl, pw, kPwChunk, q);
        if (lane == lead) unsure &= unsure - 1u;
    }
  }
}

// Split reductions: element e = t ncols + c (one thread each) adds the kQiSplit partial sums
// of the ranges (int64, exact), converts once to fp64 (exact below 2^53) and is certified
// as in the product kernel; a wave's uncertain elements take the exact chain in turn.
__global__ __launch_bounds__(256) void qproj_split_finish_kernel(const int64_t* __restrict__ part,
                                                                 const QRowMeta* __restrict__ xmeta,
                                                                 const QRowMeta* __restrict__ wmeta,
                                                                 const uint16_t* __restrict__ bias,
                                                                 const float* __restrict__ alpha,
                                                                 const float* __restrict__ beta, int n_tok, int d,
                                                                 int ncols, int n_split, const uint16_t* __restrict__ x,
                                                                 const uint16_t* __restrict__ w,
                                                                 uint16_t* __restrict__ q) {
    constexpr int kFinChunk = 512;
    __shared__ __align__(16) double scratch_pw[4][kFinChunk];
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t n_el = (int64_t)n_tok * ncols;
    const bool live = e < n_el;
    bool sure = false;
    if (live) {
        const int t = (int)(e / ncols), c = (int)(e - (int64_t)t * ncols);
        const QRowMeta xm = xmeta[t];
        const QColFmt cf = qp_col(wmeta[c], bias[c], alpha[c], beta[c]);
        // every partial sum requested before any is added (integers: exact in any order)
        int64_t pv[kQiSplit];
#pragma unroll
        for (int s = 0; s < kQiSplit; ++s) pv[s] = s < n_split ? part[(int64_t)s * n_el + e] : 0;
        int64_t P = 0;
#pragma unroll
        for (int s = 0; s < kQiSplit; ++s) P += pv[s];
        uint16_t o;
        sure = qp_certify((double)P, qp_xf(xm), qp_xi(xm), cf, d, &o);
        if (sure) q[e] = o;
    }
    bool unsure = live && !sure;
    for (uint64_t pend = __ballot(unsure); pend != 0; pend = __ballot(unsure)) {
        const int lead = __builtin_ctzll(pend);
        const int64_t el = (int64_t)blockIdx.x * 256 + (threadIdx.x & ~63) + lead;
        qp_exact_element(x, w, bias, alpha, beta, d, ncols, el, scratch_pw[threadIdx.x >> 6], kFinChunk, q);
        if ((int)(threadIdx.x & 63) == lead) unsure = false;
    }
}

size_t qproj_workspace_bytes(int64_t n_tok, int ncols, int d, int dtype) {
    return dtype == kBF16 && d <= kQiMaxD ? qproj_ws_bytes(n_tok, ncols, d) : 0;
}

// Prepared weights: Wq's digit planes [3][ncols][dpad] and row formats [ncols], computed
// once (launch_qproj_prepare) and read by every later projection with the same Wq.
size_t qproj_weights_bytes(int ncols, int d, int dtype) {
    if (dtype != kBF16 || d > kQiMaxD) return 0;
    return qproj_align(3 * (size_t)ncols * qproj_dpad(d)) + qproj_align(sizeof(QRowMeta) * (size_t)ncols);
}

static void prepared_parts(const void* prepared, int ncols, int d, const int8_t** wdig, const QRowMeta** wmeta) {
    const unsigned char* p = static_cast<const unsigned char*>(prepared);
    *wdig = reinterpret_cast<const int8_t*>(p);
    *wmeta = reinterpret_cast<const QRowMeta*>(p + qproj_align(3 * (size_t)ncols * qproj_dpad(d)));
}

int launch_qproj_prepare(const void* w, int ncols, int d, int dtype, void* prepared, hipStream_t stream) {
    if (qproj_weights_bytes(ncols, d, dtype) == 0) return 0;
    const int8_t* wdig;
    const QRowMeta* wmeta;
    prepared_parts(prepared, ncols, d, &wdig, &wmeta);
    hipLaunchKernelGGL(qproj_digits_kernel, dim3((unsigned)((ncols + 3) / 4)), dim3(256), 0, stream, nullptr,
                       (const uint16_t*)w, 0, ncols, (int64_t)ncols, d, nullptr, const_cast<int8_t*>(wdig), nullptr,
                       const_cast<QRowMeta*>(wmeta));
    return (int)hipGetLastError();
}

int launch_qproj(const void* x, const void* w, const void* prepared, const void* b, const float* alpha,
                 const float* beta, int64_t n_tok, int d, int ncols, int dtype, void* ws, void* q, int num_cus,
                 hipStream_t stream) {
    if (dtype == kBF16 && d <= kQiMaxD) {
        const QprojWs W = qproj_ws(ws, n_tok, ncols, d);
        const int8_t* wdig = W.wdig;
        const QRowMeta* wmeta = W.meta + n_tok;
        // with prepared weights only the rows of x are converted
        const int64_t rows = prepared ? n_tok : n_tok + ncols;
        if (prepared) prepared_parts(prepared, ncols, d, &wdig, &wmeta);
        hipLaunchKernelGGL(qproj_digits_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream,
                           (const uint16_t*)x, (const uint16_t*)w, (int)n_tok, ncols, rows, d, W.xdig, W.wdig, W.meta,
                           W.meta + n_tok);
        using C = QiLaunch;
        const int64_t tiles = (int64_t)((ncols + C::kCols - 1) / C::kCols) * ((n_tok + C::kRows - 1) / C::kRows);
        const unsigned tgrid = (unsigned)(8 * ((tiles + 7) / 8));  // qi_tile_t: XCD-grouped tile order
        if (W.part != nullptr) {
            hipLaunchKernelGGL((qproj_i8_kernel<C::kWaves, C::kCB, C::kStages, C::kKC, true>), dim3(tgrid, kQiSplit),
                               dim3(C::kWaves * 64), C::kSmem, stream, W.xdig, wdig, W.meta, wmeta,
                               (const uint16_t*)b, alpha, beta, (int)n_tok, d, ncols, (const uint16_t*)x,
                               (const uint16_t*)w, (uint16_t*)q, W.part);
            const int64_t n_el = n_tok * (int64_t)ncols;
            hipLaunchKernelGGL(qproj_split_finish_kernel, dim3((unsigned)((n_el + 255) / 256)), dim3(256), 0, stream,
                               (const int64_t*)W.part, (const QRowMeta*)W.meta, wmeta, (const uint16_t*)b, alpha, beta,
                               (int)n_tok, d, ncols, kQiSplit, (const uint16_t*)x, (const uint16_t*)w, (uint16_t*)q);
        } else {
            hipLaunchKernelGGL((qproj_i8_kernel<C::kWaves, C::kCB, C::kStages, C::kKC, false>), dim3(tgrid),
                               dim3(C::kWaves * 64), C::kSmem, stream, W.xdig, wdig, W.meta, wmeta,
                               (const uint16_t*)b, alpha, beta, (int)n_tok, d, ncols, (const uint16_t*)x,
                               (const uint16_t*)w, (uint16_t*)q, (int64_t*)nullptr);
        }
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
