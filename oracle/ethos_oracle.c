/*
 * ethos_oracle.c -- CPU oracle for the ETHOS expert-layer forward path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (ethos_amd/) links, loads or
 * calls this file; only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
 * leg use it, as the checker.  The product path fails loudly when its HIP library
 * is missing instead of falling back to this code.
 *
 * What it restates (reference = wrmedford/ETHOS):
 *   - query projection + eval-mode Query BatchNorm  model.py:195-202,215-216
 *   - sub-key scoring, per-half top-(2k), k_cand x k_cand combination,
 *     final top-k, fp32 softmax, index decode         model.py:217-245
 *   - head stacking [rows = token*H + head]           model.py:250-252
 *   - reordering of (token, head, k) pairs by expert id (no reference code; the
 *     paper's Algorithm 1 reorders by expert, paper/ETHOS.pdf p.10)
 *
 * Numeric contract (shared with the HIP kernels, which are written independently):
 *   dot64(a,b)   : acc = 0.0; for i in order: acc = fma((double)a_i, (double)b_i, acc)
 *                  For bf16 operands every product is exact in fp64 and the running
 *                  sum is exact unless the operands span > ~37 binades, so the result
 *                  is the exact dot product; for fp32 operands it is the fp64
 *                  sequential value.
 *   RN_T(v)      : round-to-nearest-even of a double to the layer dtype T.  For bf16
 *                  it goes through a round-to-odd double->float step, which makes the
 *                  two-step rounding equal to one correct rounding.
 *   q_lin        = RN_T(dot64(x_t, Wq_h[o]) + (double)b_h[o])
 *   q            = RN_T(fmaf((float)q_lin, alpha[o], beta[o]))   alpha/beta: fp32 BN
 *                  eval coefficients computed by the caller.
 *   s1[j], s2[j] = RN_T(dot64(q[0:dq/2], K1[j])), RN_T(dot64(q[dq/2:dq], K2[j]))
 *   canonical order everywhere: score descending, then index ascending (sub-key
 *                  index for the per-half lists, expert id for the combined list);
 *                  -0.0 compares equal to +0.0.
 *   c[a][b]      = RN_T((float)v1[a] + (float)v2[b])  (the add is an fp32 add)
 *   g            = RN_T(ex_i / sum_i ex_i), ex_i = (float)exp((double)(f_i - f_0)): the fp64
 *                  exponential rounded once to fp32, fp32 sum and divide, sum in list order
 *   e            = i1[a] * K + i2[b]
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_F32 0
#define ORC_BF16 1

/* ---------------------------------------------------------------- scalars */

static inline float orc_bits_to_f32(uint32_t b) {
    float f;
    memcpy(&f, &b, 4);
    return f;
}
static inline uint32_t orc_f32_to_bits(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    return b;
}
static inline float orc_bf16_to_f32(uint16_t h) { return orc_bits_to_f32((uint32_t)h << 16); }

/* float -> bf16, round to nearest even (NaN kept quiet). */
static inline uint16_t orc_f32_to_bf16(float f) {
    uint32_t b = orc_f32_to_bits(f);
    if ((b & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((b >> 16) | 0x0040u);
    b += 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}

/* double -> float rounded to odd: the float that truncates d, with its last bit
 * forced to 1 when the conversion was inexact. */
static inline float orc_f64_to_f32_odd(double d) {
    float f = (float)d;
    if ((double)f == d || isnan(d) || isinf(f)) return f;
    uint32_t b = orc_f32_to_bits(f);
    if ((b & 1u) == 0u) {
        if (fabs((double)f) > fabs(d)) b -= 1u; /* step toward zero */
        else b += 1u;                           /* step away from zero */
    }
    return orc_bits_to_f32(b);
}

/* Correctly rounded double -> bf16. */
static inline uint16_t orc_f64_to_bf16(double d) { return orc_f32_to_bf16(orc_f64_to_f32_odd(d)); }

/* Load element i of a dtype-T array as double / float. */
static inline double orc_ld64(const void* p, int64_t i, int dt) {
    if (dt == ORC_BF16) return (double)orc_bf16_to_f32(((const uint16_t*)p)[i]);
    return (double)((const float*)p)[i];
}

/* Round a double to T and return the T value as float (exact). */
static inline float orc_round64(double v, int dt) {
    if (dt == ORC_BF16) return orc_bf16_to_f32(orc_f64_to_bf16(v));
    return (float)v;
}
/* Round a float to T and return the T value as float (exact). */
static inline float orc_round32(float v, int dt) {
    if (dt == ORC_BF16) return orc_bf16_to_f32(orc_f32_to_bf16(v));
    return v;
}
static inline void orc_store(void* p, int64_t i, float v_in_T, int dt) {
    if (dt == ORC_BF16) ((uint16_t*)p)[i] = orc_f32_to_bf16(v_in_T);
    else ((float*)p)[i] = v_in_T;
}

/* Sequential fp64 FMA dot product of two dtype-T vectors with element strides. */
static double orc_dot64(const void* a, int64_t a0, const void* b, int64_t b0, int n, int dt) {
    double acc = 0.0;
    for (int i = 0; i < n; ++i) acc = fma(orc_ld64(a, a0 + i, dt), orc_ld64(b, b0 + i, dt), acc);
    return acc;
}

/* Order-preserving 32-bit image of a float (larger float -> larger uint); -0 == +0. */
static inline uint32_t orc_ord32(float f) {
    uint32_t b = orc_f32_to_bits(f);
    if (b == 0x80000000u) b = 0u;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
/* Canonical selection key: larger key = earlier in the canonical order. */
static inline uint64_t orc_key(float score, uint32_t idx) {
    return ((uint64_t)orc_ord32(score) << 32) | (uint64_t)(uint32_t)(~idx);
}
static inline uint32_t orc_key_idx(uint64_t key) { return ~(uint32_t)(key & 0xffffffffu); }

static int orc_cmp_desc(const void* pa, const void* pb) {
    uint64_t a = *(const uint64_t*)pa, b = *(const uint64_t*)pb;
    return (a < b) - (a > b);
}

/* Sort keys[0..n) descending: the first c entries are then the canonical top-c. */
static void orc_sort_desc(uint64_t* keys, int n) {
    qsort(keys, (size_t)n, sizeof(uint64_t), orc_cmp_desc);
}

/* ------------------------------------------------------------ public API */

/* Query projection + eval BatchNorm (model.py:215-216).
 *   x     [n_tok, d]        dtype T
 *   Wq    [H, dq, d]        dtype T   (stacked nn.Linear weights, [out, in])
 *   bq    [H, dq]           dtype T
 *   alpha [H, dq], beta [H, dq]  fp32 BN eval coefficients
 *   q_out [n_tok, H, dq]    dtype T
 */
void ethos_oracle_query_proj(const void* x, const void* Wq, const void* bq, const float* alpha,
                             const float* beta, int64_t n_tok, int d, int H, int dq, int dt,
                             void* q_out) {
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < n_tok; ++t) {
        for (int h = 0; h < H; ++h) {
            for (int o = 0; o < dq; ++o) {
                int64_t w_row = ((int64_t)h * dq + o) * d;
                double acc = orc_dot64(x, t * d, Wq, w_row, d, dt);
                acc = acc + orc_ld64(bq, (int64_t)h * dq + o, dt);
                float ql = orc_round64(acc, dt);
                float qb = fmaf(ql, alpha[(int64_t)h * dq + o], beta[(int64_t)h * dq + o]);
                orc_store(q_out, (t * H + h) * dq + o, orc_round32(qb, dt), dt);
            }
        }
    }
}

/* Sub-key scores for one row half: out[j] = RN_T(dot64(q_half, keys[j])). */
void ethos_oracle_subkey_scores(const void* q, const void* keys, int64_t rows, int dq, int half,
                                int K, int dt, float* out) {
    int dh2 = dq / 2;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r)
        for (int j = 0; j < K; ++j)
            out[r * K + j] =
                orc_round64(orc_dot64(q, r * dq + (int64_t)half * dh2, keys, (int64_t)j * dh2, dh2, dt), dt);
}

/* Recover the float from the high half of a canonical key. */
static inline float orc_key_score(uint64_t key) {
    uint32_t o = (uint32_t)(key >> 32);
    return orc_bits_to_f32((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

typedef struct {
    uint64_t *k1, *k2, *kc;
    float *v1, *v2, *fv, *ex;
    uint32_t *i1, *i2;
} orc_scratch;

static int orc_scratch_alloc(orc_scratch* s, int K, int top_k, int k_cand) {
    s->k1 = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)K);
    s->k2 = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)K);
    s->kc = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)k_cand * (size_t)k_cand);
    s->v1 = (float*)malloc(sizeof(float) * (size_t)k_cand);
    s->v2 = (float*)malloc(sizeof(float) * (size_t)k_cand);
    s->i1 = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)k_cand);
    s->i2 = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)k_cand);
    s->fv = (float*)malloc(sizeof(float) * (size_t)top_k);
    s->ex = (float*)malloc(sizeof(float) * (size_t)top_k);
    return s->k1 && s->k2 && s->kc && s->v1 && s->v2 && s->i1 && s->i2 && s->fv && s->ex;
}
static void orc_scratch_free(orc_scratch* s) {
    free(s->k1); free(s->k2); free(s->kc); free(s->v1); free(s->v2);
    free(s->i1); free(s->i2); free(s->fv); free(s->ex);
}

/* Selection stage for one row, given its two score vectors (already in T):
 * per-half canonical top-k_cand (model.py:224-226), k_cand x k_cand dtype sums
 * (model.py:229-230), canonical top-k by (score desc, expert id asc) (model.py:233),
 * fp32 softmax cast to T (model.py:234), decode e = i1*K + i2 (model.py:237-245). */
static void orc_select_row(const float* s1, const float* s2, int64_t r, int K, int top_k, int k_cand,
                           int dt, orc_scratch* s, void* out_scores, int32_t* out_ids, int32_t* out_cand) {
    for (int j = 0; j < K; ++j) {
        s->k1[j] = orc_key(s1[j], (uint32_t)j);
        s->k2[j] = orc_key(s2[j], (uint32_t)j);
    }
    orc_sort_desc(s->k1, K);
    orc_sort_desc(s->k2, K);
    for (int a = 0; a < k_cand; ++a) {
        s->i1[a] = orc_key_idx(s->k1[a]);
        s->i2[a] = orc_key_idx(s->k2[a]);
        s->v1[a] = orc_key_score(s->k1[a]);
        s->v2[a] = orc_key_score(s->k2[a]);
        if (out_cand) {
            out_cand[(r * 2 + 0) * k_cand + a] = (int32_t)s->i1[a];
            out_cand[(r * 2 + 1) * k_cand + a] = (int32_t)s->i2[a];
        }
    }
    for (int a = 0; a < k_cand; ++a)
        for (int b = 0; b < k_cand; ++b) {
            float c = orc_round32(s->v1[a] + s->v2[b], dt);
            uint32_t e = s->i1[a] * (uint32_t)K + s->i2[b];
            s->kc[a * k_cand + b] = orc_key(c, e);
        }
    orc_sort_desc(s->kc, k_cand * k_cand);
    for (int i = 0; i < top_k; ++i) {
        s->fv[i] = orc_key_score(s->kc[i]);
        out_ids[r * top_k + i] = (int32_t)orc_key_idx(s->kc[i]);
    }
    float m = s->fv[0], sum = 0.0f;
    for (int i = 0; i < top_k; ++i) {
        s->ex[i] = (float)exp((double)(s->fv[i] - m));
        sum += s->ex[i];
    }
    for (int i = 0; i < top_k; ++i) orc_store(out_scores, r * top_k + i, orc_round32(s->ex[i] / sum, dt), dt);
}

/* Product-key routing for `rows` independent (token, head) rows (model.py:217-245).
 *   q       [rows, dq]        dtype T
 *   K1, K2  [K, dq/2]         dtype T   (sub_keys_1.weight, sub_keys_2.weight)
 *   out_scores [rows, top_k]  dtype T   softmax gates
 *   out_ids    [rows, top_k]  int32     expert ids, canonical order
 *   out_cand   optional [rows, 2, k_cand] int32: per-half candidate sub-key ids
 * Returns 0, or -1 when the sizes are out of range (k_cand > K, top_k > k_cand^2).
 */
int ethos_oracle_route(const void* q, const void* K1, const void* K2, int64_t rows, int dq, int K,
                       int top_k, int k_cand, int dt, void* out_scores, int32_t* out_ids,
                       int32_t* out_cand) {
    if (k_cand > K || top_k > k_cand * k_cand || top_k < 1 || k_cand < 1 || dq % 2 != 0) return -1;
    int dh2 = dq / 2;
    int err = 0;
#pragma omp parallel
    {
        orc_scratch s;
        float* s1 = (float*)malloc(sizeof(float) * (size_t)K);
        float* s2 = (float*)malloc(sizeof(float) * (size_t)K);
        if (!orc_scratch_alloc(&s, K, top_k, k_cand) || !s1 || !s2) {
#pragma omp atomic write
            err = -2;
        } else {
#pragma omp for schedule(static)
            for (int64_t r = 0; r < rows; ++r) {
                for (int j = 0; j < K; ++j) {
                    s1[j] = orc_round64(orc_dot64(q, r * dq, K1, (int64_t)j * dh2, dh2, dt), dt);
                    s2[j] = orc_round64(orc_dot64(q, r * dq + dh2, K2, (int64_t)j * dh2, dh2, dt), dt);
                }
                orc_select_row(s1, s2, r, K, top_k, k_cand, dt, &s, out_scores, out_ids, out_cand);
            }
        }
        orc_scratch_free(&s);
        free(s1);
        free(s2);
    }
    return err;
}

/* Selection stage only, from given score matrices s1, s2 [rows, K] (float32 holding
 * T values).  Lets tests drive the selection with scores computed elsewhere. */
int ethos_oracle_select(const float* s1, const float* s2, int64_t rows, int K, int top_k, int k_cand,
                        int dt, void* out_scores, int32_t* out_ids, int32_t* out_cand) {
    if (k_cand > K || top_k > k_cand * k_cand || top_k < 1 || k_cand < 1) return -1;
    int err = 0;
#pragma omp parallel
    {
        orc_scratch s;
        if (!orc_scratch_alloc(&s, K, top_k, k_cand)) {
#pragma omp atomic write
            err = -2;
        } else {
#pragma omp for schedule(static)
            for (int64_t r = 0; r < rows; ++r)
                orc_select_row(s1 + r * K, s2 + r * K, r, K, top_k, k_cand, dt, &s, out_scores, out_ids, out_cand);
        }
        orc_scratch_free(&s);
    }
    return err;
}

/* Reordering of pairs by expert id: a stable counting sort.
 *   ids      [n_pairs] int32, each in [0, n_experts)
 *   perm     [n_pairs] int32  pair indices ordered by (expert id, pair index)
 *   uniq     [>= U]    int32  distinct expert ids, ascending
 *   seg_off  [>= U+1]  int32  seg_off[u]..seg_off[u+1] = positions in perm of slot u
 *   inv      [n_pairs] int32  slot of each pair
 * Returns U (>= 0) or -1 when an id is out of range.
 */
int64_t ethos_oracle_sort_segment(const int32_t* ids, int64_t n_pairs, int64_t n_experts, int32_t* perm,
                                  int32_t* uniq, int32_t* seg_off, int32_t* inv) {
    int64_t* cnt = (int64_t*)calloc((size_t)n_experts + 1, sizeof(int64_t));
    int32_t* slot = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n_experts > 0 ? n_experts : 1));
    if (!cnt || !slot) { free(cnt); free(slot); return -2; }
    for (int64_t p = 0; p < n_pairs; ++p) {
        if (ids[p] < 0 || ids[p] >= n_experts) { free(cnt); free(slot); return -1; }
        cnt[ids[p] + 1]++;
    }
    int64_t U = 0;
    for (int64_t e = 0; e < n_experts; ++e) {
        if (cnt[e + 1] > 0) {
            uniq[U] = (int32_t)e;
            seg_off[U] = (int32_t)cnt[e];
            slot[e] = (int32_t)U;
            ++U;
        }
        cnt[e + 1] += cnt[e];
    }
    seg_off[U] = (int32_t)n_pairs;
    for (int64_t p = 0; p < n_pairs; ++p) {
        int32_t e = ids[p];
        perm[cnt[e]++] = (int32_t)p;
        inv[p] = slot[e];
    }
    free(cnt);
    free(slot);
    return U;
}

/* Scalar helpers exported so tests can pin them against exact rational arithmetic. */
uint16_t ethos_oracle_f64_to_bf16(double d) { return orc_f64_to_bf16(d); }
uint16_t ethos_oracle_f32_to_bf16(float f) { return orc_f32_to_bf16(f); }
double ethos_oracle_dot64(const void* a, const void* b, int n, int dt) { return orc_dot64(a, 0, b, 0, n, dt); }
