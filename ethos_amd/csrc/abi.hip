// C-ABI of the ETHOS expert-layer kernels (declared in include/ethos_hip.h).
// Every entry point validates its arguments, enqueues on the caller's stream, never
// allocates, never throws, and returns 0 on success, a negative ETHOS_E* code for an
// argument error, or a positive hipError_t; ethos_last_error() describes the last
// failure of the calling thread.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

#include "../../include/ethos_hip.h"
#include "ethos_common.hpp"
#include "ethos_launch.hpp"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int hip_status(int rc, const char* what) {
    if (rc == 0) return 0;
    return fail(rc, "%s: %s", what, hipGetErrorString((hipError_t)rc));
}

constexpr int kMaxDevices = 64;
std::atomic<int> g_num_cus[kMaxDevices];

int num_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    int n = g_num_cus[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        g_num_cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
bool dtype_ok(int dtype) { return dtype == ETHOS_F32 || dtype == ETHOS_BF16; }

// Sort workspace of ethos_sort_segment_noalloc: one array per GPU, in the code object's
// device data, sized for ETHOS_NOALLOC_MAX_PAIRS pairs (a batch that size sorts without
// the expert -> slot table).  Its name is only a host-side
// stand-in; kernels receive the device address that hipGetSymbolAddress returns for the
// current device (g_scratch_ptr), looked up once per device on the first call there.
constexpr size_t kScratchWords = ethos::sort_workspace_words(ETHOS_NOALLOC_MAX_PAIRS, (int64_t)1 << 18);
static __device__ __align__(256) uint32_t scratch[kScratchWords];
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device (nullptr and the error in g_err on failure).
void* scratch_ptr(int* rc) {
    int dev = 0;
    *rc = (int)hipGetDevice(&dev);
    if (*rc != 0) {
        fail(*rc, "ethos_sort_segment_noalloc: hipGetDevice: %s", hipGetErrorString((hipError_t)*rc));
        return nullptr;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        *rc = ETHOS_EUNSUPPORTED;
        fail(*rc, "ethos_sort_segment_noalloc: device %d beyond the %d this library tracks", dev, kMaxDevices);
        return nullptr;
    }
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (p) return p;
    *rc = (int)hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (*rc != 0 || !p) {
        if (*rc == 0) *rc = (int)hipErrorInvalidSymbol;
        fail(*rc, "ethos_sort_segment_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString((hipError_t)*rc));
        return nullptr;
    }
    g_scratch_ptr[dev].store(p, std::memory_order_release);
    return p;
}

// Stage events of the calling thread (ethos_stage_events): recorded in order, one per
// stage boundary, until the list is used up.
thread_local hipEvent_t g_events[16];
thread_local int g_n_events = 0, g_next_event = 0;

}  // namespace

namespace ethos {
void stage_mark(hipStream_t stream) {
    if (g_next_event < g_n_events) (void)hipEventRecord(g_events[g_next_event++], stream);
}
}  // namespace ethos

extern "C" {

int ethos_stage_events(void* const* events, int32_t n_events) {
    g_err[0] = 0;
    if (n_events < 0 || n_events > 16 || (n_events > 0 && !events))
        return fail(ETHOS_ESIZE, "ethos_stage_events: 0 to 16 events, got %d", n_events);
    for (int i = 0; i < n_events; ++i) {
        if (!events[i]) return fail(ETHOS_ENULL, "ethos_stage_events: event %d is NULL", i);
        g_events[i] = (hipEvent_t)events[i];
    }
    g_n_events = n_events;
    g_next_event = 0;
    return 0;
}

const char* ethos_last_error(void) { return g_err; }

int ethos_abi_version(void) { return ETHOS_ABI_VERSION; }

size_t ethos_query_proj_workspace_bytes(int64_t n_tok, int32_t d_model, int32_t n_heads, int32_t d_query,
                                        int32_t dtype) {
    if (n_tok <= 0 || d_model <= 0 || n_heads <= 0 || d_query <= 0) return 256;
    const size_t b = ethos::qproj_workspace_bytes(n_tok, n_heads * d_query, d_model, dtype);
    return b < 256 ? 256 : b;
}

static int query_proj_impl(const char* name, const void* x, const void* wq, const void* prepared, const void* bq,
                           const float* bn_alpha, const float* bn_beta, int64_t n_tok, int32_t d_model,
                           int32_t n_heads, int32_t d_query, int32_t dtype, void* workspace, size_t workspace_bytes,
                           void* q_out, void* stream) {
    g_err[0] = 0;
    if (!dtype_ok(dtype)) return fail(ETHOS_EDTYPE, "%s: unknown dtype %d", name, dtype);
    if (n_tok < 0 || d_model <= 0 || n_heads <= 0 || d_query <= 0)
        return fail(ETHOS_ESIZE, "%s: bad sizes n_tok=%lld d_model=%d n_heads=%d d_query=%d", name,
                    (long long)n_tok, d_model, n_heads, d_query);
    if ((int64_t)n_heads * d_query > INT32_MAX / 2 || n_tok * (int64_t)n_heads * d_query > INT32_MAX)
        return fail(ETHOS_ESIZE, "%s: n_tok * n_heads * d_query exceeds int32", name);
    if (n_tok == 0) return 0;
    if (!x || !wq || !bq || !bn_alpha || !bn_beta || !q_out) return fail(ETHOS_ENULL, "%s: null pointer", name);
    const size_t need = ethos_query_proj_workspace_bytes(n_tok, d_model, n_heads, d_query, dtype);
    if (dtype == ETHOS_BF16) {
        if (!workspace || workspace_bytes < need)
            return fail(ETHOS_EWORKSPACE, "%s: workspace of %zu bytes, %zu needed", name, workspace_bytes, need);
        if (!aligned16(workspace) || !aligned16(x) || !aligned16(wq) || (prepared && !aligned16(prepared)) ||
            (d_model % 8))
            return fail(ETHOS_EALIGN, "%s: x, wq, prepared, workspace 16-byte aligned and d_model %% 8 == 0", name);
    }
    if (ethos::qproj_weights_bytes(n_heads * d_query, d_model, dtype) == 0) prepared = nullptr;
    return hip_status(ethos::launch_qproj(x, wq, prepared, bq, bn_alpha, bn_beta, n_tok, d_model, n_heads * d_query,
                                          dtype, workspace, q_out, num_cus(), (hipStream_t)stream),
                      name);
}

int ethos_query_proj(const void* x, const void* wq, const void* bq, const float* bn_alpha, const float* bn_beta,
                     int64_t n_tok, int32_t d_model, int32_t n_heads, int32_t d_query, int32_t dtype, void* workspace,
                     size_t workspace_bytes, void* q_out, void* stream) {
    return query_proj_impl("ethos_query_proj", x, wq, nullptr, bq, bn_alpha, bn_beta, n_tok, d_model, n_heads,
                           d_query, dtype, workspace, workspace_bytes, q_out, stream);
}

size_t ethos_query_proj_weights_bytes(int32_t d_model, int32_t n_heads, int32_t d_query, int32_t dtype) {
    if (d_model <= 0 || n_heads <= 0 || d_query <= 0 || !dtype_ok(dtype)) return 0;
    return ethos::qproj_weights_bytes(n_heads * d_query, d_model, dtype);
}

int ethos_query_proj_prepare(const void* wq, int32_t d_model, int32_t n_heads, int32_t d_query, int32_t dtype,
                             void* prepared, size_t prepared_bytes, void* stream) {
    g_err[0] = 0;
    if (!dtype_ok(dtype)) return fail(ETHOS_EDTYPE, "ethos_query_proj_prepare: unknown dtype %d", dtype);
    if (d_model <= 0 || n_heads <= 0 || d_query <= 0 || (int64_t)n_heads * d_query > INT32_MAX / 2)
        return fail(ETHOS_ESIZE, "ethos_query_proj_prepare: bad sizes d_model=%d n_heads=%d d_query=%d", d_model,
                    n_heads, d_query);
    const size_t need = ethos_query_proj_weights_bytes(d_model, n_heads, d_query, dtype);
    if (need == 0) return 0;
    if (!wq || !prepared) return fail(ETHOS_ENULL, "ethos_query_proj_prepare: null pointer");
    if (prepared_bytes < need)
        return fail(ETHOS_EWORKSPACE, "ethos_query_proj_prepare: %zu bytes, %zu needed", prepared_bytes, need);
    if (!aligned16(wq) || !aligned16(prepared) || (d_model % 8))
        return fail(ETHOS_EALIGN, "ethos_query_proj_prepare: wq, prepared 16-byte aligned and d_model %% 8 == 0");
    return hip_status(ethos::launch_qproj_prepare(wq, n_heads * d_query, d_model, dtype, prepared,
                                                  (hipStream_t)stream),
                      "ethos_query_proj_prepare");
}

int ethos_query_proj_prepared(const void* x, const void* wq, const void* prepared, size_t prepared_bytes,
                              const void* bq, const float* bn_alpha, const float* bn_beta, int64_t n_tok,
                              int32_t d_model, int32_t n_heads, int32_t d_query, int32_t dtype, void* workspace,
                              size_t workspace_bytes, void* q_out, void* stream) {
    const size_t need = ethos_query_proj_weights_bytes(d_model, n_heads, d_query, dtype);
    if (need > 0 && n_tok > 0) {
        g_err[0] = 0;
        if (!prepared) return fail(ETHOS_ENULL, "ethos_query_proj_prepared: null prepared weights");
        if (prepared_bytes < need)
            return fail(ETHOS_EWORKSPACE, "ethos_query_proj_prepared: prepared weights of %zu bytes, %zu needed",
                        prepared_bytes, need);
    }
    return query_proj_impl("ethos_query_proj_prepared", x, wq, prepared, bq, bn_alpha, bn_beta, n_tok, d_model,
                           n_heads, d_query, dtype, workspace, workspace_bytes, q_out, stream);
}

static int route_checks(const char* name, int64_t n_rows, int32_t d_query, int32_t n_sub_keys, int32_t top_k,
                        int32_t k_cand, int32_t dtype) {
    if (!dtype_ok(dtype)) return fail(ETHOS_EDTYPE, "%s: unknown dtype %d", name, dtype);
    if (n_rows < 0 || d_query <= 0 || (d_query & 1) || n_sub_keys <= 0 || top_k <= 0 || k_cand <= 0)
        return fail(ETHOS_ESIZE, "%s: bad sizes rows=%lld d_query=%d K=%d top_k=%d k_cand=%d", name,
                    (long long)n_rows, d_query, n_sub_keys, top_k, k_cand);
    if (k_cand > n_sub_keys) return fail(ETHOS_ESIZE, "%s: k_cand=%d exceeds the %d sub-keys", name, k_cand, n_sub_keys);
    if (top_k > k_cand * k_cand) return fail(ETHOS_ESIZE, "%s: top_k=%d exceeds k_cand^2=%d", name, top_k, k_cand * k_cand);
    if (k_cand > 32 || top_k > 32)
        return fail(ETHOS_EUNSUPPORTED, "%s: k_cand=%d / top_k=%d above 32 are not supported", name, k_cand, top_k);
    if ((int64_t)n_sub_keys * n_sub_keys > INT32_MAX)
        return fail(ETHOS_EUNSUPPORTED, "%s: %d sub-keys give expert ids beyond int32", name, n_sub_keys);
    if (!ethos::route_supported(n_sub_keys, d_query / 2, dtype))
        return fail(ETHOS_EUNSUPPORTED,
                    "%s: needs n_sub_keys <= 512, d_query/2 <= 256 and d_query/2 %% %d == 0 (got %d, %d)", name,
                    dtype == ETHOS_BF16 ? 16 : 4, n_sub_keys, d_query);
    return 0;
}

int ethos_route_topk(const void* q, const void* sub_keys_1, const void* sub_keys_2, const float* key_norms,
                     int64_t n_rows, int32_t d_query, int32_t n_sub_keys, int32_t top_k, int32_t k_cand, int32_t dtype,
                     void* out_scores, int32_t* out_ids, void* stream) {
    g_err[0] = 0;
    if (const int rc = route_checks("ethos_route_topk", n_rows, d_query, n_sub_keys, top_k, k_cand, dtype)) return rc;
    if (n_rows == 0) return 0;
    if (!q || !sub_keys_1 || !sub_keys_2 || !out_scores || !out_ids)
        return fail(ETHOS_ENULL, "ethos_route_topk: null pointer");
    if (!aligned16(q) || !aligned16(sub_keys_1) || !aligned16(sub_keys_2))
        return fail(ETHOS_EALIGN, "ethos_route_topk: q and sub-key tables must be 16-byte aligned");
    return hip_status(ethos::launch_route(q, sub_keys_1, sub_keys_2, key_norms, nullptr, n_rows, d_query, n_sub_keys,
                                          top_k, k_cand, dtype, out_scores, out_ids, (hipStream_t)stream),
                      "ethos_route_topk");
}

size_t ethos_route_keys_bytes(int32_t n_sub_keys, int32_t d_query, int32_t dtype) {
    if (!dtype_ok(dtype) || n_sub_keys <= 0 || d_query <= 0 || (d_query & 1) ||
        !ethos::route_supported(n_sub_keys, d_query / 2, dtype))
        return 0;
    return ethos::route_keys_bytes(n_sub_keys, d_query / 2, dtype);
}

int ethos_route_prepare_keys(const void* sub_keys_1, const void* sub_keys_2, int32_t n_sub_keys, int32_t d_query,
                             int32_t dtype, void* prepared, size_t prepared_bytes, void* stream) {
    g_err[0] = 0;
    if (!dtype_ok(dtype)) return fail(ETHOS_EDTYPE, "ethos_route_prepare_keys: unknown dtype %d", dtype);
    const size_t need = ethos_route_keys_bytes(n_sub_keys, d_query, dtype);
    if (need == 0)
        return fail(ETHOS_EUNSUPPORTED, "ethos_route_prepare_keys: unsupported sizes K=%d d_query=%d", n_sub_keys,
                    d_query);
    if (!sub_keys_1 || !sub_keys_2 || !prepared) return fail(ETHOS_ENULL, "ethos_route_prepare_keys: null pointer");
    if (prepared_bytes < need)
        return fail(ETHOS_ESIZE, "ethos_route_prepare_keys: prepared holds %zu bytes, needs %zu", prepared_bytes, need);
    if (!aligned16(prepared)) return fail(ETHOS_EALIGN, "ethos_route_prepare_keys: prepared must be 16-byte aligned");
    return hip_status(ethos::launch_route_prepare_keys(sub_keys_1, sub_keys_2, n_sub_keys, d_query, dtype, prepared,
                                                       (hipStream_t)stream),
                      "ethos_route_prepare_keys");
}

int ethos_route_topk_prepared(const void* q, const void* sub_keys_1, const void* sub_keys_2, const float* key_norms,
                              const void* prepared, size_t prepared_bytes, int64_t n_rows, int32_t d_query,
                              int32_t n_sub_keys, int32_t top_k, int32_t k_cand, int32_t dtype, void* out_scores,
                              int32_t* out_ids, void* stream) {
    g_err[0] = 0;
    if (const int rc = route_checks("ethos_route_topk_prepared", n_rows, d_query, n_sub_keys, top_k, k_cand, dtype))
        return rc;
    if (n_rows == 0) return 0;
    if (!q || !sub_keys_1 || !sub_keys_2 || !prepared || !out_scores || !out_ids)
        return fail(ETHOS_ENULL, "ethos_route_topk_prepared: null pointer");
    if (prepared_bytes < ethos::route_keys_bytes(n_sub_keys, d_query / 2, dtype))
        return fail(ETHOS_ESIZE, "ethos_route_topk_prepared: prepared holds %zu bytes, needs %zu", prepared_bytes,
                    ethos::route_keys_bytes(n_sub_keys, d_query / 2, dtype));
    if (!aligned16(q) || !aligned16(sub_keys_1) || !aligned16(sub_keys_2) || !aligned16(prepared))
        return fail(ETHOS_EALIGN, "ethos_route_topk_prepared: q, sub-key tables and prepared must be 16-byte aligned");
    return hip_status(ethos::launch_route(q, sub_keys_1, sub_keys_2, key_norms, prepared, n_rows, d_query, n_sub_keys,
                                          top_k, k_cand, dtype, out_scores, out_ids, (hipStream_t)stream),
                      "ethos_route_topk_prepared");
}

size_t ethos_sort_workspace_bytes(int64_t n_pairs, int64_t n_experts) {
    if (n_pairs <= 0 || n_experts <= 0) return 256;
    return ethos::sort_workspace_bytes(n_pairs, n_experts);
}

int ethos_sort_segment(const int32_t* ids, int64_t n_pairs, int64_t n_experts, void* workspace,
                       size_t workspace_bytes, int32_t* perm, int32_t* uniq_ids, int32_t* seg_off,
                       int32_t* pair_slot, int32_t* sorted_slot, int32_t* n_unique, void* stream) {
    g_err[0] = 0;
    if (n_pairs < 0 || n_experts <= 0 || n_experts > INT32_MAX || n_pairs > INT32_MAX)
        return fail(ETHOS_ESIZE, "ethos_sort_segment: bad sizes n_pairs=%lld n_experts=%lld", (long long)n_pairs,
                    (long long)n_experts);
    if (!seg_off || !n_unique) return fail(ETHOS_ENULL, "ethos_sort_segment: null pointer");
    if (n_pairs == 0)
        return hip_status(ethos::launch_sort_empty(seg_off, n_unique, (hipStream_t)stream), "ethos_sort_segment");
    if (!ids || !workspace || !perm || !uniq_ids || !pair_slot || !sorted_slot)
        return fail(ETHOS_ENULL, "ethos_sort_segment: null pointer");
    if (workspace_bytes < ethos::sort_workspace_bytes(n_pairs, n_experts))
        return fail(ETHOS_EWORKSPACE, "ethos_sort_segment: workspace of %zu bytes, %zu needed", workspace_bytes,
                    ethos::sort_workspace_bytes(n_pairs, n_experts));
    if (!aligned16(workspace)) return fail(ETHOS_EALIGN, "ethos_sort_segment: workspace not 16-byte aligned");
    return hip_status(ethos::launch_sort_segment(ids, n_pairs, n_experts, workspace, perm, uniq_ids, seg_off,
                                                 pair_slot, sorted_slot, n_unique, (hipStream_t)stream),
                      "ethos_sort_segment");
}

int ethos_sort_segment_token_proj(const int32_t* ids, int64_t n_pairs, int64_t n_experts, void* workspace,
                                  size_t workspace_bytes, int32_t* perm, int32_t* uniq_ids, int32_t* seg_off,
                                  int32_t* pair_slot, int32_t* sorted_slot, int32_t* n_unique, const void* x,
                                  const void* w2, const void* wut, int64_t n_tok, int32_t d_model, int32_t d_hidden,
                                  int32_t dtype, void* xp_out, void* stream) {
    g_err[0] = 0;
    if (!dtype_ok(dtype)) return fail(ETHOS_EDTYPE, "ethos_sort_segment_token_proj: unknown dtype %d", dtype);
    const int vec = dtype == ETHOS_BF16 ? 8 : 4;
    if (n_pairs < 0 || n_experts <= 0 || n_experts > INT32_MAX || n_pairs > INT32_MAX || n_tok < 0 ||
        n_tok > INT32_MAX || d_model <= 0 || d_hidden <= 0)
        return fail(ETHOS_ESIZE, "ethos_sort_segment_token_proj: bad sizes");
    if (d_model % vec || d_hidden % vec)
        return fail(ETHOS_EUNSUPPORTED, "ethos_sort_segment_token_proj: d_model and d_hidden must be multiples of %d",
                    vec);
    if (!seg_off || !n_unique) return fail(ETHOS_ENULL, "ethos_sort_segment_token_proj: null pointer");
    if (n_tok > 0 && (!x || !w2 || !xp_out)) return fail(ETHOS_ENULL, "ethos_sort_segment_token_proj: null pointer");
    if (n_tok > 0 && (!aligned16(x) || !aligned16(w2) || (wut && !aligned16(wut)) || !aligned16(xp_out)))
        return fail(ETHOS_EALIGN, "ethos_sort_segment_token_proj: x, w2, wut and xp_out must be 16-byte aligned");
    if (n_pairs > 0) {
        if (!ids || !perm || !uniq_ids || !pair_slot || !sorted_slot)
            return fail(ETHOS_ENULL, "ethos_sort_segment_token_proj: null pointer");
        if (n_tok > 0 && dtype == ETHOS_BF16) {
            const int rc = ethos::launch_sort_segment_tp(ids, n_pairs, n_experts, perm, uniq_ids, seg_off, pair_slot,
                                                         sorted_slot, n_unique, x, wut, n_tok, d_model, d_hidden,
                                                         xp_out, (hipStream_t)stream);
            if (rc >= 0) return hip_status(rc, "ethos_sort_segment_token_proj");
        }
    }
    // not one launch: the sort, then the projection
    int rc = ethos_sort_segment(ids, n_pairs, n_experts, workspace, workspace_bytes, perm, uniq_ids, seg_off, pair_slot,
                                sorted_slot, n_unique, stream);
    if (rc != 0) return rc;
    return ethos_token_proj(x, w2, wut, n_tok, d_model, d_hidden, dtype, xp_out, stream);
}

int ethos_sort_segment_noalloc(const int32_t* ids, int64_t n_pairs, int64_t n_experts, int32_t* perm,
                               int32_t* uniq_ids, int32_t* seg_off, int32_t* pair_slot, int32_t* sorted_slot,
                               int32_t* n_unique, void* stream) {
    g_err[0] = 0;
    if (n_pairs < 0 || n_experts <= 0 || n_experts > INT32_MAX)
        return fail(ETHOS_ESIZE, "ethos_sort_segment_noalloc: bad sizes n_pairs=%lld n_experts=%lld",
                    (long long)n_pairs, (long long)n_experts);
    if (n_pairs > ETHOS_NOALLOC_MAX_PAIRS)
        return fail(ETHOS_ESIZE,
                    "ethos_sort_segment_noalloc: %lld pairs exceed the %d its static workspace holds; use "
                    "ethos_sort_segment with a caller workspace", (long long)n_pairs, ETHOS_NOALLOC_MAX_PAIRS);
    if (!seg_off || !n_unique) return fail(ETHOS_ENULL, "ethos_sort_segment_noalloc: null pointer");
    if (n_pairs == 0)
        return hip_status(ethos::launch_sort_empty(seg_off, n_unique, (hipStream_t)stream),
                          "ethos_sort_segment_noalloc");
    if (!ids || !perm || !uniq_ids || !pair_slot || !sorted_slot)
        return fail(ETHOS_ENULL, "ethos_sort_segment_noalloc: null pointer");
    if (ethos::sort_workspace_bytes(n_pairs, n_experts) > sizeof(scratch))
        return fail(ETHOS_EWORKSPACE, "ethos_sort_segment_noalloc: static workspace sizing");
    int rc = 0;
    void* ws = scratch_ptr(&rc);
    if (!ws) return rc;
    return hip_status(ethos::launch_sort_segment(ids, n_pairs, n_experts, ws, perm, uniq_ids, seg_off, pair_slot,
                                                 sorted_slot, n_unique, (hipStream_t)stream),
                      "ethos_sort_segment_noalloc");
}

int ethos_generate(const void* latents, int64_t n_experts, const int32_t* uniq_ids, const int32_t* n_unique,
                   int64_t max_unique, const void* w1, const void* w2, int32_t d_latent, int32_t d_hidden,
                   int32_t d_model, int32_t dtype, void* h_out, void* v_out, void* stream) {
    g_err[0] = 0;
    if (!dtype_ok(dtype)) return fail(ETHOS_EDTYPE, "ethos_generate: unknown dtype %d", dtype);
    if (n_experts <= 0 || max_unique < 0 || d_latent <= 0 || d_hidden <= 0 || d_model <= 0)
        return fail(ETHOS_ESIZE, "ethos_generate: bad sizes");
    const int kq = dtype == ETHOS_BF16 ? 16 : 2;
    if (d_latent % kq || d_hidden % 32 || d_model % 32)
        return fail(ETHOS_EUNSUPPORTED,
                    "ethos_generate: needs d_latent %% %d == 0, d_hidden %% 32 == 0, d_model %% 32 == 0 "
                    "(got %d, %d, %d)", kq, d_latent, d_hidden, d_model);
    if (ethos::generate_smem_bytes(d_latent, d_hidden, dtype) > 160 * 1024)
        return fail(ETHOS_EUNSUPPORTED, "ethos_generate: d_latent + d_hidden too large for LDS");
    if (max_unique == 0) return 0;
    // v_out == NULL: hidden rows only (w2 is then not read)
    if (!latents || !uniq_ids || !n_unique || !w1 || !h_out || (v_out && !w2))
        return fail(ETHOS_ENULL, "ethos_generate: null pointer");
    if (dtype == ETHOS_BF16 &&
        (!aligned16(w1) || (v_out && !aligned16(w2)) || !aligned16(h_out) || (v_out && !aligned16(v_out))))
        return fail(ETHOS_EALIGN, "ethos_generate: weights and outputs must be 16-byte aligned");
    return hip_status(ethos::launch_generate(latents, n_experts, uniq_ids, n_unique, max_unique, w1, w2, d_latent,
                                             d_hidden, d_model, dtype, h_out, v_out, num_cus(), (hipStream_t)stream),
                      "ethos_generate");
}

size_t ethos_apply_workspace_bytes(int64_t n_tok, int32_t n_heads, int32_t top_k, int32_t d_hidden, int32_t dtype) {
    if (n_tok <= 0 || n_heads <= 0 || top_k <= 0 || d_hidden <= 0) return 256;
    return ethos::apply_workspace_bytes(n_tok, n_heads, top_k, d_hidden, dtype);
}

int ethos_apply_scatter(const void* x, const void* w2, const void* h, const void* v, const int32_t* perm,
                        const int32_t* sorted_slot, const int32_t* pair_slot, const void* scores, int64_t n_tok,
                        int32_t n_heads, int32_t top_k, int32_t d_model, int32_t d_hidden, int32_t dtype,
                        void* workspace, size_t workspace_bytes, void* out, void* stream) {
    g_err[0] = 0;
    if (!dtype_ok(dtype)) return fail(ETHOS_EDTYPE, "ethos_apply_scatter: unknown dtype %d", dtype);
    if (n_tok < 0 || n_heads <= 0 || top_k <= 0 || d_model <= 0 || d_hidden <= 0)
        return fail(ETHOS_ESIZE, "ethos_apply_scatter: bad sizes");
    const int vec = dtype == ETHOS_BF16 ? 8 : 4;
    if (d_model % vec || d_hidden % vec || ethos::apply_chunks(d_model, dtype) > 8 ||
        ethos::apply_chunks(d_hidden, dtype) > 8)
        return fail(ETHOS_EUNSUPPORTED,
                    "ethos_apply_scatter: d_model=%d and d_hidden=%d must be multiples of %d and <= %d", d_model,
                    d_hidden, vec, 8 * 64 * vec);
    if (n_tok * n_heads * top_k > INT32_MAX || n_tok > INT32_MAX)
        return fail(ETHOS_ESIZE, "ethos_apply_scatter: too many pairs");
    if (n_tok == 0) return 0;
    if (!x || !w2 || !h || !v || !perm || !sorted_slot || !pair_slot || !scores || !workspace || !out)
        return fail(ETHOS_ENULL, "ethos_apply_scatter: null pointer");
    const size_t need = ethos::apply_workspace_bytes(n_tok, n_heads, top_k, d_hidden, dtype);
    if (workspace_bytes < need)
        return fail(ETHOS_EWORKSPACE, "ethos_apply_scatter: workspace of %zu bytes, %zu needed", workspace_bytes,
                    need);
    if (!aligned16(x) || !aligned16(w2) || !aligned16(h) || !aligned16(v) || !aligned16(workspace) ||
        !aligned16(out))
        return fail(ETHOS_EALIGN, "ethos_apply_scatter: x, w2, h, v, workspace and out must be 16-byte aligned");
    return hip_status(ethos::launch_apply(x, w2, h, v, perm, sorted_slot, pair_slot, scores, n_tok, n_heads, top_k,
                                          d_model, d_hidden, dtype, workspace, out, num_cus(), (hipStream_t)stream),
                      "ethos_apply_scatter");
}

size_t ethos_apply_hidden_workspace_bytes(int64_t n_tok, int32_t n_heads, int32_t top_k, int32_t d_model,
                                          int32_t d_hidden, int32_t dtype) {
    if (n_tok <= 0 || n_heads <= 0 || top_k <= 0 || d_model <= 0 || d_hidden <= 0) return 256;
    return ethos::apply_hidden_workspace_bytes(n_tok, n_heads, top_k, d_model, d_hidden, dtype);
}

int ethos_apply_hidden(const void* x, const void* w2, const void* h, const int32_t* perm, const int32_t* sorted_slot,
                       const int32_t* pair_slot, const void* scores, int64_t n_tok, int32_t n_heads, int32_t top_k,
                       int32_t d_model, int32_t d_hidden, int32_t dtype, void* workspace, size_t workspace_bytes,
                       void* out, void* stream) {
    g_err[0] = 0;
    if (!dtype_ok(dtype)) return fail(ETHOS_EDTYPE, "ethos_apply_hidden: unknown dtype %d", dtype);
    if (n_tok < 0 || n_heads <= 0 || top_k <= 0 || d_model <= 0 || d_hidden <= 0)
        return fail(ETHOS_ESIZE, "ethos_apply_hidden: bad sizes");
    const int vec = dtype == ETHOS_BF16 ? 8 : 4;
    if (d_model % vec || d_hidden % vec || d_model > 4096 || ethos::apply_chunks(d_hidden, dtype) > 8)
        return fail(ETHOS_EUNSUPPORTED,
                    "ethos_apply_hidden: d_model=%d and d_hidden=%d must be multiples of %d, d_model <= 4096, "
                    "d_hidden <= %d", d_model, d_hidden, vec, 8 * 64 * vec);
    if (n_tok * n_heads * top_k > INT32_MAX || n_tok > INT32_MAX)
        return fail(ETHOS_ESIZE, "ethos_apply_hidden: too many pairs");
    if (n_tok == 0) return 0;
    if (!x || !w2 || !h || !perm || !sorted_slot || !pair_slot || !scores || !workspace || !out)
        return fail(ETHOS_ENULL, "ethos_apply_hidden: null pointer");
    const size_t need = ethos::apply_hidden_workspace_bytes(n_tok, n_heads, top_k, d_model, d_hidden, dtype);
    if (workspace_bytes < need)
        return fail(ETHOS_EWORKSPACE, "ethos_apply_hidden: workspace of %zu bytes, %zu needed", workspace_bytes,
                    need);
    if (!aligned16(x) || !aligned16(w2) || !aligned16(h) || !aligned16(workspace) || !aligned16(out))
        return fail(ETHOS_EALIGN, "ethos_apply_hidden: x, w2, h, workspace and out must be 16-byte aligned");
    const int rc = ethos::launch_apply_hidden(x, w2, h, perm, sorted_slot, pair_slot, scores, n_tok, n_heads, top_k,
                                              d_model, d_hidden, dtype, workspace, out, num_cus(), (hipStream_t)stream);
    if (rc < 0) return fail(ETHOS_EUNSUPPORTED, "ethos_apply_hidden: d_hidden=%d not supported", d_hidden);
    return hip_status(rc, "ethos_apply_hidden");
}

size_t ethos_expert_forward_workspace_bytes(int64_t n_tok, int32_t n_heads, int32_t top_k, int64_t max_unique,
                                            int32_t d_model, int32_t d_hidden, int32_t dtype, int32_t order) {
    if (n_tok <= 0 || n_heads <= 0 || top_k <= 0 || max_unique < 0 || d_model <= 0 || d_hidden <= 0 ||
        (order != 0 && order != 1))
        return 256;
    return ethos::expert_forward_workspace_bytes(n_tok, n_heads, top_k, max_unique, d_model, d_hidden, dtype, order);
}

int ethos_token_proj(const void* x, const void* w2, const void* wut, int64_t n_tok, int32_t d_model,
                     int32_t d_hidden, int32_t dtype, void* xp_out, void* stream) {
    g_err[0] = 0;
    if (!dtype_ok(dtype)) return fail(ETHOS_EDTYPE, "ethos_token_proj: unknown dtype %d", dtype);
    const int vec = dtype == ETHOS_BF16 ? 8 : 4;
    if (n_tok < 0 || d_model <= 0 || d_hidden <= 0 || n_tok > INT32_MAX)
        return fail(ETHOS_ESIZE, "ethos_token_proj: bad sizes");
    if (d_model % vec || d_hidden % vec)
        return fail(ETHOS_EUNSUPPORTED, "ethos_token_proj: d_model and d_hidden must be multiples of %d", vec);
    if (n_tok == 0) return 0;
    if (!x || !w2 || !xp_out) return fail(ETHOS_ENULL, "ethos_token_proj: null pointer");
    if (!aligned16(x) || !aligned16(w2) || (wut && !aligned16(wut)) || !aligned16(xp_out))
        return fail(ETHOS_EALIGN, "ethos_token_proj: x, w2, wut and xp_out must be 16-byte aligned");
    const int rc = ethos::launch_token_proj_out(x, w2, dtype == ETHOS_BF16 ? wut : nullptr, n_tok, d_model, d_hidden,
                                                dtype, xp_out, (hipStream_t)stream);
    if (rc < 0) return fail(ETHOS_ENULL, "ethos_token_proj: bf16 needs wut (W_u^T)");
    return hip_status(rc, "ethos_token_proj");
}

int ethos_expert_forward(const void* x, const void* latents, int64_t n_experts, const void* w1, const void* w2,
                         const void* wut, const void* xp, const int32_t* uniq_ids, const int32_t* seg_off,
                         const int32_t* n_unique, int64_t max_unique,
                         const int32_t* perm, const int32_t* sorted_slot, const int32_t* pair_slot, const void* scores,
                         int64_t n_tok, int32_t n_heads, int32_t top_k, int32_t d_latent, int32_t d_hidden,
                         int32_t d_model, int32_t dtype, int32_t order, void* workspace, size_t workspace_bytes,
                         void* h_out, void* out, void* stream) {
    g_err[0] = 0;
    if (!dtype_ok(dtype)) return fail(ETHOS_EDTYPE, "ethos_expert_forward: unknown dtype %d", dtype);
    if (order != 0 && order != 1) return fail(ETHOS_ESIZE, "ethos_expert_forward: order must be 0 or 1, got %d", order);
    if (n_tok < 0 || n_heads <= 0 || top_k <= 0 || n_experts <= 0 || max_unique < 0 || d_latent <= 0 ||
        d_hidden <= 0 || d_model <= 0)
        return fail(ETHOS_ESIZE, "ethos_expert_forward: bad sizes");
    if (n_tok * n_heads * top_k > INT32_MAX || n_tok > INT32_MAX)
        return fail(ETHOS_ESIZE, "ethos_expert_forward: too many pairs");
    const int kq = dtype == ETHOS_BF16 ? 16 : 2;
    const int vec = dtype == ETHOS_BF16 ? 8 : 4;
    if (d_latent % kq || d_hidden % 32 || d_model % 32 || d_model > 4096 ||
        ethos::apply_chunks(d_model, dtype) > 8 || ethos::apply_chunks(d_hidden, dtype) > 8 ||
        ethos::generate_smem_bytes(d_latent, d_hidden, dtype) > 160 * 1024 || d_model % vec || d_hidden % vec)
        return fail(ETHOS_EUNSUPPORTED,
                    "ethos_expert_forward: needs d_latent %% %d == 0, d_hidden and d_model multiples of 32 with "
                    "d_model <= 4096 and d_hidden <= %d (got %d, %d, %d)", kq, 8 * 64 * vec, d_latent, d_hidden,
                    d_model);
    if (n_tok == 0) return 0;
    if (max_unique < 1) return fail(ETHOS_ESIZE, "ethos_expert_forward: max_unique must be >= 1 for a nonempty batch");
    if (!x || !latents || !w1 || !w2 || !uniq_ids || !seg_off || !n_unique || !perm || !sorted_slot || !pair_slot ||
        !scores || !workspace || !h_out || !out)
        return fail(ETHOS_ENULL, "ethos_expert_forward: null pointer");
    const size_t need = ethos::expert_forward_workspace_bytes(n_tok, n_heads, top_k, max_unique, d_model, d_hidden,
                                                              dtype, order);
    if (workspace_bytes < need)
        return fail(ETHOS_EWORKSPACE, "ethos_expert_forward: workspace of %zu bytes, %zu needed", workspace_bytes,
                    need);
    if (!aligned16(x) || !aligned16(w1) || !aligned16(w2) || (wut && !aligned16(wut)) || (xp && !aligned16(xp)) ||
        !aligned16(workspace) || !aligned16(h_out) || !aligned16(out))
        return fail(ETHOS_EALIGN, "ethos_expert_forward: x, w1, w2, wut, xp, workspace, h_out and out must be "
                                  "16-byte aligned");
    const int rc = ethos::launch_expert_forward(x, latents, n_experts, w1, w2, dtype == ETHOS_BF16 ? wut : nullptr,
                                                xp, uniq_ids, seg_off, n_unique, max_unique, perm, sorted_slot,
                                                pair_slot, scores,
                                                n_tok, n_heads, top_k, d_latent, d_hidden, d_model, dtype, order,
                                                workspace, h_out, out, num_cus(), (hipStream_t)stream);
    if (rc < 0) return fail(ETHOS_EUNSUPPORTED, "ethos_expert_forward: shape not supported");
    return hip_status(rc, "ethos_expert_forward");
}

size_t ethos_expert_backward_workspace_bytes(int64_t n_tok, int32_t n_heads, int32_t top_k, int32_t d_hidden) {
    if (n_tok < 0 || n_heads <= 0 || top_k <= 0 || d_hidden <= 0) return 0;
    return ethos::expert_backward_workspace_bytes(n_tok * n_heads * top_k, d_hidden);
}

int ethos_expert_backward(const void* h, const float* xp, const float* dyb, const int32_t* pair_slot,
                          const int32_t* perm, const int32_t* sorted_slot, const int32_t* seg_off, const void* scores,
                          int64_t n_tok, int32_t n_heads, int32_t top_k, int32_t d_hidden, int32_t dtype,
                          void* workspace, size_t workspace_bytes, float* dscores, float* hacc, float* dxp, float* dh,
                          void* stream) {
    g_err[0] = 0;
    if (!dtype_ok(dtype)) return fail(ETHOS_EDTYPE, "ethos_expert_backward: unknown dtype %d", dtype);
    if (n_tok < 0 || n_heads <= 0 || top_k <= 0 || d_hidden <= 0)
        return fail(ETHOS_ESIZE, "ethos_expert_backward: bad sizes");
    const int vec = dtype == ETHOS_BF16 ? 8 : 4;
    if (d_hidden % vec || ethos::apply_chunks(d_hidden, dtype) > 8)
        return fail(ETHOS_EUNSUPPORTED, "ethos_expert_backward: d_hidden=%d must be a multiple of %d and <= %d",
                    d_hidden, vec, 8 * 64 * vec);
    if (n_tok * n_heads * top_k > INT32_MAX || n_tok > INT32_MAX)
        return fail(ETHOS_ESIZE, "ethos_expert_backward: too many pairs");
    if (n_tok == 0) return 0;
    if (!h || !xp || !dyb || !pair_slot || !perm || !sorted_slot || !seg_off || !scores || !workspace || !dscores ||
        !hacc || !dxp || !dh)
        return fail(ETHOS_ENULL, "ethos_expert_backward: null pointer");
    const size_t need = ethos::expert_backward_workspace_bytes(n_tok * n_heads * top_k, d_hidden);
    if (workspace_bytes < need)
        return fail(ETHOS_EWORKSPACE, "ethos_expert_backward: workspace of %zu bytes, %zu needed", workspace_bytes,
                    need);
    if (!aligned16(h) || !aligned16(workspace))
        return fail(ETHOS_EALIGN, "ethos_expert_backward: h and workspace must be 16-byte aligned");
    const int rc = ethos::launch_expert_backward(h, xp, dyb, pair_slot, perm, sorted_slot, seg_off, scores, n_tok,
                                                 n_heads, top_k, d_hidden, dtype, workspace, dscores, hacc, dxp, dh,
                                                 num_cus(), (hipStream_t)stream);
    if (rc < 0) return fail(ETHOS_EUNSUPPORTED, "ethos_expert_backward: d_hidden=%d not supported", d_hidden);
    return hip_status(rc, "ethos_expert_backward");
}

}  // extern "C"
