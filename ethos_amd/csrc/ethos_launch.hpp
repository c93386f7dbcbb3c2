// Internal launch functions of the ETHOS expert-layer kernels (C++ linkage; the
// public C-ABI lives in abi.hip / include/ethos_hip.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace ethos {

// Records the calling thread's next stage event (ethos_stage_events) on `stream`, if any.
void stage_mark(hipStream_t stream);

size_t qproj_workspace_bytes(int64_t n_tok, int ncols, int d, int dtype);
size_t qproj_weights_bytes(int ncols, int d, int dtype);
int launch_qproj_prepare(const void* w, int ncols, int d, int dtype, void* prepared, hipStream_t stream);
int launch_qproj(const void* x, const void* w, const void* prepared, const void* b, const float* alpha,
                 const float* beta, int64_t n_tok, int d, int ncols, int dtype, void* ws, void* q, int num_cus,
                 hipStream_t stream);

size_t route_smem_bytes(int K, int dh2, int elem_bytes);
bool route_supported(int K, int dh2, int dtype);
int launch_route(const void* q, const void* k1, const void* k2, const float* key_norms, const void* kfrag,
                 int64_t rows, int dq, int K, int top_k, int kc, int dtype, void* gates, int32_t* ids,
                 hipStream_t stream);
size_t route_keys_bytes(int K, int dh2, int dtype);
int launch_route_prepare_keys(const void* k1, const void* k2, int K, int dq, int dtype, void* out, hipStream_t stream);

// The sort's workspace: keys and values twice (4 n words), then per (digit, tile of
// kSortTileKeys keys) four counters (rows of sort_tile_pitch words: the tile count rounded
// up to a multiple of 8), two per-digit totals, and, for batches of more than
// kSortTableMinPairs pairs with ids of at most 18 bits (two 9-bit passes), an expert ->
// slot table of 2^(9 passes) words.
constexpr int kSortTileKeys = 4096;
__host__ __device__ constexpr int sort_tile_pitch(int n_tiles) { return (n_tiles + 7) / 8 * 8; }
constexpr int64_t kSortTableMinPairs = (int64_t)1 << 20;
constexpr int sort_key_bits(int64_t n_experts) {
    int b = 0;
    while (b < 32 && ((int64_t)1 << b) < n_experts) ++b;
    return b;
}
constexpr int sort_passes(int64_t n_experts) {
    const int bits = sort_key_bits(n_experts);
    return bits <= 9 ? 1 : (bits + 8) / 9;
}
constexpr size_t sort_table_words(int64_t n, int64_t n_experts) {
    return n > kSortTableMinPairs && sort_passes(n_experts) <= 2 ? (size_t)1 << (9 * sort_passes(n_experts)) : 0;
}
constexpr size_t sort_workspace_words(int64_t n, int64_t n_experts) {
    return (size_t)4 * (size_t)n + (size_t)4 * 512 * (size_t)sort_tile_pitch((int)((n + kSortTileKeys - 1) / kSortTileKeys)) +
           2 * 512 + 64 + sort_table_words(n, n_experts);
}
size_t sort_workspace_bytes(int64_t n, int64_t n_experts);
int launch_sort_segment(const int32_t* ids, int64_t n, int64_t n_experts, void* ws, int32_t* perm, int32_t* uniq,
                        int32_t* seg_off, int32_t* pair_slot, int32_t* sorted_slot, int32_t* n_unique,
                        hipStream_t stream);
int launch_sort_empty(int32_t* seg_off, int32_t* n_unique, hipStream_t stream);
// The sort with the bf16 token projection xp = RN(x W_u) (W_u^T given) in the same launch,
// for batches the single-workgroup sort takes; -1 (nothing launched) otherwise.
int launch_sort_segment_tp(const int32_t* ids, int64_t n, int64_t n_experts, int32_t* perm, int32_t* uniq,
                           int32_t* seg_off, int32_t* pair_slot, int32_t* sorted_slot, int32_t* n_unique,
                           const void* x, const void* wut, int64_t n_tok, int d, int dh, void* xp,
                           hipStream_t stream);

size_t generate_smem_bytes(int dl, int dh, int dtype);
int launch_generate(const void* latents, int64_t n_experts, const int32_t* uniq, const int32_t* n_unique,
                    int64_t max_unique, const void* w1, const void* w2, int dl, int dh, int d, int dtype, void* hout,
                    void* vout, int num_cus, hipStream_t stream);

// The bf16 generator's two kernels one at a time (part 1: hidden rows, part 2: v rows from
// them), for shapes where generate_split_supported; -1 when not supported.
bool generate_split_supported(int64_t n_experts, int64_t max_unique, int dl, int dh, int d, int dtype, int num_cus);
int launch_generate_part(const void* latents, int64_t n_experts, const int32_t* uniq, const int32_t* n_unique,
                         int64_t max_unique, const void* w1, const void* w2, int dl, int dh, int d, void* hout,
                         void* vout, int part, int num_cus, hipStream_t stream);

// The bf16 hidden rows (part 1) with the activations of their pairs computed in the same
// kernel for tiles of at most kActFusedCap pairs (act[p] for those pairs; the rest are left
// for the activation kernel with seg_off); -1 when not supported.
int launch_hidden_act(const void* latents, int64_t n_experts, const int32_t* uniq, const int32_t* n_unique,
                      int64_t max_unique, const void* w1, int dl, int dh, void* hout, const void* xp,
                      const int32_t* perm, const int32_t* sorted_slot, const int32_t* seg_off, const void* gates, int hk,
                      float* act, int64_t n_pairs, int num_cus, hipStream_t stream);

int apply_chunks(int d, int dtype);
// The expert stages' backward (per-pair scalars, token sums, then deterministic expert
// sums over the sorted pairs); ws: expert_backward_workspace_bytes.
size_t expert_backward_workspace_bytes(int64_t n_pairs, int dh);
int launch_expert_backward(const void* hid, const float* xp, const float* dyb, const int32_t* pair_slot,
                           const int32_t* perm, const int32_t* sorted_slot, const int32_t* seg_off, const void* gates,
                           int64_t n_tok, int H, int k, int dh, int dtype, void* ws, float* dg, float* hacc,
                           float* dxp, float* dhs, int num_cus, hipStream_t stream);
size_t apply_hidden_workspace_bytes(int64_t n_tok, int H, int k, int d, int dh, int dtype);
int launch_apply_hidden(const void* x, const void* w2, const void* hid, const int32_t* perm,
                        const int32_t* sorted_slot, const int32_t* pair_slot, const void* gates, int64_t n_tok, int H,
                        int k, int d, int dh, int dtype, void* ws, void* out, int num_cus, hipStream_t stream);
size_t apply_workspace_bytes(int64_t n_tok, int H, int k, int dh, int dtype);
int launch_apply(const void* x, const void* w2, const void* hid, const void* v, const int32_t* perm,
                 const int32_t* sorted_slot, const int32_t* pair_slot, const void* gates, int64_t n_tok, int H, int k,
                 int d, int dh, int dtype, void* ws, void* out, int num_cus, hipStream_t stream);
size_t expert_forward_workspace_bytes(int64_t n_tok, int H, int k, int64_t max_unique, int d, int dh, int dtype,
                                      int order);
// xp = RN_T(x W_u) into xp [n_tok, dh]; bf16 MFMA shapes need wut (-1 without it).
int launch_token_proj_out(const void* x, const void* w2, const void* wut, int64_t n_tok, int d, int dh, int dtype,
                          void* xp, hipStream_t stream);
int launch_expert_forward(const void* x, const void* latents, int64_t n_experts, const void* w1, const void* w2,
                          const void* wut, const void* xp_in, const int32_t* uniq, const int32_t* seg_off,
                          const int32_t* n_unique, int64_t max_unique,
                          const int32_t* perm, const int32_t* sorted_slot, const int32_t* pair_slot,
                          const void* gates, int64_t n_tok, int H, int k, int dl, int dh, int d, int dtype, int order,
                          void* ws, void* hout, void* out, int num_cus, hipStream_t stream);

}  // namespace ethos
