/*
 * ethos_hip.h -- C-ABI of the MI355X (gfx950) ETHOS expert-layer forward path.
 *
 * The reference (wrmedford/ETHOS) implements the path as a PyTorch nn.Module
 * (SimplifiedHypernetMoE, model.py:267-343) and a Triton launch per routing head
 * (FusedLowRankMoE_Reordered.forward, kernels.py:145-221; launch site
 * kernels.py:179-215).  This library replaces the work below those modules with
 * four stages, each an entry point here:
 *
 *   ethos_query_proj     per-head query projection + eval BatchNorm
 *   ethos_route_topk     sub-key scoring, top-k_cand per half, combination, top-k, softmax
 *                        (ethos_route_topk_prepared: with the sub-keys' prepared form)
 *   ethos_sort_segment   reordering of (token, head, k) pairs by expert id
 *   ethos_sort_segment_token_proj  the same with the token projection x W_u beside it
 *   ethos_generate       hypernetwork expert generation over the unique experts
 *   ethos_apply_scatter  per-pair activation and weighted scatter-back into tokens
 *   ethos_apply_hidden   the same, by hidden-space reordering (no v rows)
 *   ethos_expert_forward generation + apply + scatter-back in one call (either order)
 *   ethos_expert_backward  per-pair part of the expert stages' backward
 *
 * Conventions (every entry point):
 *   - All pointers are device pointers owned by the caller; nothing is allocated.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the default stream) and the
 *     call returns without synchronising.
 *   - Return 0 on success, a negative ETHOS_E* code for an argument error (nothing is
 *     enqueued), or a positive hipError_t from the launch.  ethos_last_error() gives a
 *     message for the calling thread's last failure.
 *   - dtype: ETHOS_F32 or ETHOS_BF16; tensors of "dtype T" hold that type, row-major.
 *   - Every entry point is deterministic: the same inputs give bit-identical outputs on
 *     every run (no atomics; every sum has a fixed order).
 */
#ifndef ETHOS_HIP_H
#define ETHOS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ETHOS_ABI_VERSION 8

#define ETHOS_F32 0
#define ETHOS_BF16 1

#define ETHOS_EDTYPE (-1)       /* unknown dtype code */
#define ETHOS_ESIZE (-2)        /* sizes out of range / inconsistent */
#define ETHOS_ENULL (-3)        /* a required pointer is NULL */
#define ETHOS_EALIGN (-4)       /* a pointer is not 16-byte aligned */
#define ETHOS_EWORKSPACE (-5)   /* workspace too small */
#define ETHOS_EUNSUPPORTED (-6) /* valid for the reference, outside this build's limits */

/*
 * Instrumentation, no counterpart in the reference: hand the calling thread a list of
 * n_events (<= 16) HIP events (hipEvent_t).  Later calls on this thread record them, in
 * order, on their stream at stage boundaries, until the list is used up; n_events = 0
 * clears it.  ethos_expert_forward records five per call: after the token projection, the
 * hidden rows, the activations, the v rows and the scatter-back.  Lets a caller time the
 * stages inside one call with events on the launch stream.  The library keeps the raw
 * handles: the events must stay valid until the list is used up or cleared with
 * n_events = 0 (a caller whose call fails part-way should clear it before freeing them).
 */
int ethos_stage_events(void* const* events, int32_t n_events);

/* Message for the calling thread's last failed call ("" after a success). */
const char* ethos_last_error(void);

/* ETHOS_ABI_VERSION of the loaded library. */
int ethos_abi_version(void);

/*
 * Query projection + eval-mode Query BatchNorm for all heads.
 * Replaces query_projs[h](x_flat) then query_norms[h](.) (model.py:215-216; modules
 * built at model.py:195-202).
 *   x        [n_tok, d_model]            dtype T
 *   wq       [n_heads, d_query, d_model] dtype T  (query_projs[h].weight stacked)
 *   bq       [n_heads, d_query]          dtype T  (query_projs[h].bias stacked)
 *   bn_alpha [n_heads, d_query] fp32  weight / sqrt(running_var + eps)
 *   bn_beta  [n_heads, d_query] fp32  bias - running_mean * bn_alpha
 *   workspace                        >= ethos_query_proj_workspace_bytes(...) bytes, 16-byte
 *                                    aligned (bf16 uses it; fp32 may pass NULL / 0)
 *   q_out    [n_tok, n_heads, d_query]   dtype T
 * q = RN_T(fmaf(RN_T(x . wq[h,o] + bq[h,o]), alpha, beta)); the dot product is the
 * correctly rounded one for bf16 (certified MFMA accumulation, exact fp64 recomputation of
 * the elements the certificate cannot settle) and an fp64 chain in index order for fp32.
 */
size_t ethos_query_proj_workspace_bytes(int64_t n_tok, int32_t d_model, int32_t n_heads, int32_t d_query,
                                        int32_t dtype);

int ethos_query_proj(const void* x, const void* wq, const void* bq, const float* bn_alpha, const float* bn_beta,
                     int64_t n_tok, int32_t d_model, int32_t n_heads, int32_t d_query, int32_t dtype, void* workspace,
                     size_t workspace_bytes, void* q_out, void* stream);

/*
 * The same projection with the weight-dependent part computed once.  The reference
 * re-reads query_projs[h].weight on every call (model.py:215); these split that work off
 * for callers that keep the weights between calls (the module does, per parameter version).
 *   ethos_query_proj_weights_bytes: size of the prepared form of wq (0 for fp32: nothing to
 *     prepare, and ethos_query_proj_prepared then equals ethos_query_proj).
 *   ethos_query_proj_prepare: writes the prepared form of wq (for bf16: its int8 digit
 *     planes and per-row formats) into `prepared` (>= that many bytes, 16-byte aligned).
 *   ethos_query_proj_prepared: ethos_query_proj with `prepared` (prepared_bytes long) from
 *     the same wq; bit-identical results.  wq is still read (for the exact recomputation of
 *     uncertain elements).
 */
size_t ethos_query_proj_weights_bytes(int32_t d_model, int32_t n_heads, int32_t d_query, int32_t dtype);

int ethos_query_proj_prepare(const void* wq, int32_t d_model, int32_t n_heads, int32_t d_query, int32_t dtype,
                             void* prepared, size_t prepared_bytes, void* stream);

int ethos_query_proj_prepared(const void* x, const void* wq, const void* prepared, size_t prepared_bytes,
                              const void* bq, const float* bn_alpha, const float* bn_beta, int64_t n_tok, int32_t d_model,
                              int32_t n_heads, int32_t d_query, int32_t dtype, void* workspace,
                              size_t workspace_bytes, void* q_out, void* stream);

/*
 * Product-key routing of n_rows independent query rows (row = token * n_heads + head).
 * Replaces the body of ProductKeyRouter.forward (model.py:217-245) and the head
 * stacking (model.py:250-252).
 *   q          [n_rows, d_query]        dtype T
 *   sub_keys_1 [n_sub_keys, d_query/2]  dtype T  (router.sub_keys_1.weight)
 *   sub_keys_2 [n_sub_keys, d_query/2]  dtype T  (router.sub_keys_2.weight)
 *   key_norms  [2, n_sub_keys] fp32 or NULL: upper bounds of the Euclidean norms of the
 *              rows of sub_keys_1 then sub_keys_2 (they size the error bound of the
 *              MFMA pre-filter; NULL = computed by the kernel, slower)
 *   out_scores [n_rows, top_k]          dtype T  softmax gates (fp32 softmax cast to T)
 *   out_ids    [n_rows, top_k]          int32    expert ids = i1 * n_sub_keys + i2
 * k_cand is the per-half candidate count (the reference uses 2 * top_k, model.py:224).
 * Sub-key scores are the correctly rounded (bf16) / fp64-accumulated (fp32) dot products.
 * Order: score descending, ties to the lowest index (sub-key index per half, expert id
 * for the final list).  Limits: k_cand, top_k <= 32; n_sub_keys <= 512;
 * d_query / 2 <= 256 and a multiple of 16 (bf16) or 4 (fp32); q, sub-keys 16-byte aligned.
 */
int ethos_route_topk(const void* q, const void* sub_keys_1, const void* sub_keys_2, const float* key_norms,
                     int64_t n_rows, int32_t d_query, int32_t n_sub_keys, int32_t top_k, int32_t k_cand, int32_t dtype,
                     void* out_scores, int32_t* out_ids, void* stream);

/*
 * The same routing with the sub-keys' layout for the scoring MFMAs computed once.  The
 * reference reads router.sub_keys_{1,2}.weight on every call (model.py:219-220); these
 * split the reordering off for callers that keep the tables between calls (the module
 * does, per parameter version).
 *   ethos_route_keys_bytes: size of the prepared form (0 for unsupported sizes).
 *   ethos_route_prepare_keys: writes both tables in fragment order (for each block of 32
 *     keys and each MFMA reduction step, the 64 lanes' operand pieces back to back) into
 *     `prepared` (>= that many bytes, 16-byte aligned).
 *   ethos_route_topk_prepared: ethos_route_topk with `prepared` from the same tables;
 *     bit-identical results.  The tables themselves are still read (exact rescoring).
 */
size_t ethos_route_keys_bytes(int32_t n_sub_keys, int32_t d_query, int32_t dtype);

int ethos_route_prepare_keys(const void* sub_keys_1, const void* sub_keys_2, int32_t n_sub_keys, int32_t d_query,
                             int32_t dtype, void* prepared, size_t prepared_bytes, void* stream);

int ethos_route_topk_prepared(const void* q, const void* sub_keys_1, const void* sub_keys_2, const float* key_norms,
                              const void* prepared, size_t prepared_bytes, int64_t n_rows, int32_t d_query,
                              int32_t n_sub_keys, int32_t top_k, int32_t k_cand, int32_t dtype, void* out_scores,
                              int32_t* out_ids, void* stream);

/* Workspace size for ethos_sort_segment. */
size_t ethos_sort_workspace_bytes(int64_t n_pairs, int64_t n_experts);

/*
 * Reordering of pairs by expert id (stable LSD radix sort + segmentation).
 * No reference code: the reference visits pairs in token order (model.py:306-334;
 * kernels.py:167-215); the paper's Algorithm 1 reorders by expert (paper p.10).
 *   ids         [n_pairs] int32 expert id of pair p (out_ids flattened), < n_experts
 *   workspace   >= ethos_sort_workspace_bytes(n_pairs, n_experts) bytes, 16-byte aligned
 *   perm        [n_pairs] int32   pair ids ordered by (expert id, pair id)
 *   uniq_ids    [min(n_pairs, n_experts)] int32  expert id of each unique slot, ascending
 *   seg_off     [min(n_pairs, n_experts) + 1] int32  pairs of slot u are perm[seg_off[u]..seg_off[u+1])
 *   pair_slot   [n_pairs] int32   slot of pair p
 *   sorted_slot [n_pairs] int32   slot of sorted position i
 *   n_unique    [1] int32         number of unique experts U (written on the device)
 */
int ethos_sort_segment(const int32_t* ids, int64_t n_pairs, int64_t n_experts, void* workspace,
                       size_t workspace_bytes, int32_t* perm, int32_t* uniq_ids, int32_t* seg_off,
                       int32_t* pair_slot, int32_t* sorted_slot, int32_t* n_unique, void* stream);

/*
 * ethos_sort_segment and ethos_token_proj in one call: the reordering of the pairs and the
 * token projection x_proj = RN_T(x W_u) are independent (the projection needs only x).  For
 * bf16 batches the single-workgroup sort takes (n_pairs <= 16384) with W_u^T given, both run
 * in one launch, the projection's tiles in the workgroups beside the sort's one; otherwise it
 * is the two calls in turn.  No counterpart in the reference (its pair loop forms x_proj per
 * pair, model.py:326); for callers of ethos_expert_forward that pass xp.  Arguments and
 * outputs are those of ethos_sort_segment (ids .. n_unique) and ethos_token_proj (x .. xp_out);
 * the outputs are bit-identical to theirs.  The workspace is needed only when the two run in
 * turn; it may be NULL for a single launch.
 */
int ethos_sort_segment_token_proj(const int32_t* ids, int64_t n_pairs, int64_t n_experts, void* workspace,
                                  size_t workspace_bytes, int32_t* perm, int32_t* uniq_ids, int32_t* seg_off,
                                  int32_t* pair_slot, int32_t* sorted_slot, int32_t* n_unique, const void* x,
                                  const void* w2, const void* wut, int64_t n_tok, int32_t d_model, int32_t d_hidden,
                                  int32_t dtype, void* xp_out, void* stream);

/*
 * ethos_sort_segment without a caller workspace, for callers that cannot allocate device
 * memory (code under HIP graph capture, fixed-memory serving loops).  It has no
 * counterpart in the reference.  The sort workspace is a static array in the library's
 * device data, one per GPU, sized for ETHOS_NOALLOC_MAX_PAIRS pairs (about 18 MiB, part
 * of the library's code object: held on a GPU from when the code object is loaded there,
 * i.e. the first launch of any of the library's kernels on it, until the process ends);
 * larger n_pairs returns
 * ETHOS_ESIZE.  Every other argument and every output is as for ethos_sort_segment, and
 * the outputs are bit-identical to it.  All calls on one GPU share that array: calls that
 * overlap on one GPU (on different streams, or from different threads) race and must be
 * serialised by the caller.  No allocation happens inside (no hipMalloc or hipFree); the
 * first call on a GPU looks the array's device address up once.
 */
#define ETHOS_NOALLOC_MAX_PAIRS (1 << 20)

int ethos_sort_segment_noalloc(const int32_t* ids, int64_t n_pairs, int64_t n_experts, int32_t* perm,
                               int32_t* uniq_ids, int32_t* seg_off, int32_t* pair_slot, int32_t* sorted_slot,
                               int32_t* n_unique, void* stream);

/*
 * Expert generation for the unique experts, u = 0 .. U-1, z = latents[uniq_ids[u]]:
 *   h[u] = RN_T(gelu(RN_T(W1 z)))        the hidden row h_i (model.py:323), erf-form GELU
 *   v[u] = RN_T(W_v h[u])                h_i @ W_v (model.py:332), W_v^T = w2 rows d_model .. 2 d_model - 1
 * Replaces the per-pair gelu(z @ W1) and h @ W_v of model.py:320-332 (weights read at
 * model.py:297-300; ExpertGenerationNetwork model.py:168-179); each unique expert is
 * generated once.
 *   latents  [n_experts, d_latent]          dtype T  (expert_latents.weight)
 *   uniq_ids [max_unique], n_unique [1]     from ethos_sort_segment (U read on the device)
 *   w1       [d_hidden, d_latent]           dtype T  (generation_network.net.0.weight)
 *   w2       [2 * d_model, d_hidden]        dtype T  (generation_network.net.2.weight)
 *   h_out    [max_unique, d_hidden]         dtype T  rows u < U written
 *   v_out    [max_unique, d_model]          dtype T  rows u < U written
 * v_out may be NULL: then only the hidden rows are produced (w2 is not read), as
 * ethos_apply_hidden needs.
 * Limits: d_latent % 16 (bf16) or % 2 (fp32) == 0, d_hidden % 32 == 0, d_model % 32 == 0;
 * bf16 weights and outputs 16-byte aligned.
 */
int ethos_generate(const void* latents, int64_t n_experts, const int32_t* uniq_ids, const int32_t* n_unique,
                   int64_t max_unique, const void* w1, const void* w2, int32_t d_latent, int32_t d_hidden,
                   int32_t d_model, int32_t dtype, void* h_out, void* v_out, void* stream);

/* Workspace size for ethos_apply_scatter (token projections + per-pair activations). */
size_t ethos_apply_workspace_bytes(int64_t n_tok, int32_t n_heads, int32_t top_k, int32_t d_hidden, int32_t dtype);

/*
 * Expert apply and weighted scatter-back, averaged over heads.
 * Replaces the pair loop and head average of model.py:306-341 (and the per-token
 * Triton program of kernels.py:83-120 with the head loop of kernels.py:167-220).
 *   x             [n_tok, d_model]                 dtype T
 *   w2            [2 * d_model, d_hidden]          dtype T  (generation_network.net.2.weight;
 *                                                  its first d_model rows are W_u^T)
 *   h, v          [>= U, d_hidden], [>= U, d_model] dtype T, from ethos_generate
 *   perm, sorted_slot, pair_slot                   from ethos_sort_segment
 *   scores        [n_tok, n_heads, top_k]          dtype T  gates from ethos_route_topk
 *   workspace     >= ethos_apply_workspace_bytes(...) bytes (scratch)
 *   out           [n_tok, d_model]                 dtype T
 * xp_t = RN_T(x_t W_u) (x_proj, model.py:326, formed once per token);
 * a_p = RN_T(RN_T(gelu(RN_T(h_e . xp_t))) * g_p) (model.py:329);
 * out[t] = RN_T(sum_h^T RN_T(sum_k RN_T(a_p * v_e)) / n_heads) (model.py:332-341).
 * Limits: d_model and d_hidden multiples of 8 (bf16) or 4 (fp32) and <= 4096 (bf16) /
 * 2048 (fp32); x, w2, h, v, workspace and out 16-byte aligned.
 */
int ethos_apply_scatter(const void* x, const void* w2, const void* h, const void* v, const int32_t* perm,
                        const int32_t* sorted_slot, const int32_t* pair_slot, const void* scores, int64_t n_tok,
                        int32_t n_heads, int32_t top_k, int32_t d_model, int32_t d_hidden, int32_t dtype,
                        void* workspace, size_t workspace_bytes, void* out, void* stream);

/*
 * The token projection of the expert apply, x_proj = RN_T(x W_u) with W_u the first d_model
 * rows of w2 (generation_network.net.2.weight), once per token -- the reference forms it
 * inside the pair loop (model.py:326).  For ethos_expert_forward's xp argument.
 *   x [n_tok, d_model], w2 [2 d_model, d_hidden], wut [d_hidden, d_model] (bf16: required
 *   for d_model % 64 == 0; the transpose of w2's first d_model rows), xp_out [n_tok, d_hidden]
 */
int ethos_token_proj(const void* x, const void* w2, const void* wut, int64_t n_tok, int32_t d_model,
                     int32_t d_hidden, int32_t dtype, void* xp_out, void* stream);

/* Workspace size for ethos_expert_forward (order 0: layer order, 1: hidden-space order). */
size_t ethos_expert_forward_workspace_bytes(int64_t n_tok, int32_t n_heads, int32_t top_k, int64_t max_unique,
                                            int32_t d_model, int32_t d_hidden, int32_t dtype, int32_t order);

/*
 * The expert stages of one layer call in one entry point: generation over the unique
 * experts, per-pair activation and weighted scatter-back, on the sorted pairs from
 * ethos_sort_segment.  Replaces the pair loop of model.py:306-341 with the generator of
 * model.py:168-179 (weights read at model.py:297-300) -- the work of ethos_generate
 * followed by ethos_apply_scatter (order 0) or ethos_apply_hidden (order 1), with the same
 * results (bit-identical), scheduled so that the activations are computed from the hidden
 * rows while they are on chip.
 *   x, scores, perm, sorted_slot, pair_slot, n_tok, n_heads, top_k   as for ethos_apply_scatter
 *   latents, n_experts, uniq_ids, n_unique, max_unique, w1, w2       as for ethos_generate
 *   seg_off   [max_unique + 1] int32 from ethos_sort_segment (first sorted position of
 *             each unique expert; seg_off[U] = number of pairs)
 *   wut       bf16 only, may be NULL: W_u^T [d_hidden, d_model] (the transpose of the first
 *             d_model rows of w2) prepared by the caller, e.g. once per weight version;
 *             NULL transposes it into the workspace on every call
 *   xp        may be NULL: the token projection [n_tok, d_hidden] dtype T from
 *             ethos_token_proj (computed by the caller, e.g. on a second stream while the
 *             routing runs); NULL computes it here
 *   workspace >= ethos_expert_forward_workspace_bytes(...) bytes (scratch)
 *   h_out     [max_unique, d_hidden] dtype T: the hidden rows (rows u < U written)
 *   out       [n_tok, d_model] dtype T
 * Limits: those of ethos_generate and ethos_apply_scatter; x, w1, w2, wut, workspace, h_out
 * and out 16-byte aligned.
 */
int ethos_expert_forward(const void* x, const void* latents, int64_t n_experts, const void* w1, const void* w2,
                         const void* wut, const void* xp, const int32_t* uniq_ids, const int32_t* seg_off,
                         const int32_t* n_unique, int64_t max_unique,
                         const int32_t* perm, const int32_t* sorted_slot, const int32_t* pair_slot, const void* scores,
                         int64_t n_tok, int32_t n_heads, int32_t top_k, int32_t d_latent, int32_t d_hidden,
                         int32_t d_model, int32_t dtype, int32_t order, void* workspace, size_t workspace_bytes,
                         void* h_out, void* out, void* stream);

/* Workspace size for ethos_apply_hidden. */
size_t ethos_apply_hidden_workspace_bytes(int64_t n_tok, int32_t n_heads, int32_t top_k, int32_t d_model,
                                          int32_t d_hidden, int32_t dtype);

/*
 * Expert apply by hidden-space reordering: the paper's Algorithm 1 (paper/ETHOS.pdf p.10,
 * "Reordered MoE Execution Kernel": x_proj = x W_u once, h_accum += a_j h_j over the
 * selected experts, y = h_accum W_v once), the execution order kernels.py:123-145 names,
 * with the head average of model.py:341.  The same function as ethos_apply_scatter with
 * different rounding points; v rows are never formed (generate with v_out = NULL).
 *   x, w2, h, perm, sorted_slot, pair_slot, scores, out   as for ethos_apply_scatter
 *   workspace     >= ethos_apply_hidden_workspace_bytes(...) bytes (scratch)
 * a_p as in ethos_apply_scatter;
 * hs_t = RN_T((1/n_heads) sum_p RN32(a_p h_e)) over the token's pairs (heads, then k, float32);
 * out[t] = RN_T(hs_t W_v) (W_v^T = rows d_model .. 2 d_model - 1 of w2).
 * Limits: d_model and d_hidden multiples of 8 (bf16) or 4 (fp32), d_model <= 4096,
 * d_hidden <= 4096 (bf16) / 2048 (fp32); x, w2, h, workspace and out 16-byte aligned.
 */
int ethos_apply_hidden(const void* x, const void* w2, const void* h, const int32_t* perm, const int32_t* sorted_slot,
                       const int32_t* pair_slot, const void* scores, int64_t n_tok, int32_t n_heads, int32_t top_k,
                       int32_t d_model, int32_t d_hidden, int32_t dtype, void* workspace, size_t workspace_bytes,
                       void* out, void* stream);

/*
 * Per-pair part of the expert stages' backward: the derivative of model.py:312-341, which
 * the reference obtains from autograd on its pure-PyTorch layer (its Triton layer,
 * kernels.py:145-221, has no backward).  With xp = x W_u and dyb = (dy / n_heads) W_v^T
 * (both float32 [n_tok, d_hidden], formed by the caller's GEMMs), for pair p of token t
 * with expert slot s: c = h_s . xp_t, a = gelu(c) g_p, da = dyb_t . h_s;
 *   dscores[p] = gelu(c) da                               float32 [n_tok, n_heads, top_k]
 *   hacc[t]    = sum_p a h_s                              float32 [n_tok, d_hidden]
 *   dxp[t]     = sum_p g gelu'(c) da h_s                  float32 [n_tok, d_hidden]
 *   dh[s]      = sum_p a dyb_t + g gelu'(c) da xp_t      float32 [>= U, d_hidden], rows s < U
 *                                                          written; summed over the expert's
 *                                                          pairs in sorted order (blocks of 64
 *                                                          sorted positions, then the blocks'
 *                                                          parts in order): deterministic
 *   h, pair_slot, scores            as for ethos_apply_scatter (h 16-byte aligned)
 *   perm, sorted_slot, seg_off      from ethos_sort_segment on the same routing
 *   workspace  >= ethos_expert_backward_workspace_bytes(...) bytes, 16-byte aligned (scratch)
 * Limits: d_hidden a multiple of 8 (bf16) or 4 (fp32), <= 4096 (bf16) / 2048 (fp32).
 */
size_t ethos_expert_backward_workspace_bytes(int64_t n_tok, int32_t n_heads, int32_t top_k, int32_t d_hidden);
int ethos_expert_backward(const void* h, const float* xp, const float* dyb, const int32_t* pair_slot,
                          const int32_t* perm, const int32_t* sorted_slot, const int32_t* seg_off, const void* scores,
                          int64_t n_tok, int32_t n_heads, int32_t top_k, int32_t d_hidden, int32_t dtype,
                          void* workspace, size_t workspace_bytes, float* dscores, float* hacc, float* dxp, float* dh,
                          void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ETHOS_HIP_H */
