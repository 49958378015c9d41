/*
 * dsv.h — C ABI of the MI355X (gfx950) tree-verification library (libdsv.so).
 *
 * The library implements the target-side tree-verification hot path of
 * DiffSpec: tree-masked, grouped-query attention of a draft tree's nodes
 * against a long (optionally paged) KV prefix, and the tree acceptance walk
 * that follows it.  Every entry point below replaces one function of the
 * reference's Python API; the citation names the reference file:line whose
 * contract (argument meaning, shapes, layouts, error behaviour) it follows.
 *
 * Conventions
 *   - All tensors are caller-owned device memory described by dsv_tensor
 *     (pointer + dtype + shape + strides in elements).  No torch types cross
 *     this boundary.  The innermost (head_dim / vocab) stride must be 1.
 *   - Every function returns DSV_OK (0) or a negative error code; the text of
 *     the last error on the calling thread is available from dsv_last_error().
 *     No C++ exception crosses the ABI and there is no silent fallback.
 *   - Work is enqueued on the caller's HIP stream; functions never synchronise
 *     the device.  Scratch memory comes from a caller-allocated workspace whose
 *     size the matching *_workspace_bytes() function returns.
 *   - Functions are stateless and re-entrant; concurrent calls on different
 *     streams must use different workspaces.
 */
#ifndef DSV_H_
#define DSV_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSV_MAX_DIMS 6

typedef enum dsv_dtype {
  DSV_BF16 = 0,
  DSV_F16 = 1,
  DSV_F32 = 2,
  DSV_I8 = 3,
  DSV_U8 = 4,
  DSV_BOOL = 5,
  DSV_I32 = 6,
  DSV_I64 = 7
} dsv_dtype;

typedef enum dsv_status {
  DSV_OK = 0,
  DSV_ERR_INVALID = -1,     /* bad shape / dtype / stride / argument */
  DSV_ERR_UNSUPPORTED = -2, /* valid request outside what the kernels implement */
  DSV_ERR_WORKSPACE = -3,   /* workspace missing or too small */
  DSV_ERR_HIP = -4          /* a HIP runtime call failed */
} dsv_status;

typedef struct dsv_tensor {
  void* data;                      /* device pointer (may be NULL only when ndim == 0) */
  int32_t dtype;                   /* dsv_dtype */
  int32_t ndim;                    /* 0 means "absent" for optional arguments */
  int64_t shape[DSV_MAX_DIMS];
  int64_t stride[DSV_MAX_DIMS];    /* in elements */
} dsv_tensor;

/* Library identification and error text. */
int dsv_version(void);
const char* dsv_last_error(void);

/*
 * Instrumentation (no reference counterpart; the reference times phases with
 * host clocks under DIFFSPEC_PROFILE, draft/diffspec_model.py:594-605).
 * Arms a one-shot pair of caller-created hipEvent_t handles for the next
 * entry point called on this thread, then disarms.  Attention entry points
 * attach them to kernel 1's own launch (hipExtLaunchKernel): they take that
 * kernel's start and end times, so their interval is its execution time.
 * Acceptance entry points record `start` on their stream right before the
 * vocabulary sweep and `stop` right after it.  Pass NULLs to disarm.
 */
int dsv_set_timing_events(void* start_event, void* stop_event);

/*
 * Dry run (no reference counterpart; a safety check for callers and tests).
 * While enabled on a thread, the attention entry points validate and plan as
 * usual but launch nothing and touch no device memory: instead they walk
 * every global and LDS address kernels 1-3 would access, with the kernels'
 * own address arithmetic, and fail with DSV_ERR_INVALID naming the first
 * access outside the extent of its argument (pointers are only compared,
 * never dereferenced, so the call runs on machines without a GPU).
 * dsv_dry_run_checks() returns the number of checks the last dry run made.
 */
int dsv_set_dry_run(int enable);
int64_t dsv_dry_run_checks(void);

/* ------------------------------------------------------------------------- */
/* Attention (kernels 1-3: split-K flash-decoding, tree-ancestor block, merge) */
/* ------------------------------------------------------------------------- */

/*
 * Workspace needed by any attention entry point for queries of shape
 * [B, M, H, D] against keys with Hk heads and n_keys prefix keys, with an
 * optional tree block (has_tree != 0).  Returns 0 on invalid arguments and
 * on sizes beyond the kernels' 32-bit counts (batch <= 2^20, query heads <=
 * 65536, keys <= 2^40, H / Hk * M <= 2^24, B * H * M <= 2^30), which every
 * attention entry point refuses with DSV_ERR_UNSUPPORTED.
 */
size_t dsv_attn_workspace_bytes(int64_t B, int64_t M, int64_t H, int64_t Hk,
                                int64_t D, int64_t n_keys, int64_t page_size,
                                int has_tree);

/*
 * prefix_attention_forward — runtime/tree_attention.py:414-446; LSE layout of
 * flash_attn_with_kvcache(return_softmax_lse=True), runtime/attention_compat.py:103-132.
 *   q   [B, M, H, D] bf16|f16|f32 (f32 inputs are computed in fp32)
 *   k,v [B, N, Hk, D] same dtype; H % Hk == 0 (Hk == H is the repeat_kv'd form)
 *   n_keys  keys [0, n_keys) are attended (cache_seqlens); n_keys < 0 means N
 *   out [B, M, H, D] q dtype or f32;  lse [B, H, M] f32 (natural log)
 */
int dsv_prefix_attention_forward(const dsv_tensor* q, const dsv_tensor* k,
                                 const dsv_tensor* v, int64_t n_keys,
                                 dsv_tensor* out, dsv_tensor* lse,
                                 void* workspace, size_t workspace_bytes,
                                 void* stream);

/*
 * flash_attn_with_kvcache — runtime/attention_compat.py:103-132 (the
 * flash-attn contract it stands in for: keys [0, cache_seqlens[b]) of batch
 * b, causal masking aligned to the end of that range, softmax_lse
 * [B, H, M]).
 *   q              [B, M, H, D] bf16|f16|f32;  k_cache, v_cache [B, N, Hk, D]
 *   cache_seqlens  optional [B] int32|int64 per-batch length (clamped to
 *                  [0, n_keys]); ndim 0 = every batch uses n_keys
 *   n_keys         scalar length (the reference's int cache_seqlens); < 0 = N
 *   causal         != 0: query m of batch b sees keys n <= len_b - M + m
 *                  (flash-attn's bottom-right alignment for M <= len_b)
 *   out [B, M, H, D] q dtype or f32;  softmax_lse optional [B, H, M] f32
 * A query row with no visible key gets out = 0 and lse = -inf.
 */
int dsv_flash_attn_with_kvcache(const dsv_tensor* q, const dsv_tensor* k_cache,
                                const dsv_tensor* v_cache,
                                const dsv_tensor* cache_seqlens, int64_t n_keys,
                                int causal, dsv_tensor* out,
                                dsv_tensor* softmax_lse, void* workspace,
                                size_t workspace_bytes, void* stream);

/*
 * tree_attention_forward — runtime/tree_attention.py:462-541 (mask handling of
 * _maybe_to_int8_mask, :449-460).
 *   q   [B, M, H, D];  k, v [B, M, Hk, D] (the post-cache tree block)
 *   tree_mask  [B, 1, T, T] or [B, T, T] with T >= M (M <= 1024); the lower-right M x M
 *              block is used.  Float masks are additive (keep where == 0);
 *              int8 / uint8 / bool masks keep where != 0.
 *   prefix_lse [B, H, M] f32 (any layout reshaping to it, as the reference's
 *              reshape(B, H, M, -1) does)
 *   current_out [B, M, H, D] q dtype;  weight [B, M, H, 1] q dtype with
 *              weight = sigmoid(prefix_lse - tree_lse)
 *   tree_lse   optional [B, M, H] f32 output (ndim == 0 to skip)
 */
int dsv_tree_attention_forward(const dsv_tensor* q, const dsv_tensor* k,
                               const dsv_tensor* v, const dsv_tensor* tree_mask,
                               const dsv_tensor* prefix_lse,
                               dsv_tensor* current_out, dsv_tensor* weight,
                               dsv_tensor* tree_lse, void* workspace,
                               size_t workspace_bytes, void* stream);

/*
 * FusedBundleVerifier.verify_bundle — runtime/bundle_verifier.py:166-297.
 * Masked attention of q [B, M, H, D] over k, v [B, N, Hk, D] with an int8 /
 * uint8 / bool mask [Bm, M, N] (Bm in {1, B}; 1 = keep).  shared_prefix_len
 * does not change the result in the reference (both phases apply the mask)
 * and is therefore not an argument.
 *   out [B, M, H, D] q dtype or f32;  lse [B, M, H] f32
 */
int dsv_verify_bundle(const dsv_tensor* q, const dsv_tensor* k,
                      const dsv_tensor* v, const dsv_tensor* mask,
                      dsv_tensor* out, dsv_tensor* lse, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * PagedBundleVerifier.verify_bundle_paged — runtime/bundle_verifier.py:341-366
 * (unimplemented in the reference; page-pool layout of
 * core/kv_cache/paged_kv.py:56-65, page list of :325-340).
 *   kv_pages   [L, 2, P, Hk, page_size, D]; page_size a power of two
 *   page_table [n_pages] or [B, n_pages] int32|int64 logical -> physical page
 *   mask       [Bm, M, N] int8|uint8|bool over the logical token sequence
 *   out [B, M, H, D];  lse [B, M, H] f32
 */
int dsv_verify_bundle_paged(const dsv_tensor* q, const dsv_tensor* kv_pages,
                            const dsv_tensor* page_table, int64_t layer_idx,
                            const dsv_tensor* mask, dsv_tensor* out,
                            dsv_tensor* lse, void* workspace,
                            size_t workspace_bytes, void* stream);

/*
 * Fused tree verification over a paged (or contiguous) KV cache: the hybrid
 * branch of the target attention, llama_target_model.py:834-867 (prefix
 * attention + tree-masked attention + sigmoid-LSE merge), computed in one
 * launch of kernel 1 (S prefix splits + one tree split whose ancestor bitmask
 * is built in-kernel from the parent array) and one launch of kernel 3.
 *   q          [B, M, H, D]
 *   k, v       either a page pool half kv_pages[layer, 0|1] viewed as
 *              [P, Hk, page_size, D] together with page_table [B|-, n_pages],
 *              or a contiguous cache [B, L, Hk, D] (page_table->ndim == 0).
 *   n_prefix   tokens [0, n_prefix) are the prefix; the tree's K/V rows are
 *              tokens [n_prefix, n_prefix + M) of the same cache
 *              (KVCache.cat layout, runtime/cache_state.py:52-66)
 *   parent     [B, M] or [M] int32|int64: parent node of each tree node, < 0 for
 *              the root (the ancestor relation of runtime/draft_tree.py:188-214);
 *              M <= 1024 nodes
 *   row_perm   optional [M] int32 node order used to pack query rows (bundle
 *              order, core/bundle_scheduler.py:42-123); ndim == 0 = identity.
 *              It must be a permutation of [0, M) (dsv_bundle_order's output
 *              is one): entries are clamped into [0, M), and a repeated
 *              entry leaves the rows of the missing nodes unwritten.
 *   out [B, M, H, D] bf16|f16|f32;  lse [B, M, H] f32 (ndim == 0 to skip)
 */
int dsv_tree_verify(const dsv_tensor* q, const dsv_tensor* k,
                    const dsv_tensor* v, const dsv_tensor* page_table,
                    int64_t n_prefix, const dsv_tensor* parent,
                    const dsv_tensor* row_perm, dsv_tensor* out,
                    dsv_tensor* lse, void* workspace, size_t workspace_bytes,
                    void* stream);

/*
 * dsv_tree_verify without a workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No reference counterpart.  The split
 * partials live in a fixed per-GPU device array of DSV_NOALLOC_SCRATCH_BYTES
 * that the library holds until the process ends; shapes whose split plan
 * needs more fail with DSV_ERR_UNSUPPORTED (dsv_attn_workspace_bytes gives
 * the need; at head_dim 128 with 8 KV heads on 256 CUs: one tree of <= 64
 * nodes up to 512K prefix tokens, <= 128 nodes up to 256K, <= 256 nodes up
 * to 128K, 8 trees of 64 nodes at 64K).  The call allocates nothing (its
 * first call on a GPU looks the array's address up and creates one event).
 * Every call on one GPU shares that GPU's array.  Calls issued on different
 * streams are serialised by the library: a call on another stream than the
 * previous one makes its stream wait for the previous call's kernels.
 * Under stream capture this ordering is not added (the captured kernels run
 * when the graph is replayed): replays of graphs holding this call, and
 * direct calls, must not overlap in time on one GPU; the caller orders them.
 * Arguments and results are those of dsv_tree_verify.
 */
#define DSV_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int dsv_tree_verify_noalloc(const dsv_tensor* q, const dsv_tensor* k,
                            const dsv_tensor* v, const dsv_tensor* page_table,
                            int64_t n_prefix, const dsv_tensor* parent,
                            const dsv_tensor* row_perm, dsv_tensor* out,
                            dsv_tensor* lse, void* stream);

/* ------------------------------------------------------------------------- */
/* Acceptance (kernel 4)                                                      */
/* ------------------------------------------------------------------------- */

#define DSV_ACCEPT_GREEDY 0
#define DSV_ACCEPT_TYPICAL 1

/* Workspace for dsv_tree_accept with T trees of M nodes over vocab V. */
size_t dsv_accept_workspace_bytes(int64_t T, int64_t M, int64_t V);

/*
 * Tree acceptance walk — draft/tree_verification.py:100-182 (greedy:
 * next = argmax(logits), ok[i] = draft[i] == next[parent_ext[i]], bounded
 * ancestor closure of max_hops rounds, winner = argmax(where(ok, pos, 0)),
 * traceback, next token = next[winner]).  Typical mode replaces the greedy
 * test with the posterior criterion p_T(draft[i] | parent) >
 * min(posterior_threshold, posterior_alpha * exp(-H(p_T(. | parent)))).
 *   logits  [T, M, V] bf16|f16|f32
 *   draft   [T, M] int64   draft token of every node (node 0 = root)
 *   parent  [T, M-1] int64 reference convention: parent[k] is the parent of
 *           node k+1 among the non-root nodes; -1 or k itself = the root
 *   pos     [T, M] or [M] int64 position ids
 *   max_hops  closure rounds, min(max_depth + 2, M) in the reference
 *   out_path  [T, M] int64: accepted node ids root..winner, then -1
 *   out_tokens[T, M] int64: draft tokens along the path, then -1
 *   out_info  [T, 4] int64: {winner node, accept_length, next_token, path_len}
 *   out_next  optional [T, M] int64: per-node argmax token (ndim == 0 to skip)
 */
int dsv_tree_accept(int mode, const dsv_tensor* logits, const dsv_tensor* draft,
                    const dsv_tensor* parent, const dsv_tensor* pos,
                    int64_t max_hops, float temperature,
                    float posterior_threshold, float posterior_alpha,
                    dsv_tensor* out_path, dsv_tensor* out_tokens,
                    dsv_tensor* out_info, dsv_tensor* out_next,
                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * Sampling acceptance — the logits_processor branch of verify_new
 * (draft/tree_verification.py:103-106: warp, softmax, one multinomial draw
 * per node, then the walk of :108-182) with the warpers of
 * prepare_logits_processor (:15-32).  y = logits / temperature rounded to the
 * logits dtype (temperature == 1: unchanged); top-p (applied when
 * 1e-8 <= top_p < 1) keeps the head of the order "descending y, then
 * descending index" whose probability mass reaches top_p, the masses taken
 * as exact 64-bit fixed-point integers; top-k (applied when > 0) keeps
 * y >= the k-th largest y.  The draw per node is a counter-based Gumbel-max
 * over the kept tokens: argmax of y + G, G = -ln(-ln U), U = (w + 0.5) 2^-32
 * with w the output word token & 3 of Philox4x32-10 at key (seed mod 2^32,
 * seed >> 32) and counter (token >> 2, node, tree, 0), the
 * logarithms evaluated with a fixed sequence of correctly rounded double
 * operations, so the draws are reproducible bit for bit; they are samples of
 * softmax(y) over the kept set.  A row without a finite logit draws token 0.
 *   logits, draft, parent, pos, max_hops, out_*: as dsv_tree_accept;
 *   out_next receives the per-node draws.  temperature > 1e-5, compared in
 *   double precision (the reference takes the greedy branch at or below
 *   it).  Workspace:
 *   dsv_accept_workspace_bytes.
 */
int dsv_tree_accept_sample(const dsv_tensor* logits, const dsv_tensor* draft,
                           const dsv_tensor* parent, const dsv_tensor* pos,
                           int64_t max_hops, float temperature, float top_p,
                           int64_t top_k, uint64_t seed, dsv_tensor* out_path,
                           dsv_tensor* out_tokens, dsv_tensor* out_info,
                           dsv_tensor* out_next, void* workspace,
                           size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------- */
/* Accepted-path KV commit                                                    */
/* ------------------------------------------------------------------------- */

/*
 * KV compaction after the walk — draft/tree_verification.py:197-217
 * (select_indices = path + start; data[..., start:start+n, :] =
 * data[..., select_indices, :] for every cache tensor; cache length =
 * start + n).  One launch for every row of the cache; the path and its
 * length n are read from device memory (the outputs of dsv_tree_accept),
 * so no host round trip is needed.  Every read happens before any write,
 * as with the reference's gather into a temporary.
 *   kv          page pool [L, 2, P, Hk, page, D] with page_table, or, when
 *               page_table has ndim 0, a dense cache [..., S, D] with 1..4
 *               leading dimensions; bf16|f16|f32, innermost stride 1,
 *               16-byte aligned token rows
 *   page_table  [n_logical] int32|int64 (logical page -> physical page)
 *   start       first tree token (cache length - M)
 *   path        [M] or [T, M] int64: accepted node ids, root first
 *   info        [4] or [T, 4] int64: info[3] = path length n
 *   tree        which tree of path / info (0 for one tree)
 * The cache length itself (start + n) is the caller's.
 */
int dsv_kv_commit(const dsv_tensor* kv, const dsv_tensor* page_table, int64_t start,
                  const dsv_tensor* path, const dsv_tensor* info, int64_t tree,
                  void* stream);

/* ------------------------------------------------------------------------- */
/* lm_head fused with the acceptance (kernel 5 + kernel 4's walk)             */
/* ------------------------------------------------------------------------- */

/* Workspace for dsv_lmhead_accept with T trees of M nodes over vocab V. */
size_t dsv_lmhead_accept_workspace_bytes(int64_t T, int64_t M, int64_t V);

/*
 * dsv_tree_accept over logits = hidden . weight^T computed in the same
 * launch sequence, without writing the logits: replaces the target's
 * self.base_model.lm_head(hidden_states) (draft/diffspec_model.py:229-231)
 * followed by the walk of verify_new (draft/tree_verification.py:100-182).
 * Every logit is rounded to bf16 before the argmax and the softmax
 * statistics, as the reference's bf16 logits are.
 *   hidden      [T, M, Dm] bf16 (rows of all trees at one stride); Dm a
 *               multiple of 64
 *   weight      [V, Dm] bf16 (nn.Linear.weight), rows 16-byte aligned
 *   draft, parent, pos, max_hops, temperature, thresholds, out_*: as
 *               dsv_tree_accept
 *   logits_out  optional bf16 [T, M, V]: also write the logits (ndim 0 to skip)
 * The weight is streamed once per 64 hidden rows (T * M <= 64: once).
 * Typical mode decides near-threshold nodes again in float64 from the
 * written logits, as dsv_tree_accept does; without logits_out it keeps the
 * decision of the fp32 statistics.
 */
int dsv_lmhead_accept(int mode, const dsv_tensor* hidden, const dsv_tensor* weight,
                      const dsv_tensor* draft, const dsv_tensor* parent,
                      const dsv_tensor* pos, int64_t max_hops, float temperature,
                      float posterior_threshold, float posterior_alpha,
                      dsv_tensor* out_path, dsv_tensor* out_tokens,
                      dsv_tensor* out_info, dsv_tensor* out_next,
                      dsv_tensor* logits_out, void* workspace,
                      size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------- */
/* Tree K/V append with RoPE                                                  */
/* ------------------------------------------------------------------------- */

/*
 * The tree tokens' keys and values enter the cache at logical tokens
 * [start, start + M): keys rotated by RoPE, values as they are; queries are
 * rotated into q_out in the same launch when given.  Replaces, per layer,
 * apply_rotary_pos_emb_L31 (llama_target_model.py:452-473, :408-427,
 * applied at :768-771) followed by KVCache.cat (runtime/cache_state.py:52-66,
 * used at llama_target_model.py:781-783) or the per-token
 * PagedKVCache.write_kv (core/kv_cache/paged_kv.py:168-223).  RoPE rounds
 * like torch's 16-bit elementwise ops: x * cos and rotate_half(x) * sin are
 * each rounded to the dtype, then their sum.
 *   k, v        [M, Hk, D] or [1, M, Hk, D] bf16|f16 (projected, before RoPE)
 *   cos, sin    [M, D] or [1, M, D] at the tree tokens' positions, same dtype
 *               (ndim 0: no RoPE)
 *   k_dst, v_dst  page-pool halves [P, Hk, page, D] with page_table, or
 *               (page_table ndim 0) dense caches [Hk, S, D] or [1, Hk, S, D]
 *   page_table  [n_logical] int32|int64
 *   start       cache length before the tree (first tree token)
 *   q, q_out    optional [M, H, D] or [1, M, H, D] (ndim 0 to skip)
 * D must be a multiple of 16; token rows 16-byte aligned.  Sizes: M <= 2^24,
 * Hk and H <= 65536, D <= 4096, and (2 * Hk + H) * M * D / 16 <= 2^31
 * (DSV_ERR_UNSUPPORTED beyond).
 * Aliasing: inputs (k, v, q, cos, sin) may not overlap outputs (k_dst, v_dst,
 * q_out), nor outputs each other (DSV_ERR_INVALID), except row for row in
 * place: q_out == q with the same strides, or, with a dense cache, k (v)
 * being exactly k_dst's (v_dst's) tree slots [start, start + M).
 */
int dsv_kv_append(const dsv_tensor* k, const dsv_tensor* v, const dsv_tensor* cos,
                  const dsv_tensor* sin, dsv_tensor* k_dst, dsv_tensor* v_dst,
                  const dsv_tensor* page_table, int64_t start, const dsv_tensor* q,
                  dsv_tensor* q_out, void* stream);

/* ------------------------------------------------------------------------- */
/* Bundle order (query packing permutation)                                   */
/* ------------------------------------------------------------------------- */

/*
 * The node order that packs a tree's query rows bundle by bundle (the
 * row_perm of dsv_tree_verify), computed on the GPU from the parent array.
 * Replaces the host scheduling of verify_new (draft/tree_verification.py:139-159:
 * descriptor with leaves in index order and depths) and
 * BundleScheduler.schedule_bundles with its branching-ancestor and path
 * helpers (core/bundle_scheduler.py:42-171): leaves bucketed by branching
 * ancestor (buckets in the order of their lowest leaf), stably sorted by
 * depth, cut into bundles of bundle_size leaves, at most max_bundles bundles;
 * the order lists, bundle by bundle and leaf by leaf, the not yet listed
 * nodes of each leaf's root path root first, then every node no emitted leaf
 * covers, in index order.
 *   parent       [M] or [B, M] int32|int64; a parent < 0, equal to the node or
 *                >= M means none, node 0 is a root
 *   bundle_size  leaves per bundle (>= 1) when num_bundles == 0
 *   num_bundles  > 0: bundle_size = max(1, ceil(leaves / num_bundles))
 *   max_bundles  bundles emitted; values below 1 emit one bundle, as the
 *                scheduler checks the bound after adding a bundle
 *   perm         [M] or [B, M] int32 (contiguous): perm[b, j] = node in row j
 *   bundle_of    optional, shape of perm: bundle id of the leaf through which
 *                each node was listed, -1 for uncovered nodes (ndim 0 to skip)
 * 1 <= M <= 1024.  One launch, one workgroup per tree, no host round trip.
 */
int dsv_bundle_order(const dsv_tensor* parent, int64_t bundle_size,
                     int64_t num_bundles, int64_t max_bundles, dsv_tensor* perm,
                     dsv_tensor* bundle_of, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSV_H_ */
