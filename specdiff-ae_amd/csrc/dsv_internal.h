// dsv_internal.h — device-side types, helpers and launch-argument structs
// shared by the gfx950 kernels and the C-ABI layer of libdsv.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dsv {

// ---------------------------------------------------------------------------
// Vector types used as MFMA operands / 16-byte memory transactions.
// ---------------------------------------------------------------------------
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Element-type tags (the kernels move 16-bit storage; the tag selects the
// MFMA flavour and the fp32 -> 16-bit conversion of softmax probabilities).
struct BF16 {};
struct F16 {};

// Limits of the in-kernel tables (checked by the host before launch).
constexpr int kPageLds = 1040;       // page-table entries staged per split
constexpr int kTreeMaxM = 1024;      // tree nodes handled by the tree split
constexpr int kTreeMaxW = kTreeMaxM / 64;  // 64-bit visibility words per node
// The tree split's visibility table: up to kTreeNodeM nodes it is indexed by
// node (kTreeNodeW words each); larger trees take a table indexed by the
// workgroup's 256 packed rows (query head g, node slot mi: row = g * M + mi),
// kTreeMaxW words each.
constexpr int kTreeNodeM = 256;
constexpr int kTreeNodeW = kTreeNodeM / 64;
constexpr int kTreeSlots = 256;

// A key/value source: contiguous [B, N, Hk, D] or a page pool half
// [P, Hk, page, D] addressed through a page table.
//   contiguous:  addr(b, n, h) = base + b*sb + (key0+n)*st + h*sh
//   paged:       ln = key0+n; addr = base + b*sb + pt[b][ln>>ps]*sp + h*sh + (ln & (2^ps-1))*st
struct KvSrc {
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_sb, k_sp, k_sh, k_st;
  int64_t v_sb, v_sp, v_sh, v_st;
  const void* pt;      // page table (nullptr -> contiguous)
  int pt_i64;          // page table element is int64 (else int32)
  int ps_shift;        // log2(page size)
  int64_t pt_sb;       // page-table batch stride (0 -> shared by all batches)
  int64_t key0;        // logical index of this source's key 0
  int64_t n_phys;      // physical pages in the pool (page ids are clamped to it)
  int64_t k_bytes;     // byte span of the K (V) tensor view from its base pointer
  int64_t v_bytes;
  int fast32;          // per-key byte offsets fit in 32 bits (set by the host)
};

// Arguments of the split-K attention kernel (kernels 1 and 2).
struct AttnArgs {
  const uint16_t* q;
  int64_t q_sb, q_sm, q_sh;
  int B, M, H, Hk, G, R;   // R = G*M query rows per KV head
  int n_rb;                // row blocks of 256 rows
  float scale_log2;        // log2(e) / sqrt(D)

  KvSrc pre;               // prefix source
  int64_t n_pre;           // prefix keys [0, n_pre)
  const void* seqlens;     // optional [B] per-batch prefix length (clamped to [0, n_pre])
  int seqlens_i64;
  int causal;              // row m sees prefix keys n <= len_b - M + m (flash-attn causal)
  int n_splits;            // prefix splits
  int64_t kps;             // prefix keys per split (whole 32-key tiles, Geo<D>::KT)

  // Optional byte mask [Bm, M, N] over the prefix keys (1 = keep).
  const uint8_t* dmask;
  int64_t dm_sb, dm_sm, dm_sn, dm_n;

  // Optional tree split: keys [0, M) of `tree`, visibility = ancestor-or-self.
  int has_tree;
  KvSrc tree;
  const void* tpar;        // parent array [B, M] (nullptr -> use tmask)
  int tpar_i64;
  int64_t tpar_sb, tpar_sm;
  const void* tmask;       // dense M x M mask block (float additive or byte keep)
  int tmask_dtype;         // dsv_dtype of tmask
  int64_t tm_sb, tm_sm, tm_sn;

  const int32_t* row_perm; // [M] node packing order (nullptr -> identity)

  uint16_t* opart;         // [S, B, Hk, R, D] bf16 partial outputs, normalised per split
  float2* ml;              // [S, B, Hk, R] (running max in log2 units, sum)
  int s_total;             // n_splits + has_tree
};

// Arguments of the LSE merge kernel (kernel 3).
struct MergeArgs {
  const uint16_t* opart;   // bf16, normalised per split
  const float2* ml;
  int s_total;
  int B, M, H, Hk, G, R, D;
  const int32_t* row_perm;
  void* out;               // [B, M, H, D] via strides
  int out_dtype;
  int64_t o_sb, o_sm, o_sh;
  float* lse;              // optional, natural-log LSE at (b, m, h)
  int64_t l_sb, l_sm, l_sh;
  const float* plse;       // optional prefix LSE -> weight = sigmoid(plse - lse)
  int64_t p_sb, p_sm, p_sh;
  void* weight;            // [B, M, H] via strides, dtype = wdtype
  int w_dtype;
  int64_t w_sb, w_sm, w_sh;
};

// Arguments of the acceptance kernels (kernel 4).
struct AcceptArgs {
  int mode;                // 0 greedy, 1 typical
  const void* logits;      // [T, M, V]
  int l_dtype;
  int64_t l_st, l_sm;      // tree, node strides (vocab stride 1)
  int T, M;
  int64_t V;
  int nchunk;              // vocab chunks per row
  int64_t chunk;           // elements per chunk
  const int64_t* draft; int64_t d_st, d_sm;
  const int64_t* parent; int64_t p_st, p_sm;
  const int64_t* pos; int64_t pos_st, pos_sm;
  int max_hops;
  float inv_temp, eps, alpha;
  float4* rstat;           // [T*M, nchunk] (argmax value, argmax index bits, m, l)
  float* rstat2;           // [T*M, nchunk] s = sum y*e^(y-m) (typical)
  int64_t* out_path; int64_t op_st;
  int64_t* out_tok; int64_t ot_st;
  int64_t* out_info; int64_t oi_st;
  int64_t* out_next; int64_t on_st;
  const float* xtok;       // optional [T*M] draft-token logits under the parent (fused lm_head)
  // Sampling (mode 2): warpers and the counter-based draw.
  float temperature;       // y = x / T rounded to the logits dtype (T == 1: y = x)
  uint32_t top_p_q;        // rint(top_p * 2^32); 0: no top-p
  int64_t top_k;           // 0: no top-k
  uint64_t seed;           // Philox key word 0
  uint4* sel;              // [T*M] kept-set bounds (top-k key, top-p key, top-p index); nullptr: keep all
  int cus;                 // compute units of the device (launch shapes); set by accept_chunking
};

// Arguments of the accepted-path KV commit.
constexpr int kCommitThreads = 256;
constexpr int kCommitChunks = 16;          // 16-byte chunks per thread: n * D * esize <= 64 KiB
struct CommitArgs {
  void* data;                // cache base (bf16/f16: esize 2, f32: esize 4)
  int esize;
  int64_t rows;              // cache rows moved independently
  int nlead;                 // leading dimensions decomposing a row index (<= 4)
  int64_t lead_shape[4], lead_stride[4];
  int64_t tok_stride;        // elements between tokens (within a page when paged)
  const void* pt;            // page table (nullptr: dense)
  int pt_i64;
  int ps_shift;
  int64_t page_stride, n_phys;
  int D;                     // elements per token row (innermost stride 1)
  int64_t start;             // first tree token
  int M;                     // tree nodes
  const int64_t* path;       // [M] accepted node ids (root first)
  const int64_t* info;       // info[3] = path length
};

// Arguments of the tree K/V append (+ RoPE).
struct AppendArgs {
  int f16;                   // 1: f16, 0: bf16
  int M, Hk, H, D;
  const uint16_t* k; int64_t k_sm, k_sh;   // [M, Hk, D] (token, head strides)
  const uint16_t* v; int64_t v_sm, v_sh;
  const uint16_t* q; int64_t q_sm, q_sh;   // optional [M, H, D]
  uint16_t* q_out; int64_t qo_sm, qo_sh;
  const uint16_t* cos; int64_t cs_m;       // optional [M, D] (nullptr: no RoPE)
  const uint16_t* sin; int64_t sn_m;
  uint16_t* k_dst; int64_t kd_sp, kd_sh, kd_st;  // page pool half [P, Hk, page, D] or dense [Hk, S, D]
  uint16_t* v_dst; int64_t vd_sp, vd_sh, vd_st;
  const void* pt;            // page table (nullptr: dense)
  int pt_i64, ps_shift;
  int64_t n_phys;
  int64_t start;             // logical token of tree node 0
};

// Arguments of the bundle order (query packing permutation) of B trees.
constexpr int kBundleMaxNodes = 1024;
constexpr int kBundleThreads = 256;        // lanes per workgroup at most (<= 4 nodes each)
struct BundleArgs {
  int B, M;
  const void* parent; int p_i64;           // [B, M] int32|int64
  int64_t p_st, p_sm;
  int bundle_size;                         // leaves per bundle (num_bundles == 0)
  int num_bundles;                         // > 0: bundle_size = ceil(leaves / num_bundles)
  int max_bundles;                         // bundles emitted (>= 1)
  int32_t* perm;                           // [B, M] node order
  int32_t* bundle_of;                      // optional [B, M] bundle of each node (-1: none)
};

// Arguments of the lm_head fused with the acceptance statistics.
constexpr int kLmThreads = 256;            // 4 waves
constexpr int kLmRB = 2;                   // 32-row vocabulary blocks per wave
constexpr int kLmKS = 4;                   // 16-element MFMA sub-steps per step
constexpr int kLmVocab = 128 * kLmRB;      // vocabulary rows per workgroup
constexpr int kLmRows = 64;                // hidden rows per pass over W
constexpr int kLmK = 16 * kLmKS;           // reduction elements per step
struct LmArgs {
  int mode;                                // 0 greedy, 1 typical
  const uint16_t* h; int64_t ldh;          // [R, Dm] bf16 hidden rows (row t*M + i)
  const uint16_t* w; int64_t ldw;          // [V, Dm] bf16 lm_head weight
  int R, Dm;
  int64_t V;
  int T, M;
  const int64_t* draft; int64_t d_st, d_sm;
  const int64_t* parent; int64_t p_st, p_sm;
  float inv_temp;
  int nblk;                                // vocabulary blocks = partial statistics per row
  float4* rstat; float* rstat2;            // [R, nblk] partial statistics
  float* xtok;                             // [R] draft-token logits under the parent (typical)
  uint16_t* lout; int64_t lo_sr;           // optional bf16 logits [R, V] (row stride)
};

// ---------------------------------------------------------------------------
// Launchers (defined in the .hip files, called by the C-ABI layer).
// ---------------------------------------------------------------------------
// ev0 / ev1 (may be null): timing events that take the kernel's own start and
// end times.
hipError_t launch_attn(const AttnArgs& a, int dtype, int D, bool dmask, hipStream_t s, hipEvent_t ev0 = nullptr,
                       hipEvent_t ev1 = nullptr);
// The fp32 variant (same plan, masks and partial format; dsv_attn_f32.hip).
hipError_t launch_attn_f32(const AttnArgs& a, int D, bool dmask, hipStream_t s, hipEvent_t ev0 = nullptr,
                           hipEvent_t ev1 = nullptr);
// What the host plan needs from the attention kernel's workgroup shape.
int attn_rows_per_block();
int attn_blocks_per_cu();
hipError_t launch_merge(const MergeArgs& a, hipStream_t s);
hipError_t launch_accept(const AcceptArgs& a, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1);
// Sampling mode: kept-set selection (top-p / top-k), the Gumbel-max draw per
// vocabulary range, then the walk.
hipError_t launch_sample(const AcceptArgs& a, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1);
// The walk of kernel 4 over the per-range statistics already in a.rstat.
hipError_t launch_walk(const AcceptArgs& a, hipStream_t s);
// Walk over per-row partial statistics part / part2 ([T*M, nin]) already
// computed (fused lm_head): combines them into a.rstat / a.rstat2 (one per
// row, a.nchunk == 1), then runs the walk.
// lm_head + statistics, then the combine and the walk of kernel 4.
hipError_t launch_lmhead_accept(const AcceptArgs& acc, const LmArgs& lm, hipStream_t s);
int lmhead_blocks(int64_t V);
hipError_t launch_accept_from_parts(const AcceptArgs& a, const float4* part, const float* part2, int nin,
                                    hipStream_t s);
hipError_t launch_commit(const CommitArgs& a, hipStream_t s);
hipError_t launch_append(const AppendArgs& a, hipStream_t s);
hipError_t launch_bundle_order(const BundleArgs& a, hipStream_t s);
// Vocabulary ranges of the acceptance statistics: sets a.chunk and a.nchunk
// from the logits layout, T, M, V and the GPU's CU count.
void accept_chunking(AcceptArgs& a, int cus);
// Upper bound of a.nchunk for a vocabulary of V (workspace sizing).
int64_t accept_max_chunks(int64_t V);

}  // namespace dsv
