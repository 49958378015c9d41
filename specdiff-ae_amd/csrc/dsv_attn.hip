// dsv_attn.hip — kernels 1 and 2 of the tree-verification path on gfx950.
//
// One workgroup owns (batch b, KV head kvh, block of 256 query rows, one key
// split).  The 256 rows are the G query heads x M tree nodes that share KV
// head kvh (GQA-native: K/V are never expanded), so every K/V tile staged in
// LDS feeds G*M query rows.  Key splits are either
//   * a prefix split: keys [s*kps, (s+1)*kps) of the prefix, all visible
//     (or filtered by a byte mask for the bundle-verifier contract), or
//   * the tree split: the M tree keys, filtered by an ancestor-or-self bitmask
//     built in LDS from the parent array (or from a dense mask block).
// Each split writes a normalised bf16 partial O and its (running max, sum);
// kernel 3 (dsv_merge.hip) combines the splits.
//
// Data movement per 32-key tile: K and V rows go HBM -> LDS by LDS-DMA
// (buffer_load_dwordx4 ... lds), one 1 KiB wave-instruction per 4 keys, into
// a 4-stage LDS ring (two tiles being consumed, two in flight; the ring stays
// below 64 KiB).  Each lane's global chunk is chosen so that the LDS
// image is XOR-swizzled for conflict-free operand reads.  The fast path
// resolves the page once per instruction into a scalar base wrapped in a
// buffer resource whose range ends at the tensor's end, so the hardware
// bounds-checks every lane.  Address arithmetic lives in dsv_attn_geo.h and
// is shared with the host-side emulation used by the dry-run mode.
//
// Math per tile, per wave of 32 rows:
//   S^T[key, row] = K[key, :] . Q[row, :]      v_mfma_f32_32x32x16_{bf16,f16}
//   P = exp2(S * log2(e)/sqrt(D) - m_row)      online softmax, lazy rescale
//   O^T[d, row]  += V^T[d, key] . P^T[key,row] v_mfma_f32_32x32x16_{bf16,f16}
// S^T (keys on the MFMA M side) leaves each lane one query row and 16 keys:
// exactly the B-operand layout of the P.V product, so P stays in registers;
// the V^T A-operand comes straight from row-major V in LDS through
// ds_read_b64_tr_b16 (16-lane block transpose).
//
// Reference semantics followed: runtime/tree_attention.py:116-217 (prefix
// O + LSE with an online softmax), :220-292 (tree block), :40-63 (naive tree
// attention), runtime/bundle_verifier.py:26-135 (masked bundle attention).

#include <hip/hip_ext.h>

#include "dsv_attn_geo.h"
#include "dsv_dma.h"
#include "dsv_internal.h"

namespace dsv {

namespace {

constexpr float kNegInf = -__builtin_huge_valf();
// Lazy-rescale threshold in log2 units: the running max used for the
// exponentials may lag the true max by up to this much (p <= 2^8).
constexpr float kRescaleTau = 8.0f;
// Tiles after the first skip their maximum unless a lane's probabilities sum
// above 2^kSumTau: every probability then stays below 2^kSumTau.
constexpr float kSumBound = 65536.0f;  // 2^kSumTau, kSumTau = 16

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

template <typename T>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c);

template <>
__device__ __forceinline__ f32x16 mfma32<BF16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16 mfma32<F16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Pack two fp32 values into one dword of two 16-bit values (lo, hi), RNE.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack2<BF16>(float lo, float hi) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  bf2 r = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, r);
}
template <>
__device__ __forceinline__ uint32_t pack2<F16>(float lo, float hi) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  h2 r = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, r);
}

// Combine a value with the one held by lane (lane ^ 32).
__device__ __forceinline__ float xor32_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __builtin_elementwise_maximum(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }

__device__ __forceinline__ int64_t load_index(const void* p, int is64, int64_t i) {
  return is64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t) reinterpret_cast<const int32_t*>(p)[i];
}


// LDS-DMA: 16 bytes per lane, lane l lands at LDS m0 + 16*l.  K/V bytes are
// read once per verify step: the loads are marked non-temporal (nt).
// Through a buffer resource (hardware range check; out-of-range lanes read 0).
__device__ __forceinline__ void dma_buf(uint32_t lds, const void* base, uint32_t range, uint32_t voff) {
  const uint64_t p = (uint64_t)base;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)p);
  r[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)(p >> 32));
  r[2] = __builtin_amdgcn_readfirstlane((int)range);
  r[3] = 0x00020000;
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds" ::"s"(m0), "v"(voff), "s"(r)
               : "memory", "m0");
}
// With a full per-lane address (keys clamped to valid ones by the caller).
__device__ __forceinline__ void dma_lane(uint32_t lds, const void* vaddr) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off nt" ::"s"(m0), "v"(vaddr) : "memory", "m0");
}


// Does element (i, j) of a dense tree-mask block keep the key?
__device__ __forceinline__ bool tmask_keep(const AttnArgs& a, int b, int i, int j) {
  const int64_t off = b * a.tm_sb + i * a.tm_sm + j * a.tm_sn;
  switch (a.tmask_dtype) {
    case 2: return reinterpret_cast<const float*>(a.tmask)[off] == 0.0f;            // f32 additive
    case 0:                                                                          // bf16 additive
    case 1: return (reinterpret_cast<const uint16_t*>(a.tmask)[off] & 0x7fff) == 0;  // f16 additive (+-0 keep)
    default: return reinterpret_cast<const uint8_t*>(a.tmask)[off] != 0;             // int8/uint8/bool
  }
}

enum KernelMode : int { kModeAny = 0, kModeF32Paged = 1, kModeF32Dense = 2 };

// A compile-time integer: the ring stage of an unrolled loop step, so that
// every LDS address of the stage folds into an instruction offset.
template <int N>
struct IC {
  static constexpr int value = N;
};

// Row maximum of a lane's 16 scores (NaN-propagating, like torch.max;
// v_maximum3_f32 on gfx950).
__device__ __forceinline__ float max16(const f32x16& s) {
  float m = __builtin_elementwise_maximum(s[0], s[1]);
#pragma unroll
  for (int v = 2; v < 16; ++v) m = __builtin_elementwise_maximum(m, s[v]);
  return m;
}

// One workgroup = 8 waves x 32 query rows (two waves per SIMD).
//
// Software pipeline per wave: iteration t owns the scores S(t), already
// computed.  It waits for tile t+1 (two tiles stay in flight), then runs
// the softmax of S(t) on the VALU while the MFMA pipe computes S(t+1) from
// tile t+1's K, and finally O += V(t)^T P(t)^T.  Ring stage of tile t: t & 3;
// tile t+3 goes into stage (t+3) & 3, whose previous tile (t-1) every wave has
// finished with once the barrier of iteration t is passed.
// MODE: kModeF32Paged / kModeF32Dense when both sources are known to use
// 32-bit DMA offsets (the host checks), else kModeAny (per-source choice at
// run time).
// BIG: trees of more than kTreeNodeM nodes (the tree split's visibility table
// indexed by packed row instead of node).
template <typename T, int D, bool DMASK, int MODE, bool BIG = false>
__global__ void __launch_bounds__(512, 2) attn_splitk_kernel(const AttnArgs a) {
  using G = Geo<D>;
  constexpr int NW = 8;
  constexpr int NT = NW * 64;
  constexpr int KT = G::KT;
  constexpr int KS = D / 16;                   // k-steps of the Q.K^T product
  constexpr int DT = D / 32;                   // 32-row d tiles of the P.V product
  constexpr int CH = G::CH;
  constexpr int IPW = 2 * G::NINS / NW;        // DMA instructions per wave per tile
  static_assert(IPW * NW == 2 * G::NINS, "tile DMA must split evenly over waves");
  static_assert(G::STAGES == 4, "the loop is unrolled over a 4-stage ring");
  constexpr int PT_OFF = G::RING;
  constexpr int VIS_OFF = PT_OFF + kPageLds * 4;
  constexpr int VIS_W = BIG ? kTreeMaxW : kTreeNodeW;  // words per table entry
  constexpr int LDS_BYTES = VIS_OFF + (BIG ? kTreeSlots : kTreeNodeM) * VIS_W * 8;

  // One LDS allocation so that the DMA ring sits at offset 0 (addresses < 64 KiB).
  __shared__ __attribute__((aligned(1024))) uint8_t smem[LDS_BYTES];
  int32_t* pt_lds = reinterpret_cast<int32_t*>(smem + PT_OFF);
  uint64_t* vis_lds = reinterpret_cast<uint64_t*>(smem + VIS_OFF);

  const int tid = threadIdx.x;
  // The wave index is uniform: readfirstlane lets every address derived from it
  // live in SGPRs (scalar math) instead of being replicated per lane.
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, lj = lane & 31, lg = lane >> 5;

  // Block -> work item.  Dispatch ids go round-robin over the 8 XCDs; remap
  // so that neighbouring work items (row blocks of one split) share an XCD.
  const int nblk = gridDim.x;
  int w = ((nblk & 7) == 0) ? (blockIdx.x & 7) * (nblk >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const int rb = w % a.n_rb;
  w /= a.n_rb;
  const int split = w % a.s_total;
  w /= a.s_total;
  const int kvh = w % a.Hk;
  const int b = w / a.Hk;
  const bool is_tree = a.has_tree && split == a.n_splits;
  const KvSrc src = is_tree ? a.tree : a.pre;

  // This batch's prefix length (flash-attn cache_seqlens), clamped to [0, n_pre].
  int64_t n_pre_b = a.n_pre;
  if (a.seqlens != nullptr) {
    n_pre_b = load_index(a.seqlens, a.seqlens_i64, b);
    n_pre_b = n_pre_b < 0 ? 0 : (n_pre_b > a.n_pre ? a.n_pre : n_pre_b);
  }
  int64_t kstart, kend;
  if (is_tree) {
    kstart = 0;
    kend = a.M;
  } else {
    kstart = (int64_t)split * a.kps;
    kend = min(kstart + a.kps, n_pre_b);
  }
  const int64_t nkeys = kend - kstart;
  const int ntiles = nkeys > 0 ? (int)((nkeys + KT - 1) / KT) : 0;
  const int nfull = nkeys > 0 ? (int)(nkeys / KT) : 0;  // tiles without tail keys
  // Causal prefix (bottom-right aligned): row m sees keys n <= c0 + m with
  // c0 = len - M.  Tiles below nvis are visible to every row.
  const bool causal = a.causal != 0 && !is_tree;
  const int64_t c0 = n_pre_b - a.M;
  int nvis = nfull;
  if (causal) {
    const int64_t v = c0 + 1 - kstart;
    nvis = v <= 0 ? 0 : (int)min((int64_t)nfull, v / KT);
  }
  const bool paged = MODE == kModeF32Paged || (MODE == kModeAny && src.pt != nullptr);
  const int mode = MODE == kModeAny ? dma_mode<D>(src) : (int)kFast32;

  // ---- set-up: page-table slice, tree bitmask --------------------------------
  int64_t pt_lo = 0, pt_hi = -1;
  if (paged && ntiles > 0) {
    pt_lo = (src.key0 + kstart) >> src.ps_shift;
    pt_hi = (src.key0 + kend - 1) >> src.ps_shift;
    for (int64_t i = tid; i <= pt_hi - pt_lo; i += NT)
      pt_lds[i] = (int32_t)clamp_page(load_index(src.pt, src.pt_i64, b * src.pt_sb + pt_lo + i), src.n_phys);
  }
  if (is_tree) {
    const int M = a.M;
    // The parent array is staged in the DMA ring, idle until the first tile
    // is issued after the barrier that ends the set-up: the ancestor walks
    // then hop through LDS instead of chains of dependent global loads.
    static_assert(kTreeMaxM * 4 <= G::RING, "parent staging fits the ring");
    int32_t* par_lds = reinterpret_cast<int32_t*>(smem);
    if (a.tpar != nullptr) {
      for (int i = tid; i < M; i += NT)
        par_lds[i] = (int32_t)load_index(a.tpar, a.tpar_i64, b * a.tpar_sb + i * a.tpar_sm);
      __syncthreads();
    }
    // Entry e of the table: the ancestor-or-self bits of node e (up to
    // kTreeNodeM nodes), or, with BIG, of the node of this workgroup's packed
    // row e (0 <= e < 256, row = 256 * rb + e, node slot mi = row mod M).
    const int n_ent = BIG ? min(kTreeSlots, a.R - rb * (NW * 32)) : M;
    for (int e = tid; e < n_ent; e += NT) {
      int i = e;
      if constexpr (BIG) {
        const int mi = (rb * (NW * 32) + e) % M;
        // A permutation entry outside [0, M) is clamped, as for the Q rows.
        i = a.row_perm ? min(max(a.row_perm[mi], 0), M - 1) : mi;
      }
      uint64_t wd[VIS_W];
#pragma unroll
      for (int x = 0; x < VIS_W; ++x) wd[x] = 0;
      if (a.tpar != nullptr) {
        int node = i;
        for (int step = 0; step < M && node >= 0 && node < M; ++step) {
#pragma unroll
          for (int x = 0; x < VIS_W; ++x)
            if ((node >> 6) == x) wd[x] |= 1ull << (node & 63);
          const int p = par_lds[node];
          if (p == node) break;
          node = p;
        }
      } else {
        for (int j = 0; j < M; ++j) {
          if (tmask_keep(a, b, i, j)) {
#pragma unroll
            for (int x = 0; x < VIS_W; ++x)
              if ((j >> 6) == x) wd[x] |= 1ull << (j & 63);
          }
        }
      }
#pragma unroll
      for (int x = 0; x < VIS_W; ++x) vis_lds[e * VIS_W + x] = wd[x];
    }
  }
  __syncthreads();

  // ---- DMA issue of one tile into its ring stage ------------------------------
  // Instruction i covers keys [j*KPI, (j+1)*KPI) of the tile's K or V; lane p
  // fills LDS bytes [16p, 16p+16) of that KiB = key j*KPI + p/CH, slot p%CH,
  // which holds global chunk slot ^ swizzle(key).  In a full tile the lane's
  // byte offset from the instruction's base key does not change from tile to
  // tile: it is computed once.
  const int kii = lane / CH;
  const int slot = lane % CH;
  uint32_t voff_full[IPW];
#pragma unroll
  for (int x = 0; x < IPW; ++x) {
    bool is_v;
    int j;
    dma_ins<D>(wid * IPW + x, is_v, j);
    const int key_t = j * G::KPI + kii;
    const int c = is_v ? v_slot(CH, key_t, slot) : k_slot(CH, key_t, slot);
    voff_full[x] = (uint32_t)(fast_lane_elem(src, is_v, 0, kii, c) * 2);
  }
  // Waves [0, NW/2) issue the K half of each tile's DMA, the others the V
  // half (NINS is a multiple of IPW, so no wave issues both).
  const bool dma_v = wid >= NW / 2;
  // kFast32: the buffer resource of this wave's half for this workgroup,
  // built once.
  i32x4 rs = i32x4{0, 0, 0, 0};
  if (mode == kFast32) {
    const int64_t wb = wg_base_elem(src, dma_v, b, kvh);
    rs = make_rsrc((dma_v ? src.v : src.k) + wb, rsrc_range(dma_v ? src.v_bytes : src.k_bytes, wb));
  }
  // Page window (32-bit paged mode): lane l of pgw[x] holds the byte offset,
  // from the workgroup's buffer base, of this wave's DMA instruction x in full
  // tile pgw_t0 + l (physical page * page stride + key-in-page * key stride),
  // so that a tile's address costs one lane read instead of an LDS round trip
  // and its scalar arithmetic.  The window is refilled from the LDS page-table
  // slice once per 64 tiles; windows start at tile 0 and every 64th tile, all
  // multiples of 4, so only ring stage 0 can start one.
  uint32_t pgw[IPW];
  int pgw_t0 = -64;
#pragma unroll
  for (int x = 0; x < IPW; ++x) pgw[x] = 0;
  auto fill_pgw = [&](int t0) {
    pgw_t0 = t0;
    const int last = (int)(pt_hi - pt_lo);
#pragma unroll
    for (int x = 0; x < IPW; ++x) {
      bool is_v;
      int j;
      dma_ins<D>(wid * IPW + x, is_v, j);
      const uint32_t nb = (uint32_t)(src.key0 + kstart) + (uint32_t)(t0 + lane) * KT + (uint32_t)(j * G::KPI);
      const int e = min((int)(nb >> src.ps_shift) - (int)pt_lo, last);  // lanes past the split: any valid entry
      pgw[x] = tile_off32_s(true, (uint32_t)(2 * (is_v ? src.v_st : src.k_st)), (uint32_t)(2 * (is_v ? src.v_sp : src.k_sp)),
                            (1u << src.ps_shift) - 1u, nb, (uint32_t)pt_lds[e]);
    }
  };

  // 32-bit modes: this wave's half (K or V) byte strides, uniform.
  const uint32_t key0_32 = (uint32_t)(src.key0 + kstart);
  const uint32_t st2 = (uint32_t)__builtin_amdgcn_readfirstlane((int)(2 * (dma_v ? src.v_st : src.k_st)));
  const uint32_t sp2 = (uint32_t)__builtin_amdgcn_readfirstlane((int)(2 * (dma_v ? src.v_sp : src.k_sp)));
  const uint32_t psm = (1u << src.ps_shift) - 1u;
  KvSrc s32 = src;
  if (MODE == kModeF32Dense) s32.pt = nullptr;

  auto issue_tile = [&](auto stage_c, int t) {
    constexpr int stage = decltype(stage_c)::value;
    if (MODE != kModeAny && t < nfull) {
      // Full tile in a 32-bit mode: the lane offsets of voff_full plus the
      // tile's offset (from the window when paged).
      if (MODE == kModeF32Paged && stage == 0 && t - pgw_t0 >= 64) fill_pgw(t);
      const uint32_t nbt = key0_32 + (uint32_t)t * KT;
#pragma unroll
      for (int x = 0; x < IPW; ++x) {
        bool is_v;
        int j;
        dma_ins<D>(wid * IPW + x, is_v, j);
        const uint32_t dst = lds_addr(smem + (stage * 2 + (is_v ? 1 : 0)) * G::TILE + j * 1024);
        const uint32_t toff = MODE == kModeF32Paged ? (uint32_t)__builtin_amdgcn_readlane((int)pgw[x], t - pgw_t0)
                                                    : tile_off32_s(false, st2, sp2, psm, nbt + (uint32_t)(j * G::KPI), 0u);
        dma_rs(dst, rs, voff_full[x] + toff);
      }
      return;
    }
    const int64_t kb = kstart + (int64_t)t * KT;
    const bool full = t < nfull;
#pragma unroll
    for (int x = 0; x < IPW; ++x) {
      bool is_v;
      int j;
      dma_ins<D>(wid * IPW + x, is_v, j);
      const int key_t = j * G::KPI + kii;  // key within the tile
      const uint32_t dst = lds_addr(smem + (stage * 2 + (is_v ? 1 : 0)) * G::TILE + j * 1024);
      const uint16_t* base = is_v ? src.v : src.k;
      if (MODE != kModeAny || mode == kFast32) {
        // Keys fit in 31 bits in this mode: per-tile arithmetic is 32-bit scalar.
        const int kb32 = (int)(src.key0 + kb);
        uint32_t nb = (uint32_t)(kb32 + j * G::KPI);
        uint32_t vo = voff_full[x];
        if (!full) {
          const int64_t nb64 = fast_base_key(src, kb, kend, j, G::KPI);
          const int c = is_v ? v_slot(CH, key_t, slot) : k_slot(CH, key_t, slot);
          vo = (uint32_t)(fast_lane_elem(src, is_v, nb64, fast_lane_key(src, kb, kend, j, G::KPI, kii), c) * 2);
          nb = (uint32_t)nb64;
        }
        const uint32_t page =
            paged ? (uint32_t)__builtin_amdgcn_readfirstlane(pt_lds[(int)(nb >> src.ps_shift) - (int)pt_lo]) : 0u;
        dma_rs(dst, rs, vo + tile_off32(s32, is_v, nb, page));
      } else if (mode == kFast) {
        const int64_t nb = fast_base_key(src, kb, kend, j, G::KPI);
        const int64_t page = paged ? __builtin_amdgcn_readfirstlane(pt_lds[(nb >> src.ps_shift) - pt_lo]) : 0;
        const int64_t be = src_elem(src, is_v, b, kvh, nb, page, 0);
        uint32_t vo = voff_full[x];
        if (!full) {
          const int c = is_v ? v_slot(CH, key_t, slot) : k_slot(CH, key_t, slot);
          vo = (uint32_t)(fast_lane_elem(src, is_v, nb, fast_lane_key(src, kb, kend, j, G::KPI, kii), c) * 2);
        }
        dma_buf(dst, base + be, rsrc_range(is_v ? src.v_bytes : src.k_bytes, be), vo);
      } else {
        const int c = is_v ? v_slot(CH, key_t, slot) : k_slot(CH, key_t, slot);
        const int64_t n = lane_key(src, kb, kend, key_t);
        const int64_t page = paged ? pt_lds[(n >> src.ps_shift) - pt_lo] : 0;
        dma_lane(dst, base + src_elem(src, is_v, b, kvh, n, page, c));
      }
    }
  };

  // ---- this wave's query rows: Q fragments (B operand of S^T = K.Q^T) --------
  // lane (row lj, group lg) holds Q[row, 16*ks + 8*lg .. +8].
  const int row0 = rb * (NW * 32) + wid * 32;
  const bool wave_active = row0 < a.R;
  const int r_me = row0 + lj;
  const bool rvalid = r_me < a.R;
  u32x4 qf[KS];
  int node_of = 0;
  if (rvalid) {
    const int g = r_me / a.M;
    const int mi = r_me - g * a.M;
    // A permutation entry outside [0, M) is clamped: no access leaves q.
    const int m = a.row_perm ? min(max(a.row_perm[mi], 0), a.M - 1) : mi;
    node_of = m;
    const uint16_t* qp = a.q + b * a.q_sb + (int64_t)m * a.q_sm + (int64_t)(kvh * a.G + g) * a.q_sh + lg * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = ld16(qp + ks * 16);
  } else {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = u32x4{0, 0, 0, 0};
  }

  // Score scale (log2 units), a kernel argument held in an SGPR for the loop.
  const float scale_log2 = a.scale_log2;

  f32x16 acc[DT];
  float mx = kNegInf, lsum = 0.f;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16{};

  // Per-lane LDS byte offsets of the operand reads within a tile (the stage
  // part is a compile-time offset).
  //   K (A operand of S^T): key lj, chunk 2*ks + lg.
  //   V^T (two transposed reads per d tile): 16-lane block bl = lane/16 holds
  //   d rows [16*(bl&1), +16) of a 32-row d tile and key group g = bl>>1;
  //   lane i of the block addresses key row 16*hh + 4*g + i/4 (+8 for the
  //   second read), columns d0 + 4*(i%4) .. +3.
  uint32_t koff[KS], voff[DT];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) koff[ks] = lj * (2 * D) + k_slot(CH, lj, 2 * ks + lg) * 16;
  {
    const int bl = lane >> 4, bi = lane & 15;
    const int vkey = 4 * (bl >> 1) + (bi >> 2);
    const int vcol = 16 * (bl & 1) + 4 * (bi & 3);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int col = dt * 32 + vcol;
      // (vkey + 16*hh + 8*e) & 3 == vkey & 3: the swizzle is the same for all
      // four reads of a d tile.
      voff[dt] = vkey * (2 * D) + v_slot(CH, vkey, col >> 3) * 16 + (col & 7) * 2;
    }
  }

  // Keep mask of the scores of tile t (tail keys, tree visibility, byte mask).
  // Bit v of a lane <-> key 4*lg + 8*(v/4) + v%4 of the tile.
  auto mask_scores = [&](f32x16& s, int t) {
    const int64_t kb = kstart + (int64_t)t * KT;
    const int64_t ke = causal ? min(kend, c0 + 1 + node_of) : kend;  // this row's key end
    const int lim = (int)max(min(ke - kb, (int64_t)KT), (int64_t)-KT) - 4 * lg;  // valid keys from 4*lg
    uint32_t keep = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = min(max(lim - 8 * q, 0), 4);  // valid keys among 8q .. 8q+3
      keep |= ((1u << c) - 1u) << (4 * q);
    }
    if (is_tree) {
      // Visibility bits of this tile's keys, shifted to this lane's keys.
      const int ent = BIG ? wid * 32 + lj : node_of;
      const uint64_t vw = rvalid ? vis_lds[ent * VIS_W + (t >> 1)] : 0ull;
      const uint32_t vb = (uint32_t)(vw >> ((t & 1) * 32 + 4 * lg));
      keep &= (vb & 0xFu) | ((vb >> 4) & 0xF0u) | ((vb >> 8) & 0xF00u) | ((vb >> 12) & 0xF000u);
    }
    if constexpr (DMASK) {
      const uint8_t* mrow = a.dmask + (int64_t)b * a.dm_sb + (int64_t)node_of * a.dm_sm;
      const int64_t n0 = kb + 4 * lg;
      uint32_t mb = 0;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t n = n0 + 8 * (v >> 2) + (v & 3);
        mb |= (uint32_t)((n < a.dm_n) && (mrow[n * a.dm_sn] != 0)) << v;
      }
      keep &= rvalid ? mb : 0u;
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) s[v] = ((keep >> v) & 1u) ? s[v] : kNegInf;
  };

  // ---- ping-pong schedule ------------------------------------------------------
  // Waves [0, NW/2) issue the K half of every tile's DMA, waves [NW/2, NW) the
  // V half; tile t lives in ring stage t & 3 of the K and V rings.  QK(t) reads
  // K(t) one interval before PV(t) reads V(t), so K is issued three tiles
  // ahead and V two: barrier j (one per interval) follows the waits for
  // K(j+1) and V(j), after it nothing reads K(j-1) or V(j-2) any more, and
  // K(j+3) / V(j+2) go into those stages.  Two tiles of each stay in flight.
  //
  // Every wave runs, per tile k, Y_k (softmax of S(k) -> P(k), VALU) and then
  // X_k (S(k+1) = QK(k+1) and O += PV(k), MFMA).  K waves meet barrier k
  // before Y_k, V waves meet barrier k+1 between Y_k and X_k: on each SIMD one
  // wave is in its MFMA phase while the other is in its VALU phase.
  const bool v_wave = wid >= NW / 2;
  static_assert(2 * G::NINS / IPW == NW && G::NINS % IPW == 0, "K and V DMA halves map to wave halves");

  // The barrier of step k (barrier k for K waves, before Y_k; barrier k+1
  // for V waves, before X_k), the wait before it and this wave's DMA issue
  // after it.  K waves: K(k+1) must have landed, K(k+2) may be in flight, and
  // K(k+3) is issued.  V waves: V(k+1) must have landed, V(k+2) may be in
  // flight, and V(k+3) is issued.  Either way: tile k+3 into stage (k+3) & 3.
  auto sync = [&](auto stage3_c, int k) {
    if (k + 2 < ntiles)
      wait_vmcnt<IPW>();
    else
      wait_vmcnt<0>();
    barrier_lds();
    if (k + 3 < ntiles) issue_tile(stage3_c, k + 3);
  };

  f32x16 s_cur = f32x16{};
  auto read_k = [&](auto stage_c, u32x4 (&kf)[KS]) {
    constexpr int stage = decltype(stage_c)::value;
    const uint8_t* kt = smem + stage * 2 * G::TILE;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kf[ks] = *reinterpret_cast<const u32x4*>(kt + koff[ks]);
  };
  // V^T operands of half hh (keys 16*hh .. 16*hh+15) of a tile.
  auto read_vh = [&](auto stage_c, int hh, u32x4 (&vf)[2][DT]) {
    constexpr int stage = decltype(stage_c)::value;
    const uint8_t* vt = smem + (stage * 2 + 1) * G::TILE;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const uint8_t* p = vt + voff[dt] + hh * 16 * (2 * D);
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p);
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p + 8 * (2 * D)));
      const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
      vf[hh][dt] = u32x4{l2[0], l2[1], h2[0], h2[1]};
    }
  };

  // Tile k in ring stage S (k & 3 == S).
  auto step = [&](auto stage_c, int k) {
    constexpr int S = decltype(stage_c)::value;
    if (!v_wave && k > 0) sync(IC<(S + 3) & 3>{}, k);
    u32x4 kf[KS], vf[2][DT];
    u32x4 pk[2];
    if (wave_active) {
      // Operands of X_k, read now so that their latency hides behind Y_k
      // (past the last tile K(k+1) is a stale stage whose product is unused).
      // The V^T reads are spread over the two halves of the exponentials so
      // that the LDS burst after the barrier is shorter.
      read_k(IC<(S + 1) & 3>{}, kf);

      // ---- Y_k: online softmax of S(k) (log2 domain, lazy rescale) ----------
      // The exponentials run against the lagging row maximum mx.  The tile's
      // own maximum is taken only where mx is not known yet or the tile is
      // masked; on other tiles a score above mx + kSumTau shows as a lane's
      // sum of this tile's probabilities above 2^kSumTau (inf included), and
      // only then is the tile redone against its maximum.
      const bool masked = is_tree || DMASK || k >= nvis;
      if (masked) mask_scores(s_cur, k);
      auto rescale = [&]() {
        const float mt = xor32_max(max16(s_cur)) * scale_log2;
        if (__ballot(mt > mx + kRescaleTau) != 0ull) {
          const float mn = __builtin_elementwise_maximum(mx, mt);
          const float al = (mn == mx) ? 1.f : __builtin_amdgcn_exp2f(mx - mn);
          mx = mn;
          lsum *= al;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) acc[dt] *= al;
        }
      };
      if (masked || __ballot(mx == kNegInf) != 0ull) rescale();
      auto exps = [&](bool with_v) {
        const float ms = (mx == kNegInf) ? 0.f : mx;
        float ts = 0.f;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          if (with_v) {
            __builtin_amdgcn_sched_barrier(0);
            read_vh(IC<S>{}, hh, vf);
            __builtin_amdgcn_sched_barrier(0);
          }
          uint32_t w4[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float p0 = __builtin_amdgcn_exp2f(fmaf(s_cur[hh * 8 + 2 * e], scale_log2, -ms));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(s_cur[hh * 8 + 2 * e + 1], scale_log2, -ms));
            w4[e] = pack2<T>(p0, p1);
            // The normaliser sums the unrounded probabilities: the LSE is an
            // output in its own right and keeps fp32 accuracy.
            ts += p0 + p1;
          }
          pk[hh] = u32x4{w4[0], w4[1], w4[2], w4[3]};
        }
        return ts;
      };
      float ts = exps(true);
      if (!masked && __ballot(!(ts <= kSumBound)) != 0ull) {
        rescale();
        ts = exps(false);
      }
      lsum += ts;
    }
    if (v_wave) sync(IC<(S + 3) & 3>{}, k);
    if (wave_active) {
      // ---- X_k: S(k+1) = K(k+1) . Q^T, then O^T += V(k)^T . P(k)^T ----------
      f32x16 sn = f32x16{};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) sn = mfma32<T>(kf[ks], qf[ks], sn);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] = mfma32<T>(vf[hh][dt], pk[hh], acc[dt]);
      s_cur = sn;
    }
  };

  // ---- prologue: K(0..2) and V(0..1) issued, barrier 0, S(0) ---------------------
  if (ntiles > 0) issue_tile(IC<0>{}, 0);
  if (ntiles > 1) issue_tile(IC<1>{}, 1);
  if (ntiles > 2 && !v_wave) issue_tile(IC<2>{}, 2);
  // The Q fragments must be complete before the loop.  The compiler counts
  // only its own loads (the DMA is inline asm): left to itself it would place
  // the Q waits at their first use inside the loop, where each one waits for
  // every DMA in flight, on every tile.  Using the fragments here puts those
  // waits before the loop.  They need not cover the DMA (the compiler may
  // count spill stores issued after the Q loads): the tiles are waited for
  // explicitly.
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) asm volatile("" ::"v"(qf[ks]));
  // The same holds for the scalar load of the score scale: the counter that
  // tracks it also tracks the LDS operand reads, so a first wait inside the
  // loop would wait for every operand read of the tile, ahead of the softmax
  // that is meant to hide their latency.
  asm volatile("" ::"s"(scale_log2));
  if (ntiles > 0) {
    // Barrier 0: K(0), K(1) and V(0) landed (K(2) and V(1) may stay in flight).
    if (v_wave ? ntiles > 1 : ntiles > 2)
      wait_vmcnt<IPW>();
    else
      wait_vmcnt<0>();
    barrier_lds();
    if (v_wave) {
      if (ntiles > 2) issue_tile(IC<2>{}, 2);
    } else {
      if (ntiles > 3) issue_tile(IC<3>{}, 3);
    }
    if (wave_active) {
      u32x4 kf[KS];
      read_k(IC<0>{}, kf);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) s_cur = mfma32<T>(kf[ks], qf[ks], s_cur);
    }
  }
  for (int t0 = 0; t0 < ntiles; t0 += 4) {
    step(IC<0>{}, t0);
    if (t0 + 1 < ntiles) step(IC<1>{}, t0 + 1);
    if (t0 + 2 < ntiles) step(IC<2>{}, t0 + 2);
    if (t0 + 3 < ntiles) step(IC<3>{}, t0 + 3);
  }
  // K waves meet the last barrier (V waves met it after Y of the last tile).
  if (ntiles > 0 && !v_wave) {
    wait_vmcnt<0>();
    barrier_lds();
  }

  // ---- epilogue: normalised bf16 partial + (max, sum) per row ----------------
  // After this barrier no wave reads the ring any more.  Each wave stages its
  // 32 partial rows there (16-byte chunks XOR-swizzled by row, against bank
  // conflicts) and writes its contiguous block of rows with whole 16-byte
  // lanes: one KiB of consecutive bytes per store instruction.
  __syncthreads();
  if (!wave_active) return;
  const float ltot = xor32_sum(lsum);
  const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
  constexpr int CHR = D / 8;  // 16-byte chunks per row
  static_assert(NW * 32 * D * 2 <= G::RING, "the partial rows of all waves fit the ring");
  uint8_t* stage = smem + wid * (32 * D * 2);
  // Accumulator value v of d tile dt holds d = 32*dt + 8*(v/4) + 4*lg + v%4.
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const f32x16 x = acc[dt];
      const u32x2 val = {pack2<BF16>(x[4 * q4] * inv, x[4 * q4 + 1] * inv),
                         pack2<BF16>(x[4 * q4 + 2] * inv, x[4 * q4 + 3] * inv)};
      const int c = 4 * dt + q4;
      *reinterpret_cast<u32x2*>(stage + lj * (2 * D) + ((c ^ (lj % CHR)) * 16) + 8 * lg) = val;
    }
  }
  // Each lane now reads 16-byte chunks that other lanes of this wave wrote:
  // order the reads after the writes explicitly (wave-scope release, wave
  // barrier, acquire), so no compiler reordering can move them ahead.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int64_t pbase = (((int64_t)split * a.B + b) * a.Hk + kvh) * a.R + row0;
  uint16_t* op = a.opart + pbase * D;
  // All of the lane's chunks are read from LDS first (one wait), then stored.
  u32x4 chunk[CHR / 2];
#pragma unroll
  for (int k = 0; k < CHR / 2; ++k) {
    const int f = k * 64 + lane, r = f / CHR, i = f % CHR;
    chunk[k] = *reinterpret_cast<const u32x4*>(stage + r * (2 * D) + ((i ^ (r % CHR)) * 16));
  }
#pragma unroll
  for (int k = 0; k < CHR / 2; ++k) {
    const int f = k * 64 + lane, r = f / CHR, i = f % CHR;
    if (row0 + r < a.R) *reinterpret_cast<u32x4*>(op + (int64_t)r * D + i * 8) = chunk[k];
  }
  if (rvalid && lg == 0) a.ml[pbase + lj] = make_float2(mx, ltot);
}

// A launch with timing events records them from the kernel's own dispatch
// packet (its start and end), so their interval is the kernel's execution
// time; without events it is a plain launch.
template <typename K>
hipError_t launch_k(K kernel, dim3 grid, dim3 block, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1,
                    const AttnArgs& a) {
  if (ev0 != nullptr || ev1 != nullptr)
    hipExtLaunchKernelGGL(kernel, grid, block, 0, s, ev0, ev1, 0, a);
  else
    hipLaunchKernelGGL(kernel, grid, block, 0, s, a);
  return hipGetLastError();
}

template <typename T, int D, bool DMASK>
hipError_t launch_t(const AttnArgs& a, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  const int64_t nblk = (int64_t)a.B * a.Hk * a.s_total * a.n_rb;
  if (nblk <= 0) return hipSuccess;
  // Both sources in 32-bit mode and of one kind: the specialised kernel.
  const int mp = dma_mode<D>(a.pre), mt = a.has_tree ? dma_mode<D>(a.tree) : mp;
  const bool pp = a.pre.pt != nullptr, tp = a.has_tree ? a.tree.pt != nullptr : pp;
  const dim3 grid((unsigned)nblk), block(512);
  if constexpr (!DMASK) {
    if (mp == kFast32 && mt == kFast32 && pp == tp && !(a.has_tree && a.M > kTreeNodeM)) {
      if (pp) return launch_k(attn_splitk_kernel<T, D, DMASK, kModeF32Paged>, grid, block, s, ev0, ev1, a);
      return launch_k(attn_splitk_kernel<T, D, DMASK, kModeF32Dense>, grid, block, s, ev0, ev1, a);
    }
  }
  if constexpr (!DMASK) {
    if (a.has_tree && a.M > kTreeNodeM)
      return launch_k(attn_splitk_kernel<T, D, DMASK, kModeAny, true>, grid, block, s, ev0, ev1, a);
  }
  return launch_k(attn_splitk_kernel<T, D, DMASK, kModeAny>, grid, block, s, ev0, ev1, a);
}

template <typename T, bool DMASK>
hipError_t launch_d(const AttnArgs& a, int D, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  switch (D) {
    case 64: return launch_t<T, 64, DMASK>(a, s, ev0, ev1);
    case 128: return launch_t<T, 128, DMASK>(a, s, ev0, ev1);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

int attn_rows_per_block() { return 256; }
int attn_blocks_per_cu() { return 1; }

hipError_t launch_attn(const AttnArgs& a, int dtype, int D, bool dmask, hipStream_t s, hipEvent_t ev0,
                       hipEvent_t ev1) {
  if (dtype == 0) return dmask ? launch_d<BF16, true>(a, D, s, ev0, ev1) : launch_d<BF16, false>(a, D, s, ev0, ev1);
  return dmask ? launch_d<F16, true>(a, D, s, ev0, ev1) : launch_d<F16, false>(a, D, s, ev0, ev1);
}

}  // namespace dsv
