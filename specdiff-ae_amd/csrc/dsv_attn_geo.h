// dsv_attn_geo.h — tile geometry and address arithmetic of the split-K
// attention kernel, shared by the gfx950 kernel and the host-side address
// emulation (dry-run mode of the C ABI), so the code that is bounds-checked on
// the CPU is the code the GPU executes.
#pragma once

#include <stdint.h>

#include "dsv_internal.h"

namespace dsv {

#define DSV_HD __host__ __device__ __forceinline__

// Geometry for head_dim D.
//   KT    keys per LDS tile
//   CH    16-byte chunks per key row
//   TILE  bytes of one K (or V) tile
//   NINS  1 KiB DMA wave-instructions per K (or V) tile
//   KPI   keys per DMA instruction
//   RING  bytes of the LDS ring (kStages tiles of K and V); kept <= 64 KiB so
//         every LDS-DMA destination address fits in 16 bits
template <int D>
struct Geo {
  static constexpr int KT = 32;
  static constexpr int CH = D / 8;
  static constexpr int ROWB = 2 * D;
  static constexpr int TILE = KT * ROWB;
  static constexpr int NINS = TILE / 1024;
  static constexpr int KPI = 1024 / ROWB;
  static constexpr int STAGES = 4;
  static constexpr int RING = STAGES * 2 * TILE;
  static_assert(RING <= 65536, "LDS-DMA ring must stay below 64 KiB");
};

// Chunk swizzles of the LDS image (an XOR, hence its own inverse):
//   K: chunk c of key k at slot c ^ (k & 15)         conflict-free S^T operand reads
//   V: chunk c of key k at slot c ^ ((k & 3) << 2)   conflict-free transposed reads
DSV_HD int k_slot(int ch, int key, int c) { return c ^ (key & ((ch < 16 ? ch : 16) - 1)); }
DSV_HD int v_slot(int ch, int key, int c) { return c ^ (((key & 3) << 2) & (ch - 1)); }

// Element offset of chunk c of logical key n of a source, for a given page id.
DSV_HD int64_t src_elem(const KvSrc& s, bool v, int b, int kvh, int64_t n, int64_t page, int c) {
  const int64_t sb = v ? s.v_sb : s.k_sb, sp = v ? s.v_sp : s.k_sp, sh = v ? s.v_sh : s.k_sh,
                st = v ? s.v_st : s.k_st;
  if (s.pt != nullptr) return b * sb + page * sp + kvh * sh + (n & ((1ll << s.ps_shift) - 1)) * st + c * 8;
  return b * sb + n * st + kvh * sh + c * 8;
}

// How a tile's DMA is issued.
//   kFast:   scalar base at the instruction's first key (page resolved once),
//            per-lane offset kii*st + chunk*8, through a bounds-checked buffer
//            resource; also used for tail tiles with per-lane keys clamped to
//            the last valid key (an instruction's keys never straddle a page)
//   kFast32: kFast with the workgroup's batch/head base folded into one
//            buffer resource per workgroup; per tile only the key's byte
//            offset from that base changes, in 32-bit arithmetic, added to
//            the lane offset (the hardware range check covers the sum); the
//            host selects it when every such offset fits (fast32_ok)
//   kLane:   per-lane full address (keys clamped, page per lane); used when a
//            page can split an instruction's keys (page < KPI or unaligned key0)
enum DmaMode : int { kFast = 0, kLane = 1, kFast32 = 2 };

template <int D>
DSV_HD int dma_mode(const KvSrc& s) {
  const bool fast = s.pt == nullptr || ((1ll << s.ps_shift) >= Geo<D>::KPI && (s.key0 & (Geo<D>::KPI - 1)) == 0);
  return fast ? (s.fast32 ? kFast32 : kFast) : kLane;
}

// kFast32: element offset of the workgroup's (batch, head) base, and the byte
// offset of key n's chunk 0 from that base (page = the key's physical page).
DSV_HD int64_t wg_base_elem(const KvSrc& s, bool v, int b, int kvh) {
  return b * (v ? s.v_sb : s.k_sb) + kvh * (v ? s.v_sh : s.k_sh);
}
// The same with the half's byte strides given (st2 = 2*st, sp2 = 2*sp,
// psm = page_size - 1) and the paging known.
DSV_HD uint32_t tile_off32_s(bool paged, uint32_t st2, uint32_t sp2, uint32_t psm, uint32_t n, uint32_t page) {
  return paged ? page * sp2 + (n & psm) * st2 : n * st2;
}
DSV_HD uint32_t tile_off32(const KvSrc& s, bool v, uint32_t n, uint32_t page) {
  return tile_off32_s(s.pt != nullptr, (uint32_t)(2 * (v ? s.v_st : s.k_st)), (uint32_t)(2 * (v ? s.v_sp : s.k_sp)),
                      (1u << s.ps_shift) - 1u, n, page);
}
// Host-side choice of kFast32: both views span less than 4 GiB from their
// base (so every key offset from a workgroup base does too), strides fit,
// and logical keys up to key_end fit in 31 bits.
inline bool fast32_ok(const KvSrc& s, int64_t key_end) {
  const int64_t lim = 1ll << 32;
  auto fits = [&](int64_t x) { return x >= 0 && 2 * x < lim; };
  if (s.k_bytes >= lim || s.v_bytes >= lim || key_end >= (1ll << 31)) return false;
  if (!fits(s.k_st) || !fits(s.v_st)) return false;
  return s.pt == nullptr || (fits(s.k_sp) && fits(s.v_sp));
}

// Instruction i of a tile (0..2*NINS-1: K first, then V): which half and block.
template <int D>
DSV_HD void dma_ins(int i, bool& is_v, int& j) {
  is_v = i >= Geo<D>::NINS;
  j = is_v ? i - Geo<D>::NINS : i;
}

// Fast mode.  Logical key of the instruction's scalar base and of a lane.
//   n0 = key0 + kb + j*KPI (first key); nb = min(n0, last); nl = min(n0 + kii, last)
DSV_HD int64_t fast_base_key(const KvSrc& s, int64_t kb, int64_t kend, int j, int kpi) {
  const int64_t n0 = s.key0 + kb + (int64_t)j * kpi, last = s.key0 + kend - 1;
  return n0 < last ? n0 : last;
}
DSV_HD int64_t fast_lane_key(const KvSrc& s, int64_t kb, int64_t kend, int j, int kpi, int kii) {
  const int64_t n = s.key0 + kb + (int64_t)j * kpi + kii, last = s.key0 + kend - 1;
  return n < last ? n : last;
}
// Per-lane element offset relative to the scalar base (key nb, chunk 0).
DSV_HD int64_t fast_lane_elem(const KvSrc& s, bool v, int64_t nb, int64_t nl, int c) {
  return (nl - nb) * (v ? s.v_st : s.k_st) + c * 8;
}

// Buffer-resource range: bytes from the scalar base to the end of the source
// (accesses at or beyond it read zeros instead of faulting).
DSV_HD uint32_t rsrc_range(int64_t span_bytes, int64_t base_elem) {
  const int64_t r = span_bytes - 2 * base_elem;
  return r <= 0 ? 0u : (r >= 0xffffffffll ? 0xffffffffu : (uint32_t)r);
}

// Lane mode: logical key of a lane (clamped to the last valid key).
DSV_HD int64_t lane_key(const KvSrc& s, int64_t kb, int64_t kend, int key_in_tile) {
  const int64_t n = s.key0 + kb + key_in_tile, last = s.key0 + kend - 1;
  return n < last ? n : last;
}

DSV_HD int64_t clamp_page(int64_t pg, int64_t n_phys) { return pg < 0 ? 0 : (pg >= n_phys ? n_phys - 1 : pg); }

}  // namespace dsv
