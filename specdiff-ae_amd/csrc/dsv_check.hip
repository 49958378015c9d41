// dsv_check.hip — host-side emulation of every memory access of the attention
// kernels (1-3), for the dry-run mode of the C ABI.
//
// For a fully planned launch (the AttnArgs / MergeArgs the entry point would
// launch with), walk every workgroup, tile, DMA instruction and lane with the
// address arithmetic the kernel itself uses (dsv_attn_geo.h) and check each
// global byte range against the extent of the tensor it must stay inside, and
// each LDS address against the kernel's LDS layout.  Page-table contents are
// not known on the host: the kernel clamps page ids into [0, n_phys), so both
// ends of that range are checked (offsets are monotone in the page id).

#include <cstdio>
#include <string>

#include "dsv_attn_f32_geo.h"
#include "dsv_attn_geo.h"
#include "dsv_check.h"

namespace dsv {

namespace {

struct Checker {
  std::string* err;
  int64_t n_checked = 0;
  bool ok = true;

  bool range(const Extent& e, uintptr_t addr, int64_t nbytes, const char* what) {
    ++n_checked;
    if (e.hi > e.lo && addr >= e.lo && addr + (uintptr_t)nbytes <= e.hi) return true;
    if (ok) {
      char buf[256];
      snprintf(buf, sizeof(buf), "%s: %lld bytes at %#llx outside %s [%#llx, %#llx)", what, (long long)nbytes,
               (unsigned long long)addr, e.name, (unsigned long long)e.lo, (unsigned long long)e.hi);
      *err = buf;
    }
    ok = false;
    return false;
  }
  bool cond(bool c, const char* what) {
    ++n_checked;
    if (!c && ok) *err = what;
    ok = ok && c;
    return c;
  }
};

uintptr_t elem_addr(const void* base, int64_t elem, int esize) {
  return (uintptr_t)base + (uintptr_t)(elem * esize);
}

// Highest LDS byte address (exclusive) an LDS-DMA destination may reach.
constexpr int kLdsDmaLimit = 65536;

template <int D>
void check_kernel1(const AttnArgs& a, bool dmask, const AttnExtents& ex, Checker& ck) {
  using G = Geo<D>;
  const int RING = G::RING;
  ck.cond(RING <= 65536, "LDS-DMA ring above 64 KiB");
  const int64_t nrows_all = (int64_t)a.s_total * a.B * a.Hk * a.R;
  for (int b = 0; b < a.B && ck.ok; ++b) {
    for (int kvh = 0; kvh < a.Hk && ck.ok; ++kvh) {
      for (int split = 0; split < a.s_total && ck.ok; ++split) {
        const bool is_tree = a.has_tree && split == a.n_splits;
        const KvSrc& src = is_tree ? a.tree : a.pre;
        const Extent& ek = is_tree ? ex.tree_k : ex.pre_k;
        const Extent& ev = is_tree ? ex.tree_v : ex.pre_v;
        const Extent& ept = is_tree ? ex.tree_pt : ex.pre_pt;
        int64_t kstart, kend;
        if (is_tree) {
          kstart = 0;
          kend = a.M;
        } else {
          kstart = (int64_t)split * a.kps;
          kend = std::min(kstart + a.kps, a.n_pre);
        }
        const int64_t nkeys = kend - kstart;
        const int ntiles = nkeys > 0 ? (int)((nkeys + G::KT - 1) / G::KT) : 0;
        const bool paged = src.pt != nullptr;
        int64_t pt_lo = 0;
        if (paged && ntiles > 0) {
          pt_lo = (src.key0 + kstart) >> src.ps_shift;
          const int64_t pt_hi = (src.key0 + kend - 1) >> src.ps_shift;
          ck.cond(pt_hi - pt_lo + 1 <= kPageLds, "page-table slice exceeds its LDS table");
          const int es = src.pt_i64 ? 8 : 4;
          ck.range(ept, elem_addr(src.pt, b * src.pt_sb + pt_lo, es), (pt_hi - pt_lo + 1) * es, "page-table read");
          ck.cond(src.n_phys > 0, "empty page pool");
        }
        if (is_tree) {
          ck.cond(a.M <= kTreeMaxM, "tree larger than the LDS bitmask table");
          if (a.tpar != nullptr) {
            const int es = a.tpar_i64 ? 8 : 4;
            for (int node = 0; node < a.M; ++node)
              ck.range(ex.tpar, elem_addr(a.tpar, b * a.tpar_sb + node * a.tpar_sm, es), es, "parent read");
          } else {
            const int es = a.tmask_dtype == 2 ? 4 : (a.tmask_dtype <= 1 ? 2 : 1);
            const int64_t last = b * a.tm_sb + (int64_t)(a.M - 1) * a.tm_sm + (int64_t)(a.M - 1) * a.tm_sn;
            ck.range(ex.tmask, elem_addr(a.tmask, b * a.tm_sb, es), 1, "tree-mask read (first)");
            ck.range(ex.tmask, elem_addr(a.tmask, last, es), es, "tree-mask read (last)");
          }
        }
        const int mode = dma_mode<D>(src);
        const int64_t pages[2] = {0, paged ? src.n_phys - 1 : 0};
        for (int t = 0; t < ntiles && ck.ok; ++t) {
          const int stage = t & (G::STAGES - 1);
          const int64_t kb = kstart + (int64_t)t * G::KT;
          for (int i = 0; i < 2 * G::NINS && ck.ok; ++i) {
            bool is_v;
            int j;
            dma_ins<D>(i, is_v, j);
            const int dst = (stage * 2 + (is_v ? 1 : 0)) * G::TILE + j * 1024;
            ck.cond(dst >= 0 && dst + 1024 <= RING, "LDS-DMA destination outside the ring");
            // Lane l of an LDS-DMA instruction writes 16 bytes at M0 + 16 l:
            // every such destination stays below 64 KiB.
            for (int l = 0; l < 64; ++l)
              ck.cond(dst + 16 * l + 16 <= kLdsDmaLimit, "LDS-DMA lane destination at or above 64 KiB");
            const uint16_t* base = is_v ? src.v : src.k;
            const Extent& e = is_v ? ev : ek;
            for (int lane = 0; lane < 64 && ck.ok; ++lane) {
              const int kii = lane / G::CH, slot = lane % G::CH;
              const int key_t = j * G::KPI + kii;
              const int c = is_v ? v_slot(G::CH, key_t, slot) : k_slot(G::CH, key_t, slot);
              ck.cond(c >= 0 && c < G::CH, "chunk index out of range");
              for (int pi = 0; pi < (paged ? 2 : 1); ++pi) {
                if (mode == kFast32) {
                  const int64_t nb = fast_base_key(src, kb, kend, j, G::KPI);
                  const int64_t nl = fast_lane_key(src, kb, kend, j, G::KPI, kii);
                  ck.cond(nb >= 0 && nb < (1ll << 31), "key beyond 31 bits in 32-bit mode");
                  ck.cond(!paged || (nb >> src.ps_shift) == (nl >> src.ps_shift), "DMA instruction straddles a page");
                  ck.cond(!paged || ((nb >> src.ps_shift) - pt_lo >= 0 && (nb >> src.ps_shift) - pt_lo < kPageLds),
                          "page slot outside the staged slice");
                  const int64_t wb = wg_base_elem(src, is_v, b, kvh);
                  const int64_t le = fast_lane_elem(src, is_v, nb, nl, c);
                  // The kernel adds a 32-bit lane offset and a 32-bit key offset
                  // without overflow checks: the true sum must stay below 2^32.
                  const int64_t off = le * 2 + (int64_t)tile_off32(src, is_v, (uint32_t)nb, (uint32_t)pages[pi]);
                  ck.cond(le >= 0 && off >= 0 && off + 16 <= 0xffffffffll, "32-bit DMA offset overflow");
                  ck.cond(off == 2 * (src_elem(src, is_v, b, kvh, nb, pages[pi], 0) - wb) + le * 2,
                          "32-bit offset differs from the 64-bit address");
                  const uint32_t range = rsrc_range(is_v ? src.v_bytes : src.k_bytes, wb);
                  ck.cond(off + 16 <= (int64_t)range, "lane beyond the buffer range");
                  ck.range(e, elem_addr(base, wb, 2) + (uintptr_t)off, 16, is_v ? "V DMA (fast32)" : "K DMA (fast32)");
                } else if (mode == kFast) {
                  const int64_t nb = fast_base_key(src, kb, kend, j, G::KPI);
                  const int64_t nl = fast_lane_key(src, kb, kend, j, G::KPI, kii);
                  ck.cond(!paged || (nb >> src.ps_shift) == (nl >> src.ps_shift), "DMA instruction straddles a page");
                  ck.cond(!paged || ((nb >> src.ps_shift) - pt_lo >= 0 &&
                                     (nb >> src.ps_shift) - pt_lo < kPageLds),
                          "page slot outside the staged slice");
                  const int64_t be = src_elem(src, is_v, b, kvh, nb, pages[pi], 0);
                  const int64_t le = fast_lane_elem(src, is_v, nb, nl, c);
                  ck.cond(le >= 0 && le * 2 < 0xffffffffll, "lane offset outside 32 bits");
                  const uint32_t range = rsrc_range(is_v ? src.v_bytes : src.k_bytes, be);
                  ck.cond((int64_t)le * 2 + 16 <= (int64_t)range, "lane beyond the buffer range");
                  ck.range(e, elem_addr(base, be + le, 2), 16, is_v ? "V DMA (fast)" : "K DMA (fast)");
                } else {
                  const int64_t n = lane_key(src, kb, kend, key_t);
                  ck.cond(!paged || ((n >> src.ps_shift) - pt_lo >= 0 && (n >> src.ps_shift) - pt_lo < kPageLds),
                          "page slot outside the staged slice");
                  ck.range(e, elem_addr(base, src_elem(src, is_v, b, kvh, n, pages[pi], c), 2), 16,
                           is_v ? "V DMA (lane)" : "K DMA (lane)");
                }
              }
            }
          }
          if (dmask && a.dmask != nullptr) {
            // Highest mask byte the tile can read (n < dm_n is checked before reading).
            const int64_t nmax = std::min(kb + G::KT, a.dm_n) - 1;
            if (nmax >= 0 && nmax >= kb) {
              const int64_t last = b * a.dm_sb + (int64_t)(a.M - 1) * a.dm_sm + nmax * a.dm_sn;
              ck.range(ex.dmask, elem_addr(a.dmask, last, 1), 1, "byte-mask read");
              ck.range(ex.dmask, elem_addr(a.dmask, b * a.dm_sb + kb * a.dm_sn, 1), 1, "byte-mask read");
            }
          }
        }
        // Query rows and partial outputs of every row block.
        for (int rb = 0; rb < a.n_rb && ck.ok; ++rb) {
          const int rpb = attn_rows_per_block();
          for (int r = rb * rpb; r < std::min(a.R, (rb + 1) * rpb) && ck.ok; ++r) {
            const int g = r / a.M, mi = r - g * a.M;
            const int m = mi;  // row_perm entries are clamped into [0, M) by the kernel
            ck.range(ex.q, elem_addr(a.q, b * a.q_sb + (int64_t)m * a.q_sm + (int64_t)(kvh * a.G + g) * a.q_sh, 2),
                     2 * D, "Q row read");
            if (a.row_perm != nullptr) ck.range(ex.perm, elem_addr(a.row_perm, mi, 4), 4, "row_perm read");
            const int64_t prow = (((int64_t)split * a.B + b) * a.Hk + kvh) * a.R + r;
            ck.cond(prow < nrows_all, "partial row out of range");
            ck.range(ex.ws, elem_addr(a.opart, prow * D, 2), 2 * D, "partial write");
            ck.range(ex.ws, (uintptr_t)(a.ml + prow), 8, "partial stats write");
          }
        }
      }
    }
  }
}

// The fp32 kernel: per workgroup, the page-table slice and tree inputs as in
// the 16-bit kernel; per tile, every thread's 16-byte K and V chunk loads
// (keys clamped to the split, pages at both ends of the clamp range); the Q
// rows (fp32) and the bf16 partial rows it writes.
template <int D>
void check_kernel_f32(const AttnArgs& a, bool dmask, const AttnExtents& ex, Checker& ck) {
  using G = GeoF32<D>;
  const int64_t nrows_all = (int64_t)a.s_total * a.B * a.Hk * a.R;
  for (int b = 0; b < a.B && ck.ok; ++b) {
    for (int kvh = 0; kvh < a.Hk && ck.ok; ++kvh) {
      for (int split = 0; split < a.s_total && ck.ok; ++split) {
        const bool is_tree = a.has_tree && split == a.n_splits;
        const KvSrc& src = is_tree ? a.tree : a.pre;
        const Extent& ek = is_tree ? ex.tree_k : ex.pre_k;
        const Extent& ev = is_tree ? ex.tree_v : ex.pre_v;
        const Extent& ept = is_tree ? ex.tree_pt : ex.pre_pt;
        int64_t kstart, kend;
        if (is_tree) {
          kstart = 0;
          kend = a.M;
        } else {
          kstart = (int64_t)split * a.kps;
          kend = std::min(kstart + a.kps, a.n_pre);
        }
        const int64_t nkeys = kend - kstart;
        const int ntiles = nkeys > 0 ? (int)((nkeys + G::KT - 1) / G::KT) : 0;
        const bool paged = src.pt != nullptr;
        int64_t pt_lo = 0;
        if (paged && ntiles > 0) {
          pt_lo = (src.key0 + kstart) >> src.ps_shift;
          const int64_t pt_hi = (src.key0 + kend - 1) >> src.ps_shift;
          ck.cond(pt_hi - pt_lo + 1 <= kPageLds, "page-table slice exceeds its LDS table");
          const int es = src.pt_i64 ? 8 : 4;
          ck.range(ept, elem_addr(src.pt, b * src.pt_sb + pt_lo, es), (pt_hi - pt_lo + 1) * es, "page-table read");
          ck.cond(src.n_phys > 0, "empty page pool");
        }
        if (is_tree) {
          ck.cond(a.M <= kTreeMaxM, "tree larger than the LDS bitmask table");
          if (a.tpar != nullptr) {
            const int es = a.tpar_i64 ? 8 : 4;
            for (int node = 0; node < a.M; ++node)
              ck.range(ex.tpar, elem_addr(a.tpar, b * a.tpar_sb + node * a.tpar_sm, es), es, "parent read");
          } else {
            const int es = a.tmask_dtype == 2 ? 4 : (a.tmask_dtype <= 1 ? 2 : 1);
            const int64_t last = b * a.tm_sb + (int64_t)(a.M - 1) * a.tm_sm + (int64_t)(a.M - 1) * a.tm_sn;
            ck.range(ex.tmask, elem_addr(a.tmask, b * a.tm_sb, es), 1, "tree-mask read (first)");
            ck.range(ex.tmask, elem_addr(a.tmask, last, es), es, "tree-mask read (last)");
          }
        }
        const int64_t pages[2] = {0, paged ? src.n_phys - 1 : 0};
        for (int t = 0; t < ntiles && ck.ok; ++t) {
          const int64_t kb = kstart + (int64_t)t * G::KT;
          for (int ch = 0; ch < G::CHUNKS && ck.ok; ++ch) {
            const int kk = ch / G::CPR, c4 = ch % G::CPR;
            const int64_t n = f32_key(src, kb, kend, kk);
            ck.cond(!paged || ((n >> src.ps_shift) - pt_lo >= 0 && (n >> src.ps_shift) - pt_lo < kPageLds),
                    "page slot outside the staged slice");
            for (int pi = 0; pi < (paged ? 2 : 1); ++pi) {
              ck.range(ek, elem_addr(src.k, f32_elem(src, false, b, kvh, n, pages[pi], c4), 4), 16, "K load (f32)");
              ck.range(ev, elem_addr(src.v, f32_elem(src, true, b, kvh, n, pages[pi], c4), 4), 16, "V load (f32)");
            }
          }
          if (dmask && a.dmask != nullptr) {
            const int64_t nmax = std::min(kb + G::KT, a.dm_n) - 1;
            if (nmax >= 0 && nmax >= kb) {
              const int64_t last = b * a.dm_sb + (int64_t)(a.M - 1) * a.dm_sm + nmax * a.dm_sn;
              ck.range(ex.dmask, elem_addr(a.dmask, last, 1), 1, "byte-mask read");
              ck.range(ex.dmask, elem_addr(a.dmask, b * a.dm_sb + kb * a.dm_sn, 1), 1, "byte-mask read");
            }
          }
        }
        for (int r = 0; r < a.R && ck.ok; ++r) {
          const int g = r / a.M, mi = r - g * a.M;
          ck.range(ex.q, elem_addr(a.q, b * a.q_sb + (int64_t)mi * a.q_sm + (int64_t)(kvh * a.G + g) * a.q_sh, 4),
                   4 * D, "Q row read (f32)");
          if (a.row_perm != nullptr) ck.range(ex.perm, elem_addr(a.row_perm, mi, 4), 4, "row_perm read");
          const int64_t prow = (((int64_t)split * a.B + b) * a.Hk + kvh) * a.R + r;
          ck.cond(prow < nrows_all, "partial row out of range");
          ck.range(ex.ws, elem_addr(a.opart, prow * D, 2), 2 * D, "partial write");
          ck.range(ex.ws, (uintptr_t)(a.ml + prow), 8, "partial stats write");
        }
      }
    }
  }
}

void check_merge(const MergeArgs& m, const AttnExtents& ex, Checker& ck) {
  const int64_t nrows = (int64_t)m.B * m.Hk * m.R;
  for (int64_t row = 0; row < nrows && ck.ok; ++row) {
    const int r = (int)(row % m.R);
    const int kvh = (int)((row / m.R) % m.Hk);
    const int b = (int)(row / ((int64_t)m.R * m.Hk));
    for (int s = 0; s < m.s_total && ck.ok; ++s) {
      ck.range(ex.ws, elem_addr(m.opart, (s * nrows + row) * m.D, 2), 2 * m.D, "merge partial read");
      ck.range(ex.ws, (uintptr_t)(m.ml + s * nrows + row), 8, "merge stats read");
    }
    const int g = r / m.M, mi = r - g * m.M;
    const int h = kvh * m.G + g;
    const int oes = m.out_dtype == 2 ? 4 : 2;
    for (int mm : {0, m.M - 1}) {
      (void)mi;
      ck.range(ex.out, elem_addr(m.out, (int64_t)b * m.o_sb + (int64_t)mm * m.o_sm + (int64_t)h * m.o_sh, oes),
               (int64_t)m.D * oes, "output write");
      if (m.lse != nullptr)
        ck.range(ex.lse, elem_addr(m.lse, (int64_t)b * m.l_sb + (int64_t)mm * m.l_sm + (int64_t)h * m.l_sh, 4), 4,
                 "lse write");
      if (m.weight != nullptr) {
        const int wes = m.w_dtype == 2 ? 4 : 2;
        ck.range(ex.weight, elem_addr(m.weight, (int64_t)b * m.w_sb + (int64_t)mm * m.w_sm + (int64_t)h * m.w_sh, wes),
                 wes, "weight write");
        ck.range(ex.plse, elem_addr(m.plse, (int64_t)b * m.p_sb + (int64_t)mm * m.p_sm + (int64_t)h * m.p_sh, 4), 4,
                 "prefix lse read");
      }
    }
  }
}

}  // namespace

int emulate_attention(const AttnArgs& a, const MergeArgs& m, int D, bool dmask, bool f32, const AttnExtents& ex,
                      std::string& err, int64_t* n_checked) {
  Checker ck{&err};
  if (D == 128)
    f32 ? check_kernel_f32<128>(a, dmask, ex, ck) : check_kernel1<128>(a, dmask, ex, ck);
  else if (D == 64)
    f32 ? check_kernel_f32<64>(a, dmask, ex, ck) : check_kernel1<64>(a, dmask, ex, ck);
  else
    ck.cond(false, "unsupported head_dim in emulation");
  if (ck.ok) check_merge(m, ex, ck);
  if (n_checked) *n_checked = ck.n_checked;
  return ck.ok ? 0 : -1;
}

}  // namespace dsv
