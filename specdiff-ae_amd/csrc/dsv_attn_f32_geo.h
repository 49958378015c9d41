// dsv_attn_f32_geo.h — tile geometry and address arithmetic of the fp32
// split-K attention kernel, shared by the kernel and the host-side address
// emulation (dry-run mode), like dsv_attn_geo.h for the 16-bit kernel.
#pragma once

#include <stdint.h>

#include "dsv_attn_geo.h"

namespace dsv {

// Geometry for head_dim D, fp32 elements.
//   KT      keys per tile
//   CPR     16-byte chunks (4 floats) per key row
//   CHUNKS  16-byte chunks per K (or V) tile
template <int D>
struct GeoF32 {
  static constexpr int KT = 32;
  static constexpr int CPR = D / 4;
  static constexpr int CHUNKS = KT * CPR;
};

// Logical key of row kk of the tile starting at split-relative key kb,
// clamped to the split's last key (tail rows re-read a valid key; their
// scores are masked).
DSV_HD int64_t f32_key(const KvSrc& s, int64_t kb, int64_t kend, int kk) {
  const int64_t n = s.key0 + kb + kk, last = s.key0 + kend - 1;
  return n < last ? n : last;
}

// fp32 element offset of 16-byte chunk c4 (floats 4*c4 .. 4*c4+3) of key n.
DSV_HD int64_t f32_elem(const KvSrc& s, bool v, int b, int kvh, int64_t n, int64_t page, int c4) {
  return src_elem(s, v, b, kvh, n, page, 0) + 4 * (int64_t)c4;
}

}  // namespace dsv
