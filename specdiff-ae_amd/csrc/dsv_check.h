// dsv_check.h — host-side access emulation of the attention kernels (dry run).
#pragma once

#include <stdint.h>

#include <string>

#include "dsv_internal.h"

namespace dsv {

// Byte range [lo, hi) a kernel may touch for one argument (hi == lo: absent).
struct Extent {
  const char* name;
  uintptr_t lo;
  uintptr_t hi;
};

struct AttnExtents {
  Extent q{"q", 0, 0};
  Extent pre_k{"prefix K", 0, 0}, pre_v{"prefix V", 0, 0}, pre_pt{"prefix page table", 0, 0};
  Extent tree_k{"tree K", 0, 0}, tree_v{"tree V", 0, 0}, tree_pt{"tree page table", 0, 0};
  Extent tpar{"parent", 0, 0}, tmask{"tree mask", 0, 0}, dmask{"byte mask", 0, 0}, perm{"row_perm", 0, 0};
  Extent ws{"workspace", 0, 0};
  Extent out{"out", 0, 0}, lse{"lse", 0, 0}, plse{"prefix_lse", 0, 0}, weight{"weight", 0, 0};
};

// 0 when every access of kernels 1 and 3 stays inside its extent; otherwise
// -1 with a description of the first violation in `err`.  f32: the fp32
// variant of kernel 1 (dsv_attn_f32.hip).
int emulate_attention(const AttnArgs& a, const MergeArgs& m, int D, bool dmask, bool f32, const AttnExtents& ex,
                      std::string& err, int64_t* n_checked);

}  // namespace dsv
