// dsv_commit.hip — accepted-path KV commit on gfx950.
//
// After the acceptance walk, the K/V rows of the accepted path move to the
// front of the tree's slots: for every (layer, K/V half, head) row of the
// cache, tokens [start, start + n) receive tokens start + path[0..n), a
// gather in which every read happens before any write (the reference gathers
// into a temporary, then copies:
// draft/tree_verification.py:197-217).  path and n = info[3] come from the
// acceptance kernel in device memory, so the commit needs no host round trip.
//
// One workgroup per cache row.  The n x D row segment is moved in 16-byte
// chunks: every thread loads its chunks into registers, the workgroup meets a
// barrier, then every thread stores them.  Path entries are clamped to the
// tree (0..M-1) and n to the tree size, so a bad path cannot address outside
// the rows of [start, start + M), which the host checked against the cache.
// The layout is either a page pool (a row = (layer, half, head); token t at
// page page_table[t / page] slot t % page) or a dense [..., S, D] cache.

#include "dsv_internal.h"

namespace dsv {

namespace {

template <typename E>
__global__ void __launch_bounds__(kCommitThreads) kv_commit_kernel(const CommitArgs a) {
  constexpr int CE = 16 / (int)sizeof(E);  // elements per 16-byte chunk
  const int64_t row = blockIdx.x;
  // Row base: the leading index decomposed over up to 4 leading dimensions.
  int64_t off = 0, r = row;
#pragma unroll
  for (int d = 3; d >= 0; --d) {
    if (d < a.nlead) {
      off += (r % a.lead_shape[d]) * a.lead_stride[d];
      r /= a.lead_shape[d];
    }
  }
  const E* base = reinterpret_cast<const E*>(a.data) + off;
  E* wbase = reinterpret_cast<E*>(a.data) + off;

  int64_t n = a.info[3];
  n = n < 0 ? 0 : (n > a.M ? a.M : n);
  const int cpt = a.D / CE;  // chunks per token
  const int total = (int)n * cpt;

  auto token_off = [&](int64_t t) -> int64_t {
    if (a.pt == nullptr) return t * a.tok_stride;
    int64_t pg = a.pt_i64 ? reinterpret_cast<const int64_t*>(a.pt)[t >> a.ps_shift]
                          : (int64_t) reinterpret_cast<const int32_t*>(a.pt)[t >> a.ps_shift];
    pg = pg < 0 ? 0 : (pg >= a.n_phys ? a.n_phys - 1 : pg);
    return pg * a.page_stride + (t & ((1ll << a.ps_shift) - 1)) * a.tok_stride;
  };

  u32x4 buf[kCommitChunks];
#pragma unroll
  for (int k = 0; k < kCommitChunks; ++k) {
    const int c = threadIdx.x + k * kCommitThreads;
    if (c < total) {
      const int i = c / cpt, part = c - i * cpt;
      int64_t p = a.path[i];
      p = p < 0 ? 0 : (p >= a.M ? a.M - 1 : p);
      buf[k] = *reinterpret_cast<const u32x4*>(base + token_off(a.start + p) + part * CE);
    }
  }
  // Every load has returned its data before any thread of the row stores.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kCommitChunks; ++k) {
    const int c = threadIdx.x + k * kCommitThreads;
    if (c < total) {
      const int i = c / cpt, part = c - i * cpt;
      *reinterpret_cast<u32x4*>(wbase + token_off(a.start + i) + part * CE) = buf[k];
    }
  }
}

}  // namespace

hipError_t launch_commit(const CommitArgs& a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  const dim3 grid((unsigned)a.rows), block(kCommitThreads);
  if (a.esize == 2)
    hipLaunchKernelGGL(kv_commit_kernel<uint16_t>, grid, block, 0, s, a);
  else
    hipLaunchKernelGGL(kv_commit_kernel<float>, grid, block, 0, s, a);
  return hipGetLastError();
}

}  // namespace dsv
