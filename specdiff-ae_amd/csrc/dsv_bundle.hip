// dsv_bundle.hip — bundle scheduling and bundle-ordered query packing on gfx950.
//
// From a tree's parent array, computes on the GPU the node order in which the
// tree-attention kernel packs its query rows, so that a step needs no host
// round trip between the draft tree and the verify launch.  The order is the
// one the host scheduler produces:
//
//   * every leaf (a node that is nobody's parent) gets its branching ancestor:
//     walking up from the leaf, the first parent with more than one child, or
//     the root when the walk reaches it first (core/bundle_scheduler.py:125-145);
//   * leaves are bucketed by that ancestor, buckets in the order of their
//     lowest leaf, each bucket stably sorted by depth and cut into bundles of
//     bundle_size leaves, at most max_bundles bundles in all
//     (core/bundle_scheduler.py:42-123, with the descriptor of
//     draft/tree_verification.py:139-159: leaves in index order, depth = hops
//     to the root);
//   * packing: for each bundle in order and each of its leaves, the nodes of
//     the leaf's root path not placed yet are appended root first; nodes no
//     emitted leaf covers follow in index order.
//
// Formulated without a sequential pass: a node's place is fixed by the key
// (rank of the first emitted leaf whose root path holds it, depth), and
// uncovered nodes by (infinity, index).  The ranks, depths, branching
// ancestors and "first covering leaf" (a minimum over the node's subtree)
// come from pointer jumping over the parent links in LDS: ceil(log2 M) rounds
// of two barriers each, every loop bounded by M, so a malformed parent array
// (a cycle) still ends with some permutation.  Places within a bucket and in
// the final order are counts of smaller packed 32-bit keys, scanned from LDS
// four keys per read (every lane reads the same address: a broadcast).
//
// One workgroup per tree of up to kBundleThreads lanes, each holding up to
// 4 nodes in registers (M <= kBundleMaxNodes).

#include <algorithm>

#include "dsv_internal.h"

namespace dsv {

namespace {

constexpr int kInf = 0x7fffffff;
constexpr int kUnk = -2;

// Calls body(e) for every entry e of x[0, 32 * n32), in order, in every lane:
// eight 16-byte LDS reads in flight per step, every lane reading the same
// address (a broadcast).
template <typename F>
__device__ __forceinline__ void scan_entries(const uint32_t* x, int n32, F&& body) {
  const uint4* x4 = reinterpret_cast<const uint4*>(x);
  for (int c = 0; c < n32; ++c) {
    uint4 q[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = x4[c * 8 + j];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      body(q[j].x);
      body(q[j].y);
      body(q[j].z);
      body(q[j].w);
    }
  }
}

template <int K>
__global__ void __launch_bounds__(kBundleThreads) bundle_order_kernel(const BundleArgs a) {
  constexpr int N = kBundleMaxNodes;
  // State of the pointer-jumping rounds, then of the bucket and rank scans;
  // arrays whose lifetimes do not overlap share storage.
  __shared__ __align__(16) int dep[N], anc[N], nx[N], rs[N], cnt[N], wmin[N], lor[N], bidl[N];
  __shared__ __align__(16) uint32_t x0[N], x1[N];
  __shared__ int s_nleaf, s_more[2];
  int* bfirst = nx;                                   // after the jumping rounds
  int* bsize = rs;
  uint32_t* bpk = x0;                                 // bucket (first leaf, leaves, bundles)
  uint32_t* lk = x1;                                  // leaf (bucket, depth, index)
  int* boff = nx;                                     // after the bucket scan
  int* bbund = rs;
  uint32_t* key = x0;                                 // after the leaf scan

  // Lane i holds nodes i + k * T (k < K); the scans read all nodes' packed
  // keys and compare each with all the lane's nodes.
  const int M = a.M, T = blockDim.x, i = threadIdx.x, t = blockIdx.x;
  const int M32 = (M + 31) >> 5;                      // entries [M, 32*M32) hold neutral values
  int rounds = 0;                                     // 2^rounds >= M > the length of any path
  while ((1 << rounds) < M) ++rounds;
  auto nid = [&](int k) { return i + k * T; };

  // ---- parents and child counts ----------------------------------------------
  // A parent equal to the node, negative or outside the tree means "no
  // parent"; node 0 is always a root.
  int p[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int n = nid(k);
    p[k] = -1;
    if (n < M) {
      const int64_t off = (int64_t)t * a.p_st + (int64_t)n * a.p_sm;
      const int64_t raw = a.p_i64 ? reinterpret_cast<const int64_t*>(a.parent)[off]
                                  : (int64_t) reinterpret_cast<const int32_t*>(a.parent)[off];
      p[k] = (n == 0 || raw == n || raw < 0 || raw >= M) ? -1 : (int)raw;
      cnt[n] = 0;
      wmin[n] = kInf;
    }
  }
  if (i == 0) {
    s_nleaf = 0;
    s_more[0] = s_more[1] = 0;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < K; ++k)
    if (p[k] >= 0) atomicAdd(&cnt[p[k]], 1);
  __syncthreads();

  // Rounds end early once no lane has work left: lanes with work set
  // s_more[r & 1] before the round's second barrier, lane 0 clears the other
  // slot for the next round (nobody reads it between the two barriers).
  auto round_end = [&](int r, bool any) -> bool {
    if (any) s_more[r & 1] = 1;
    if (i == 0) s_more[(r + 1) & 1] = 0;
    __syncthreads();
    return s_more[r & 1] != 0;
  };

  // ---- depth (hops to the root) and branching ancestor, jumped together -------------
  // Depth: (hops covered, node reached) doubles each round.  Branching
  // ancestor: a walk stops at x when x is a root (result x) or x's parent has
  // more than one child (result: the parent), else it moves to the parent;
  // after r rounds every walk that stops within 2^r - 1 hops is resolved.
  int d[K], up[K], res[K], nxt[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int n = nid(k);
    d[k] = p[k] >= 0 ? 1 : 0;
    up[k] = p[k];
    res[k] = 0;
    nxt[k] = -1;
    if (n < M) {
      if (p[k] < 0) {
        res[k] = n;
      } else if (cnt[p[k]] > 1) {
        res[k] = p[k];
      } else {
        res[k] = kUnk;
        nxt[k] = p[k];
      }
      dep[n] = d[k];
      anc[n] = up[k];
      rs[n] = res[k];
      nx[n] = nxt[k];
    }
  }
  __syncthreads();
  for (int r = 0; r < rounds; ++r) {
    bool any = false;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      // every load of the round is issued before any result is used
      const int yu = up[k] >= 0 ? up[k] : 0, yn = res[k] == kUnk ? nxt[k] : 0;
      const int du = dep[yu], au = anc[yu], ry = rs[yn], ny = nx[yn];
      if (up[k] >= 0) {
        d[k] += du;
        up[k] = au;
      }
      if (res[k] == kUnk) {
        if (ry != kUnk)
          res[k] = ry;
        else
          nxt[k] = ny;
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int n = nid(k);
      if (n < M) {
        dep[n] = d[k];
        anc[n] = up[k];
        rs[n] = res[k];
        nx[n] = nxt[k];
        any = any || up[k] >= 0 || res[k] == kUnk;
      }
    }
    if (!round_end(r, any)) break;
  }

  // ---- buckets ----------------------------------------------------------------------
  bool leaf[K];
  int dk[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int n = nid(k);
    if (res[k] == kUnk) res[k] = 0;   // a walk around a cycle
    dk[k] = min(d[k], 2047);          // depth field of the packed keys (< M on a tree)
    leaf[k] = n < M && cnt[n] == 0;
    if (n < M) {
      bfirst[n] = kInf;
      bsize[n] = 0;
    }
    // leaf key: (bucket, depth, index) -- a bucket's leaves in the scheduler's
    // order (stable sort by depth) are consecutive keys
    if (n < 32 * M32) lk[n] = leaf[k] ? ((uint32_t)res[k] << 21) | ((uint32_t)dk[k] << 10) | (uint32_t)n : 0xffffffffu;
  }
  if (i == 0) s_more[0] = s_more[1] = 0;
  __syncthreads();
#pragma unroll
  for (int k = 0; k < K; ++k) {
    if (leaf[k]) {
      atomicMin(&bfirst[res[k]], nid(k));
      atomicAdd(&bsize[res[k]], 1);
      atomicAdd(&s_nleaf, 1);
    }
  }
  __syncthreads();
  const int nleaf = s_nleaf;
  const int bs = a.num_bundles > 0 ? max(1, (nleaf + a.num_bundles - 1) / a.num_bundles) : a.bundle_size;
  // bucket key: (first leaf, leaves, bundles) -- buckets come in the order of
  // their lowest leaf
  uint32_t lim[K];
  bool head[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int n = nid(k);
    const int f = n < M ? bfirst[n] : kInf;
    head[k] = f != kInf;
    lim[k] = 0;
    if (n < 32 * M32) {
      uint32_t v = 0xffffffffu;
      if (f != kInf) {
        const int sz = bsize[n];
        const int nb = min((sz + bs - 1) / bs, 2047);
        v = ((uint32_t)f << 22) | ((uint32_t)sz << 11) | (uint32_t)nb;
        lim[k] = (uint32_t)f << 22;
      }
      bpk[n] = v;
    }
  }
  __syncthreads();
  // A bucket's offsets in leaves and in bundles: sums over the buckets before
  // it (lim == 0 for nodes that head no bucket: nothing is below it).
  {
    int o[K], ob[K];
#pragma unroll
    for (int k = 0; k < K; ++k) o[k] = ob[k] = 0;
    scan_entries(bpk, M32, [&](uint32_t e) {
      const int sz = (int)((e >> 11) & 2047), nb = (int)(e & 2047);
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const bool below = e < lim[k];
        o[k] += below ? sz : 0;
        ob[k] += below ? nb : 0;
      }
    });
    // (bfirst / bsize, whose storage boff / bbund reuse, were read before the
    // last barrier)
#pragma unroll
    for (int k = 0; k < K; ++k) {
      if (head[k]) {
        boff[nid(k)] = o[k];
        bbund[nid(k)] = ob[k];
      }
    }
  }
  __syncthreads();
  // A leaf's place in its bucket: the leaf keys of its bucket below its own.
  {
    uint32_t lo[K], span[K];
    int pos[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const uint32_t mine = leaf[k] ? ((uint32_t)res[k] << 21) | ((uint32_t)dk[k] << 10) | (uint32_t)nid(k) : 0u;
      lo[k] = mine & 0xffe00000u;
      span[k] = mine - lo[k];       // 0 for a non-leaf: counts nothing
      pos[k] = 0;
    }
    scan_entries(lk, M32, [&](uint32_t e) {
#pragma unroll
      for (int k = 0; k < K; ++k) pos[k] += (e - lo[k] < span[k]) ? 1 : 0;
    });
#pragma unroll
    for (int k = 0; k < K; ++k) {
      if (!leaf[k]) continue;
      const int n = nid(k);
      const int bid = bbund[res[k]] + pos[k] / bs;
      if (bid < a.max_bundles) {
        const int rank = boff[res[k]] + pos[k];
        wmin[n] = rank;
        lor[rank] = n;
        bidl[n] = bid;
      }
    }
  }

  // ---- first covering leaf: minimum rank over each node's subtree ------------------
  // Round r pushes every node's running minimum to its ancestor 2^r hops up;
  // after r rounds a node holds the minimum over its descendants fewer than
  // 2^r hops below (values only ever come from descendants, so the in-place
  // updates within a round are safe).
  int u[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    u[k] = p[k];
    if (nid(k) < M) anc[nid(k)] = u[k];
  }
  __syncthreads();
  for (int r = 0; r < rounds; ++r) {
    bool any = false;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int n = nid(k);
      const int y = u[k] >= 0 ? u[k] : 0;
      const int wn = n < M ? wmin[n] : kInf, ay = anc[y];
      if (u[k] >= 0) {
        atomicMin(&wmin[u[k]], wn);
        u[k] = ay;
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < K; ++k) {
      if (nid(k) < M) {
        anc[nid(k)] = u[k];
        any = any || u[k] >= 0;
      }
    }
    if (!round_end(r, any)) break;
  }

  // ---- order: rank of each node's key ------------------------------------------------
  // covered: (first covering leaf's rank, depth, index); uncovered: (1, index)
  // -- all distinct; padding entries sort last.
  uint32_t ki[K];
  int w[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int n = nid(k);
    ki[k] = 0xffffffffu;
    w[k] = kInf;
    if (n < M) {
      w[k] = wmin[n];
      ki[k] = w[k] != kInf ? ((uint32_t)w[k] << 21) | ((uint32_t)dk[k] << 10) | (uint32_t)n : 0x80000000u | (uint32_t)n;
    }
    if (n < 32 * M32) key[n] = ki[k];
  }
  __syncthreads();
  {
    int pos[K];
#pragma unroll
    for (int k = 0; k < K; ++k) pos[k] = 0;
    scan_entries(key, M32, [&](uint32_t e) {
#pragma unroll
      for (int k = 0; k < K; ++k) pos[k] += e < ki[k] ? 1 : 0;
    });
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int n = nid(k);
      if (n < M) {
        a.perm[(int64_t)t * M + pos[k]] = n;
        if (a.bundle_of != nullptr) a.bundle_of[(int64_t)t * M + n] = w[k] != kInf ? bidl[lor[w[k]]] : -1;
      }
    }
  }
}

}  // namespace

hipError_t launch_bundle_order(const BundleArgs& a, hipStream_t s) {
  if (a.B <= 0 || a.M < 1 || a.M > kBundleMaxNodes) return hipSuccess;
  // One lane per node up to kBundleThreads nodes, then 2 or 4 nodes per lane.
  const int threads = std::min(kBundleThreads, ((a.M + 63) / 64) * 64);
  const int per_lane = (a.M + threads - 1) / threads;
  const dim3 grid((unsigned)a.B), block((unsigned)threads);
  if (per_lane == 1)
    hipLaunchKernelGGL(bundle_order_kernel<1>, grid, block, 0, s, a);
  else if (per_lane == 2)
    hipLaunchKernelGGL(bundle_order_kernel<2>, grid, block, 0, s, a);
  else
    hipLaunchKernelGGL(bundle_order_kernel<4>, grid, block, 0, s, a);
  return hipGetLastError();
}

}  // namespace dsv
