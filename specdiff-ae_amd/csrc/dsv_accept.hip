// dsv_accept.hip — kernel 4: tree acceptance on gfx950.
//
// Stage A (accept_rowstat_kernel): one workgroup per (tree node row, vocab
// chunk) streams the row's logits with 16-byte loads and reduces
//   * argmax with the first-index tie rule of torch.argmax (NaN ranks above
//     every number, as torch's max does), and
//   * for typical acceptance, the online softmax statistics of y = x / T:
//     m = max y (kept in log2 units), l = sum 2^(y*log2e - m), s = sum y*2^(...)
//     which give the entropy H = ln2*(m + log2 l) - s/l in one pass.
// Stage B (accept_walk_kernel): one workgroup per tree, one thread per node:
// combines the chunk statistics, evaluates the acceptance test of every
// node against its parent's distribution, runs the bounded ancestor closure,
// picks the winner and traces the path back to the root.
//
// Walk semantics follow draft/tree_verification.py:100-182 line by line:
//   next = argmax(logits)                          (:101-102)
//   parent_ext = [0] + (parent + 1), parent[k]==k -> -1   (:120-125)
//   ok[i] = draft[i] == next[parent_ext[i]]; ok[0] = True  (:127-129)
//   ok &= ok[parent_ext], max_hops rounds           (:131-137)
//   winner = argmax(where(ok, pos, 0))  (first max)  (:161-162)
//   path = traceback to the root, next_token = next[winner] (:165-182)
// Typical acceptance (absent from the reference) replaces the equality test
// with the posterior criterion of Cai et al. 2024 (Medusa, typical acceptance):
//   p_T(draft[i] | parent) > min(eps, alpha * exp(-H(p_T(. | parent)))).

#include <algorithm>

#include "dsv_internal.h"
#include "dsv_stats.h"

namespace dsv {

namespace {

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634074f;
constexpr float kLn2 = 0.69314718055994530942f;
constexpr int kRowThreads = 256;

template <typename LT>
__device__ __forceinline__ float to_f(LT x);
template <>
__device__ __forceinline__ float to_f<uint16_t>(uint16_t x) {  // bf16 bits
  return __uint_as_float((uint32_t)x << 16);
}
template <>
__device__ __forceinline__ float to_f<_Float16>(_Float16 x) { return (float)x; }
template <>
__device__ __forceinline__ float to_f<float>(float x) { return x; }

template <typename LT, bool TYPICAL>
__global__ void __launch_bounds__(kRowThreads) accept_rowstat_kernel(const AcceptArgs a) {
  const int c = blockIdx.x;
  const int64_t row = blockIdx.y;  // t * M + i
  const int t = (int)(row / a.M), i = (int)(row % a.M);
  const LT* base = reinterpret_cast<const LT*>(a.logits) + (int64_t)t * a.l_st + (int64_t)i * a.l_sm;
  const int64_t lo = (int64_t)c * a.chunk;
  const int64_t hi = min(lo + a.chunk, a.V);
  constexpr int VEC = 16 / sizeof(LT);

  ArgMax best{kNegInf, 0x7fffffff};
  bool have = false;
  Soft sm{kNegInf, 0.f, 0.f};
  const float zs = a.inv_temp * kLog2e;

  auto consume = [&](const float* xs, int n, int64_t idx0) {
    float vmax = kNegInf;
    for (int e = 0; e < n; ++e) {
      const float x = xs[e];
      if (!have || am_better(x, (int)(idx0 + e), best.v, best.i)) {
        best.v = x;
        best.i = (int)(idx0 + e);
        have = true;
      }
      if constexpr (TYPICAL) vmax = fmaxf(vmax, x * zs);
    }
    if constexpr (TYPICAL) {
      if (vmax > sm.m) {
        const float f = (sm.m == kNegInf) ? 0.f : __builtin_amdgcn_exp2f(sm.m - vmax);
        sm.l *= f;
        sm.s *= f;
        sm.m = vmax;
      }
      if (sm.m != kNegInf) {
        for (int e = 0; e < n; ++e) {
          const float p = __builtin_amdgcn_exp2f(fmaf(xs[e], zs, -sm.m));
          sm.l += p;
          // 0 log 0 = 0: a -inf logit (p = 0) adds nothing to s.
          if (p > 0.f) sm.s = fmaf(xs[e] * a.inv_temp, p, sm.s);
        }
      }
    }
  };

  const bool aligned = ((reinterpret_cast<uintptr_t>(base + lo) & 15) == 0);
  if (aligned) {
    const int64_t nvec = (hi - lo) / VEC;
    auto consume_vec = [&](const u32x4& raw, int64_t vi) {
      float xs[VEC];
      const LT* el = reinterpret_cast<const LT*>(&raw);
#pragma unroll
      for (int e = 0; e < VEC; ++e) xs[e] = to_f<LT>(el[e]);
      consume(xs, VEC, lo + vi * VEC);
    };
    // Four of the thread's vectors in flight at a time, consumed in the
    // same (increasing) order as one at a time.
    int64_t vi = threadIdx.x;
    for (; vi + 3 * kRowThreads < nvec; vi += 4 * kRowThreads) {
      u32x4 raw[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) raw[u] = *reinterpret_cast<const u32x4*>(base + lo + (vi + u * kRowThreads) * VEC);
#pragma unroll
      for (int u = 0; u < 4; ++u) consume_vec(raw[u], vi + u * kRowThreads);
    }
    for (; vi < nvec; vi += kRowThreads) consume_vec(*reinterpret_cast<const u32x4*>(base + lo + vi * VEC), vi);
    for (int64_t k = lo + nvec * VEC + threadIdx.x; k < hi; k += kRowThreads) {
      const float x = to_f<LT>(base[k]);
      consume(&x, 1, k);
    }
  } else {
    for (int64_t k = lo + threadIdx.x; k < hi; k += kRowThreads) {
      const float x = to_f<LT>(base[k]);
      consume(&x, 1, k);
    }
  }

  // Wave reduction.
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best.v, o);
    const int oi = __shfl_xor(best.i, o);
    const int oh = __shfl_xor((int)have, o);
    if (oh && (!have || am_better(ov, oi, best.v, best.i))) {
      best.v = ov;
      best.i = oi;
      have = true;
    }
    if constexpr (TYPICAL) {
      Soft other{__shfl_xor(sm.m, o), __shfl_xor(sm.l, o), __shfl_xor(sm.s, o)};
      sm = soft_merge(sm, other);
    }
  }
  __shared__ float sv[kRowThreads / 64], sm_m[kRowThreads / 64], sm_l[kRowThreads / 64], sm_s[kRowThreads / 64];
  __shared__ int si[kRowThreads / 64], sh[kRowThreads / 64];
  const int wid = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wid] = best.v;
    si[wid] = best.i;
    sh[wid] = have;
    sm_m[wid] = sm.m;
    sm_l[wid] = sm.l;
    sm_s[wid] = sm.s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int x = 1; x < kRowThreads / 64; ++x) {
      if (sh[x] && (!have || am_better(sv[x], si[x], best.v, best.i))) {
        best.v = sv[x];
        best.i = si[x];
        have = true;
      }
      if constexpr (TYPICAL) sm = soft_merge(sm, Soft{sm_m[x], sm_l[x], sm_s[x]});
    }
    const int64_t o = row * a.nchunk + c;
    a.rstat[o] = make_float4(best.v, __int_as_float(have ? best.i : -1), sm.m, sm.l);
    if constexpr (TYPICAL) a.rstat2[o] = sm.s;
  }
}

// ---------------------------------------------------------------------------
// Stage A for 16-bit logits (bf16 / f16), rows 16-byte aligned: streaming.
//
// A 16-bit float maps to an unsigned key that orders like the value:
// key = bits ^ (bits < 0 ? 0xFFFF : 0x8000) (sign-magnitude -> offset), so
// the argmax is "largest key, then lowest index".  Keys are formed two per
// dword with packed 16-bit ops (v_pk_ashrrev_i16 / v_pk_max_u16).
//
// A workgroup covers a contiguous vocabulary range of one row and streams it
// in sub-tiles of kSub elements, the loads of sub-tile s+1 in flight while
// sub-tile s is reduced.  A thread's elements have increasing indices from
// sub-tile to sub-tile, so each thread keeps running statistics:
//   * the largest key and the first index holding it: only a strictly larger
//     key of a later sub-tile replaces it, and the index is then located by
//     a scan of the thread's 32 elements (rare after the first sub-tiles);
//   * the first NaN index (torch ranks NaN above every number; a range with
//     a NaN reports NaN at its first NaN, and NaN typical statistics);
//   * typical: (m, l, s) against the thread's running maximum, rescaled when
//     it grows (online softmax).  -inf logits contribute p = 0 and, by
//     0 log 0 = 0, nothing to s: they are clamped to the lowest finite value
//     (their exponential underflows to exactly 0) before the products.
// The workgroup then reduces the thread statistics.  -0 and +0 compare equal
// (keys 0x7FFF and 0x8000): a range whose maximum is +0 is rescanned from
// memory for the first zero of either sign (exact, and rare).
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef short i16x2 __attribute__((ext_vector_type(2)));

constexpr int kStrThreads = 256;
constexpr int kStrVec = 4;                                   // 16-byte vectors per thread per sub-tile
constexpr int kSubVec = kStrThreads * kStrVec;               // vectors per sub-tile
constexpr int64_t kSub = (int64_t)kSubVec * 8;               // elements per sub-tile

__device__ __forceinline__ uint32_t key2(uint32_t x) {
  const i16x2 sx = __builtin_bit_cast(i16x2, x);
  const i16x2 sgn = sx >> (short)15;  // 0xFFFF for negative halves
  return x ^ (__builtin_bit_cast(uint32_t, sgn) | 0x80008000u);
}
__device__ __forceinline__ uint32_t pk_max(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b)));
}
__device__ __forceinline__ uint32_t pk_min(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b)));
}
template <bool F16>
__device__ __forceinline__ float half_to_f(uint32_t h) {
  if constexpr (F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  return __uint_as_float(h << 16);
}
__device__ __forceinline__ uint32_t key_to_bits(uint32_t k) { return (k & 0x8000u) ? (k ^ 0x8000u) : (~k & 0xFFFFu); }
// The bits of a 16-bit value held exactly as a float.
template <bool F16>
__device__ __forceinline__ uint32_t f_to_half_bits(float x) {
  if constexpr (F16) return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
  return __float_as_uint(x) >> 16;
}

template <bool F16, bool TYPICAL>
__global__ void __launch_bounds__(kStrThreads) accept_stream16_kernel(const AcceptArgs a) {
  constexpr uint32_t kNanAbove = F16 ? 0x7C00u : 0x7F80u;    // |bits| above: NaN
  constexpr uint32_t kNegInfBits = F16 ? 0xFC00u : 0xFF80u;
  constexpr uint32_t kLowest2 = F16 ? 0xFBFFFBFFu : 0xFF7FFF7Fu;  // lowest finite, both halves
  constexpr int kNw = kStrThreads / 64;
  const int c = blockIdx.x;
  const int64_t row = blockIdx.y;  // t * M + i
  const int t = (int)(row / a.M), i = (int)(row % a.M);
  const int64_t lo = (int64_t)c * a.chunk;
  const uint16_t* rb = reinterpret_cast<const uint16_t*>(a.logits) + (int64_t)t * a.l_st + (int64_t)i * a.l_sm + lo;
  const int n = (int)(min(lo + a.chunk, a.V) - lo);
  const int nvec = n >> 3;
  const int nsub = (nvec + kSubVec - 1) / kSubVec;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  __shared__ uint32_t red_u[kNw];
  __shared__ int red_i[kNw], red_n[kNw];
  __shared__ float red_m[kNw], red_l[kNw], red_s[kNw];

  // Vector v of sub-tile s of this thread: range vector s*kSubVec + tid + kStrThreads*v.
  // Vectors past the range hold -inf (they come after every real element);
  // their loads re-read the last vector, so that every load is unconditional
  // and the loads of the next sub-tile stay in flight (counted waits).
  const uint32_t pad = kNegInfBits | (kNegInfBits << 16);
  auto load = [&](int s, u32x4 (&r)[kStrVec]) {
#pragma unroll
    for (int v = 0; v < kStrVec; ++v) {
      const int vi = s * kSubVec + tid + kStrThreads * v;
      r[v] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rb) + min(vi, nvec - 1));
    }
  };
  auto pad_tail = [&](int s, u32x4 (&r)[kStrVec]) {
#pragma unroll
    for (int v = 0; v < kStrVec; ++v)
      if (s * kSubVec + tid + kStrThreads * v >= nvec) r[v] = u32x4{pad, pad, pad, pad};
  };

  uint32_t bk = 0;          // largest key seen (0: none; no number has key 0)
  int bs = -1;              // the sub-tile where it first occurred
  int nan_i = 0x7fffffff;   // first NaN index in the range
  float m = kNegInf, l = 0.f, sx = 0.f;
  const float zs = a.inv_temp * kLog2e;

  auto reduce_sub = [&](int s, u32x4 (&r)[kStrVec]) {
    if (s == nsub - 1) pad_tail(s, r);
    if (nan_i != 0x7fffffff) return;  // this thread's result is already NaN
    if constexpr (TYPICAL) {
      // The values as floats: their NaN-propagating maximum gives the NaN
      // test, the key of the maximum (+0 for a zero maximum: IEEE maximum
      // orders -0 below +0) and the softmax's reference.  The exponentials
      // then read the words again with -inf raised to the lowest finite value.
      float xv[kStrVec * 8];
#pragma unroll
      for (int v = 0; v < kStrVec; ++v)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          xv[8 * v + 2 * w] = half_to_f<F16>(r[v][w] & 0xFFFFu);
          xv[8 * v + 2 * w + 1] = half_to_f<F16>(r[v][w] >> 16);
        }
      float vmax = xv[0];
#pragma unroll
      for (int e = 1; e < kStrVec * 8; ++e) vmax = __builtin_elementwise_maximum(vmax, xv[e]);
      if (vmax != vmax) {  // rare: locate the first NaN
#pragma unroll
        for (int v = 0; v < kStrVec; ++v) {
          const int vi = s * kSubVec + tid + kStrThreads * v;
          for (int w = 0; w < 8 && nan_i == 0x7fffffff; ++w)
            if (vi < nvec && ((r[v][w >> 1] >> (16 * (w & 1))) & 0x7FFFu) > kNanAbove) nan_i = 8 * vi + w;
        }
        return;
      }
      const uint32_t km = key2(f_to_half_bits<F16>(vmax)) & 0xFFFFu;
      if (km > bk) {  // a larger maximum; its index is located at the end
        bk = km;
        bs = s;
      }
      const float mt = vmax * zs;
      if (mt > m) {
        const float sc = __builtin_amdgcn_exp2f(m - mt);  // m = -inf: 0
        l *= sc;
        sx *= sc;
        m = mt;
      }
      if (m != kNegInf) {
        float la = 0.f;
#pragma unroll
        for (int v = 0; v < kStrVec; ++v)
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const uint32_t cw = pk_min(r[v][w], kLowest2);  // -inf -> lowest finite (bits order = value order for < 0)
            const float x0 = half_to_f<F16>(cw & 0xFFFFu), x1 = half_to_f<F16>(cw >> 16);
            const float p0 = __builtin_amdgcn_exp2f(fmaf(x0, zs, -m));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(x1, zs, -m));
            la += p0 + p1;
            sx = fmaf(x0, p0, fmaf(x1, p1, sx));
          }
        l += la;
      }
      return;
    }
    uint32_t amax = 0, km = 0;
#pragma unroll
    for (int v = 0; v < kStrVec; ++v)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        amax = pk_max(amax, r[v][w] & 0x7FFF7FFFu);
        km = pk_max(km, key2(r[v][w]));
      }
    amax = max(amax & 0xFFFFu, amax >> 16);
    if (amax > kNanAbove) {  // rare: locate the first NaN
#pragma unroll
      for (int v = 0; v < kStrVec; ++v) {
        const int vi = s * kSubVec + tid + kStrThreads * v;
        for (int w = 0; w < 8 && nan_i == 0x7fffffff; ++w)
          if (vi < nvec && ((r[v][w >> 1] >> (16 * (w & 1))) & 0x7FFFu) > kNanAbove) nan_i = 8 * vi + w;
      }
      return;
    }
    km = max(km & 0xFFFFu, km >> 16);
    if (km > bk) {  // a larger maximum; its index is located at the end
      bk = km;
      bs = s;
    }
  };

  // Software pipeline: the loads of sub-tile s+1 are issued before sub-tile s
  // is reduced.  They are issued on every iteration (the last one re-reads
  // the last sub-tile) so that the wait counts are the same on every path.
  if (nsub > 0) {
    u32x4 cur[kStrVec], nxt[kStrVec];
    load(0, cur);
#pragma unroll 2
    for (int s = 0; s < nsub; ++s) {
      load(min(s + 1, nsub - 1), nxt);
      reduce_sub(s, cur);
#pragma unroll
      for (int v = 0; v < kStrVec; ++v) cur[v] = nxt[v];
    }
  }
  // Elements past the last whole vector (n % 8 of them), one per thread; they
  // follow every vector element of the range.
  const int ntail = n - 8 * nvec;
  if (tid < ntail && nan_i == 0x7fffffff) {
    const uint32_t h = rb[8 * nvec + tid];
    const int idx = 8 * nvec + tid;
    if ((h & 0x7FFFu) > kNanAbove) {
      nan_i = idx;
    } else {
      const uint32_t k = key2(h) & 0xFFFFu;
      if (k > bk) {
        bk = k;
        bs = nsub;  // the tail, past every sub-tile
      }
      if constexpr (TYPICAL) {
        const float mt = half_to_f<F16>(h) * zs;
        if (mt > m) {
          const float sc = __builtin_amdgcn_exp2f(m - mt);
          l *= sc;
          sx *= sc;
          m = mt;
        }
        if (m != kNegInf) {
          const float x = half_to_f<F16>(pk_min(h, kLowest2) & 0xFFFFu);
          const float p = __builtin_amdgcn_exp2f(fmaf(x, zs, -m));
          l += p;
          sx = fmaf(x, p, sx);
        }
      }
    }
  }

  // ---- workgroup reduction ---------------------------------------------------
  // NaN: first NaN index.  Else: largest key, then its first index.
  int nmin = nan_i;
  uint32_t kmax = bk;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    nmin = min(nmin, __shfl_xor(nmin, o));
    kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o));
  }
  if (lane == 0) {
    red_n[wv] = nmin;
    red_u[wv] = kmax;
  }
  __syncthreads();
  int nanf = red_n[0];
  uint32_t kstar = red_u[0];
#pragma unroll
  for (int x = 1; x < kNw; ++x) {
    nanf = min(nanf, red_n[x]);
    kstar = max(kstar, red_u[x]);
  }
  const bool has_nan = nanf != 0x7fffffff;
  int f = 0x7fffffff;
  if (!has_nan && bk == kstar && bs >= 0) {
    // This thread holds the maximum: its first index, from the sub-tile where
    // the thread's maximum first occurred, re-read with all of the thread's
    // vectors of it in flight at once (one round trip instead of one per
    // vector).
    if (bs == nsub) {
      f = 8 * nvec + tid;
    } else {
      u32x4 rr[kStrVec];
#pragma unroll
      for (int v = 0; v < kStrVec; ++v)
        rr[v] = reinterpret_cast<const u32x4*>(rb)[min(bs * kSubVec + tid + kStrThreads * v, nvec - 1)];
#pragma unroll
      for (int v = 0; v < kStrVec; ++v) {
        const int vi = bs * kSubVec + tid + kStrThreads * v;
#pragma unroll
        for (int w = 0; w < 8; ++w)
          if (f == 0x7fffffff && vi < nvec &&
              (key2((rr[v][w >> 1] >> (16 * (w & 1))) & 0xFFFFu) & 0xFFFFu) == kstar)
            f = 8 * vi + w;
      }
    }
  }
  if (!has_nan && kstar == 0x8000u) {
    // Maximum +0: the first zero of either sign, rescanned exactly.
    f = 0x7fffffff;
    for (int vi = tid; vi < nvec && f == 0x7fffffff; vi += kStrThreads) {
      const u32x4 r = reinterpret_cast<const u32x4*>(rb)[vi];
      for (int w = 0; w < 8; ++w)
        if (((r[w >> 1] >> (16 * (w & 1))) & 0x7FFFu) == 0) {
          f = 8 * vi + w;
          break;
        }
    }
    if (f == 0x7fffffff && tid < ntail && (rb[8 * nvec + tid] & 0x7FFFu) == 0) f = 8 * nvec + tid;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) f = min(f, __shfl_xor(f, o));
  // Typical statistics of the wave, merged against the wave maximum.
  if constexpr (TYPICAL) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float mo = __shfl_xor(m, o), lo2 = __shfl_xor(l, o), so = __shfl_xor(sx, o);
      const float mn = fmaxf(m, mo);
      if (mn != kNegInf) {
        const float fa = __builtin_amdgcn_exp2f(m - mn), fb = __builtin_amdgcn_exp2f(mo - mn);
        l = l * fa + lo2 * fb;
        sx = sx * fa + so * fb;
      }
      m = mn;
    }
  }
  __syncthreads();
  if (lane == 0) {
    red_i[wv] = f;
    red_m[wv] = m;
    red_l[wv] = l;
    red_s[wv] = sx;
  }
  __syncthreads();
  if (tid == 0) {
    int fbest = red_i[0];
    float M = red_m[0], L = red_l[0], S = red_s[0];
#pragma unroll
    for (int x = 1; x < kNw; ++x) {
      fbest = min(fbest, red_i[x]);
      if constexpr (TYPICAL) {
        const float mn = fmaxf(M, red_m[x]);
        if (mn != kNegInf) {
          const float fa = __builtin_amdgcn_exp2f(M - mn), fb = __builtin_amdgcn_exp2f(red_m[x] - mn);
          L = L * fa + red_l[x] * fb;
          S = S * fa + red_s[x] * fb;
        }
        M = mn;
      }
    }
    const float qnan = __builtin_nanf("");
    float vbest, mz = kNegInf, lsum = 0.f, ssum = 0.f;
    int ibest;
    if (has_nan) {
      vbest = qnan;
      ibest = nanf;
      if constexpr (TYPICAL) mz = lsum = ssum = qnan;
    } else {
      vbest = half_to_f<F16>(key_to_bits(kstar));
      ibest = fbest;
      if constexpr (TYPICAL) {
        mz = M;
        if (M != kNegInf) {
          lsum = L;
          ssum = S * a.inv_temp;
        }
      }
    }
    const int64_t o = row * a.nchunk + c;
    a.rstat[o] = make_float4(vbest, __int_as_float((int)(lo + ibest)), mz, lsum);
    if constexpr (TYPICAL) a.rstat2[o] = ssum;
  }
}

// Relative margin around the typical threshold within which the fp32
// decision is not trusted.  The sweep's statistics carry relative errors of
// about 2^-16 from the fp32 sums (at most a few hundred terms per thread,
// then tree merges) plus 2^-20 (1 + |m| + 12) from the per-element
// exponentials and the rounded 1/T log2(e) (weighted by the probabilities,
// whose mean distance below the maximum m is at most the entropy, <= ln V);
// the entropy's error, through s / l, is that relative error times at most
// |m| + 13 (natural units).  At |m| = 10 this is below 1e-3 relative in the
// threshold; the margin 2^-7 (1 + |m| / 16) is more than ten times the bound.
__device__ __forceinline__ float typical_margin(float m_log2) {
  return 0x1p-7f * (1.f + fabsf(m_log2 * kLn2) * 0.0625f);
}

__device__ __forceinline__ double logit_at(const AcceptArgs& a, int64_t off) {
  if (a.l_dtype == 0) return (double)__uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(a.logits)[off] << 16);
  if (a.l_dtype == 1) return (double)(float)reinterpret_cast<const _Float16*>(a.logits)[off];
  return (double)reinterpret_cast<const float*>(a.logits)[off];
}

// Block-wide reductions of a double (every thread gets the result).
__device__ __forceinline__ double block_sum_d(double v, double* scratch) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int nw = (blockDim.x + 63) >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  double r = 0.0;
  for (int w = 0; w < nw; ++w) r += scratch[w];
  return r;
}
// Maximum that propagates NaN (numpy's max).
__device__ __forceinline__ double nan_max(double x, double y) { return (x != x || y != y) ? x + y : (x > y ? x : y); }
__device__ __forceinline__ double block_max_d(double v, double* scratch) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = nan_max(v, __shfl_xor(v, o));
  const int nw = (blockDim.x + 63) >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  double r = scratch[0];
  for (int w = 1; w < nw; ++w) r = nan_max(r, scratch[w]);
  return r;
}

// The typical test of every flagged node (okv[n] == 2) decided from float64
// statistics of its parent's row, the definition's own arithmetic:
//   y = x / T, m = max y, z = sum e^(y - m), H = m + ln z - sum_{e > 0} e^(y - m) y / z,
//   accept iff e^(y_tok - m) / z > min(eps, alpha e^-H)
// with T, eps and alpha the arguments as given (float).  The whole workgroup
// takes one flagged node at a time: two passes over the parent's row.
__device__ __forceinline__ void typical_recheck(const AcceptArgs& a, int t, const int* par, int* okv, const float* xtok) {
  __shared__ double scratch[16];
  const double T = (double)a.temperature;
  const int64_t V = a.V;
  for (int n = 1; n < a.M; ++n) {
    if (okv[n] != 2) continue;  // uniform: every thread reads the same LDS word
    const int64_t base = (int64_t)t * a.l_st + (int64_t)par[n] * a.l_sm;
    double mx = -__builtin_huge_val();
    for (int64_t v = threadIdx.x; v < V; v += blockDim.x) mx = nan_max(mx, logit_at(a, base + v) / T);
    mx = block_max_d(mx, scratch);
    double z = 0.0, sy = 0.0;
    for (int64_t v = threadIdx.x; v < V; v += blockDim.x) {
      const double y = logit_at(a, base + v) / T;
      const double e = exp(y - mx);
      z += e;
      if (e > 0.0) sy += e * y;
    }
    z = block_sum_d(z, scratch);
    sy = block_sum_d(sy, scratch);
    const double ent = mx + log(z) - sy / z;
    const double prob = exp((double)xtok[n] / T - mx) / z;
    const double thr = fmin((double)a.eps, (double)a.alpha * exp(-ent));
    __syncthreads();
    if (threadIdx.x == 0) okv[n] = prob > thr;
    __syncthreads();
  }
}

__global__ void __launch_bounds__(1024) accept_walk_kernel(const AcceptArgs a) {
  extern __shared__ int64_t smem64[];
  const int M = a.M;
  const int t = blockIdx.x;
  const int i = threadIdx.x;
  // LDS carve-up: par[M] int, nxt[M] int, ok[M] int, mz[M], lz[M], hz[M] float,
  // path[M] int, reduction scratch.
  int* par = reinterpret_cast<int*>(smem64);
  int* nxt = par + M;
  int* okv = nxt + M;
  float* mz = reinterpret_cast<float*>(okv + M);
  float* lz = mz + M;
  float* hz = lz + M;
  int* path = reinterpret_cast<int*>(hz + M);
  int64_t* red_v = reinterpret_cast<int64_t*>(smem64) + (((int64_t)7 * M + 1) / 2 + 1);
  int* red_i = reinterpret_cast<int*>(red_v + 16);
  __shared__ int s_err;
  if (i == 0) s_err = 0;
  __syncthreads();

  // Every global load a node needs is issued up front (one round trip for
  // the statistics, parent, draft token and position; one more for the
  // typical test's logit, addressed by the node's own parent and token).
  int64_t tok = 0, pv = 0, praw = -1;
  if (i < M) {
    tok = a.draft[(int64_t)t * a.d_st + (int64_t)i * a.d_sm];
    pv = a.pos[(int64_t)t * a.pos_st + (int64_t)i * a.pos_sm];
    if (i > 0) praw = a.parent[(int64_t)t * a.p_st + (int64_t)(i - 1) * a.p_sm];
  }
  if (i < M) {
    // 1. Combine vocab-chunk statistics of row (t, i), four chunks per round trip.
    const int64_t row = (int64_t)t * M + i;
    float bv = kNegInf;
    int bi = -1;
    Soft sm{kNegInf, 0.f, 0.f};
    if (a.mode == 2) {
      // Sampling: the ranges' Gumbel-max draws (z as a double, index; -1 =
      // nothing kept); the largest z wins, then the lowest index.
      double bz = 0.0;
      for (int c = 0; c < a.nchunk; ++c) {
        const float4 st = a.rstat[row * a.nchunk + c];
        const int ci = __float_as_int(st.z);
        const double z = __builtin_bit_cast(
            double, (uint64_t)__float_as_uint(st.x) | ((uint64_t)__float_as_uint(st.y) << 32));
        if (ci >= 0 && (bi < 0 || z > bz || (z == bz && ci < bi))) {
          bz = z;
          bi = ci;
        }
      }
      if (bi < 0) bi = 0;
    }
    for (int c0 = 0; a.mode != 2 && c0 < a.nchunk; c0 += 4) {
      float4 st[4];
      float s2[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int c = min(c0 + u, a.nchunk - 1);
        st[u] = a.rstat[row * a.nchunk + c];
        s2[u] = a.mode == 1 ? a.rstat2[row * a.nchunk + c] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (c0 + u >= a.nchunk) break;
        const int ci = __float_as_int(st[u].y);
        if (ci >= 0 && (bi < 0 || am_better(st[u].x, ci, bv, bi))) {
          bv = st[u].x;
          bi = ci;
        }
        if (a.mode == 1) sm = soft_merge(sm, Soft{st[u].z, st[u].w, s2[u]});
      }
    }
    nxt[i] = bi;
    mz[i] = sm.m;
    lz[i] = sm.l;
    // H = ln2 * (m + log2 l) - s / l
    hz[i] = (sm.l > 0.f) ? kLn2 * (sm.m + __log2f(sm.l)) - sm.s / sm.l : 0.f;
    if (a.out_next != nullptr) a.out_next[(int64_t)t * a.on_st + i] = bi;

    // 2. Extended parent (root = node 0 points to itself).
    int pe = 0;
    if (i > 0) {
      const int k = i - 1;
      int64_t p = praw;
      if (p == k) p = -1;
      if (p < -1 || p >= M - 1) {
        atomicOr(&s_err, 1);
        p = -1;
      }
      pe = (int)p + 1;
    }
    par[i] = pe;
  }
  // Typical: the draft token's logit under the parent's distribution.
  float xtok = 0.f;
  bool tok_ok = false;
  if (i > 0 && i < M && a.mode == 1) {
    const int p = par[i];  // written by this thread
    tok_ok = tok >= 0 && tok < a.V;
    if (tok_ok && a.xtok != nullptr) {
      xtok = a.xtok[(int64_t)t * M + i];  // computed with the statistics (fused lm_head)
    } else if (tok_ok) {
      const int64_t off = (int64_t)t * a.l_st + (int64_t)p * a.l_sm + tok;
      if (a.l_dtype == 0)
        xtok = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(a.logits)[off] << 16);
      else if (a.l_dtype == 1)
        xtok = (float)reinterpret_cast<const _Float16*>(a.logits)[off];
      else
        xtok = reinterpret_cast<const float*>(a.logits)[off];
    }
  }
  __syncthreads();

  // 3. Per-node acceptance test against the parent's distribution.  The
  // typical test is decided from the sweep's fp32 statistics unless the
  // draft token's probability lies within the margin typical_margin() of the
  // threshold: such nodes (okv = 2) are decided again from float64
  // statistics of the parent's row, below (with the fused lm_head, only when
  // it writes the logits: a.logits is null otherwise).
  bool recheck = false;
  if (i < M) {
    int ok = 1;
    if (i > 0) {
      const int p = par[i];
      if (a.mode != 1) {
        ok = (tok == (int64_t)nxt[p]);
      } else {
        ok = 0;
        if (tok_ok && lz[p] > 0.f) {
          const float prob = __builtin_amdgcn_exp2f(fmaf(xtok, a.inv_temp * kLog2e, -mz[p])) / lz[p];
          const float thr = fminf(a.eps, a.alpha * __expf(-hz[p]));
          ok = prob > thr;
          recheck = a.logits != nullptr && prob == prob && thr == thr &&
                    fabsf(prob - thr) <= typical_margin(mz[p]) * thr;
        }
      }
    }
    okv[i] = recheck ? 2 : ok;
  }
  if (a.mode == 1 && __syncthreads_or(recheck)) {  // a.mode is uniform
    // The flagged nodes' draft-token logits (lz is not read again).
    if (recheck) lz[i] = xtok;
    __syncthreads();
    typical_recheck(a, t, par, okv, lz);
  }
  __syncthreads();

  // 4. Bounded ancestor closure + masked position value.  The draft tokens
  // go to LDS for the path output: 8-byte aligned from the start of mz, over
  // mz, lz and at most 4 bytes of hz, all read for the last time in step 3.
  int64_t* tok_lds = smem64 + (3 * M + 1) / 2;
  int64_t val = INT64_MIN;
  int vidx = 0x7fffffff;
  if (i < M) {
    tok_lds[i] = tok;
    int okc = okv[i];
    int node = i;
    for (int h = 0; h < a.max_hops && okc && node != 0; ++h) {  // the root's parent is itself
      node = par[node];
      okc &= okv[node];
    }
    val = okc ? pv : 0;
    vidx = i;
  }
  // 5. argmax(val), first index on ties: wave then block reduction.
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const int64_t ov = __shfl_xor(val, o);
    const int oi = __shfl_xor(vidx, o);
    if (ov > val || (ov == val && oi < vidx)) {
      val = ov;
      vidx = oi;
    }
  }
  const int wid = i >> 6;
  if ((i & 63) == 0) {
    red_v[wid] = val;
    red_i[wid] = vidx;
  }
  __syncthreads();

  // 6. Traceback (one thread; path length <= M).
  if (i == 0) {
    const int nw = (blockDim.x + 63) >> 6;
    int64_t bvv = red_v[0];
    int bi = red_i[0];
    for (int x = 1; x < nw; ++x)
      if (red_v[x] > bvv || (red_v[x] == bvv && red_i[x] < bi)) {
        bvv = red_v[x];
        bi = red_i[x];
      }
    int len = 0;
    int cur = bi;
    while (cur != -1 && len < M) {
      path[len++] = cur;
      cur = (cur == 0) ? -1 : par[cur];
    }
    if (cur != -1) s_err = 1;
    // reverse in place (root first)
    for (int x = 0; x < len / 2; ++x) {
      const int tmp = path[x];
      path[x] = path[len - 1 - x];
      path[len - 1 - x] = tmp;
    }
    red_i[0] = bi;
    red_i[1] = len;
  }
  __syncthreads();
  const int winner = red_i[0];
  const int len = red_i[1];
  for (int k = i; k < M; k += blockDim.x) {
    int64_t pid = -1, tok = -1;
    if (k < len) {
      pid = path[k];
      tok = tok_lds[pid];
    }
    a.out_path[(int64_t)t * a.op_st + k] = pid;
    a.out_tok[(int64_t)t * a.ot_st + k] = tok;
  }
  if (i == 0) {
    int64_t* info = a.out_info + (int64_t)t * a.oi_st;
    info[0] = winner;
    info[1] = len - 1;
    info[2] = nxt[winner];
    info[3] = s_err ? -1 : len;
  }
}

template <bool F16>
hipError_t launch_stream16(const AcceptArgs& a, hipStream_t s) {
  dim3 grid((unsigned)a.nchunk, (unsigned)((int64_t)a.T * a.M));
  if (a.mode == 1)
    hipLaunchKernelGGL((accept_stream16_kernel<F16, true>), grid, dim3(kStrThreads), 0, s, a);
  else
    hipLaunchKernelGGL((accept_stream16_kernel<F16, false>), grid, dim3(kStrThreads), 0, s, a);
  return hipGetLastError();
}

template <typename LT>
hipError_t launch_rowstat(const AcceptArgs& a, hipStream_t s) {
  dim3 grid((unsigned)a.nchunk, (unsigned)((int64_t)a.T * a.M));
  if (a.mode == 1)
    hipLaunchKernelGGL((accept_rowstat_kernel<LT, true>), grid, dim3(kRowThreads), 0, s, a);
  else
    hipLaunchKernelGGL((accept_rowstat_kernel<LT, false>), grid, dim3(kRowThreads), 0, s, a);
  return hipGetLastError();
}

// Reduces the nin partial statistics of every row (row-major [rows, nin])
// to one per row in a.rstat / a.rstat2 (a.nchunk == 1): argmax with the
// lowest index on ties, softmax statistics by rescaled merges.
template <bool TYPICAL>
__global__ void __launch_bounds__(kRowThreads) accept_combine_kernel(const AcceptArgs a, const float4* part,
                                                                     const float* part2, int nin) {
  const int64_t row = blockIdx.x;
  ArgMax best{kNegInf, 0x7fffffff};
  bool have = false;
  Soft sm{kNegInf, 0.f, 0.f};
  for (int c = threadIdx.x; c < nin; c += kRowThreads) {
    const float4 st = part[row * nin + c];
    const int ci = __float_as_int(st.y);
    if (ci >= 0 && (!have || am_better(st.x, ci, best.v, best.i))) {
      best.v = st.x;
      best.i = ci;
      have = true;
    }
    if constexpr (TYPICAL) sm = soft_merge(sm, Soft{st.z, st.w, part2[row * nin + c]});
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best.v, o);
    const int oi = __shfl_xor(best.i, o);
    const int oh = __shfl_xor((int)have, o);
    if (oh && (!have || am_better(ov, oi, best.v, best.i))) {
      best.v = ov;
      best.i = oi;
      have = true;
    }
    if constexpr (TYPICAL) {
      Soft other{__shfl_xor(sm.m, o), __shfl_xor(sm.l, o), __shfl_xor(sm.s, o)};
      sm = soft_merge(sm, other);
    }
  }
  __shared__ float sv[kRowThreads / 64], sm_m[kRowThreads / 64], sm_l[kRowThreads / 64], sm_s[kRowThreads / 64];
  __shared__ int si[kRowThreads / 64], sh[kRowThreads / 64];
  const int wid = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wid] = best.v;
    si[wid] = best.i;
    sh[wid] = have;
    sm_m[wid] = sm.m;
    sm_l[wid] = sm.l;
    sm_s[wid] = sm.s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int x = 1; x < kRowThreads / 64; ++x) {
      if (sh[x] && (!have || am_better(sv[x], si[x], best.v, best.i))) {
        best.v = sv[x];
        best.i = si[x];
        have = true;
      }
      if constexpr (TYPICAL) sm = soft_merge(sm, Soft{sm_m[x], sm_l[x], sm_s[x]});
    }
    a.rstat[row] = make_float4(best.v, __int_as_float(have ? best.i : -1), sm.m, sm.l);
    if constexpr (TYPICAL) a.rstat2[row] = sm.s;
  }
}

}  // namespace

size_t accept_walk_lds_bytes(int M);

// The walk runs one thread per node; in typical mode at least 256 threads,
// so that the re-check streams a row with a whole workgroup.
static int walk_threads(const AcceptArgs& a) {
  const int t = ((a.M + 63) / 64) * 64;
  return a.mode == 1 ? std::max(256, t) : t;
}

hipError_t launch_accept_from_parts(const AcceptArgs& a, const float4* part, const float* part2, int nin,
                                    hipStream_t s) {
  if (a.T <= 0 || a.M <= 0) return hipSuccess;
  const dim3 grid((unsigned)((int64_t)a.T * a.M));
  if (a.mode == 1)
    hipLaunchKernelGGL(accept_combine_kernel<true>, grid, dim3(kRowThreads), 0, s, a, part, part2, nin);
  else
    hipLaunchKernelGGL(accept_combine_kernel<false>, grid, dim3(kRowThreads), 0, s, a, part, part2, nin);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int threads = walk_threads(a);
  hipLaunchKernelGGL(accept_walk_kernel, dim3((unsigned)a.T), dim3(threads), accept_walk_lds_bytes(a.M), s, a);
  return hipGetLastError();
}

size_t accept_walk_lds_bytes(int M) {
  // par, nxt, ok, mz, lz, hz, path: 7*M words, plus reduction scratch.
  return ((size_t)7 * M + 1) / 2 * 8 + 8 + 16 * 8 + 16 * 4 + 64;
}

// 16-bit logits with 16-byte aligned rows stream their rows in ranges of
// whole sub-tiles (per_cu workgroups per CU over all rows, below); other
// logits take fixed chunks of kChunkGeneric elements.
constexpr int64_t kChunkGeneric = 16384;

static bool stream16_ok(const AcceptArgs& a) {
  return a.l_dtype != 2 && ((uintptr_t)a.logits & 15) == 0 && (a.l_st * 2) % 16 == 0 && (a.l_sm * 2) % 16 == 0;
}

void accept_chunking(AcceptArgs& a, int cus) {
  a.cus = cus;
  if (stream16_ok(a)) {
    const int64_t rows = (int64_t)a.T * a.M, nsub = (a.V + kSub - 1) / kSub;
    // Greedy / typical: about one workgroup per CU over all rows (fewer,
    // longer streams measured 5% faster at 8 trees of 64 nodes and 15-19% at
    // one tree than four per CU); the sampling kernels keep four per CU.
    const int64_t per_cu = a.mode == 2 ? 4 : 1;
    const int64_t want = std::max<int64_t>(1, (per_cu * cus + rows - 1) / rows);
    const int64_t nb = std::min(want, nsub);
    a.chunk = ((a.V + nb - 1) / nb + kSub - 1) / kSub * kSub;
  } else {
    a.chunk = kChunkGeneric;
  }
  a.nchunk = (int)((a.V + a.chunk - 1) / a.chunk);
}

int64_t accept_max_chunks(int64_t V) { return (V + kSub - 1) / kSub; }

hipError_t launch_accept(const AcceptArgs& a, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  if (a.T <= 0 || a.M <= 0) return hipSuccess;
  hipError_t e;
  if (ev0 != nullptr && (e = hipEventRecord(ev0, s)) != hipSuccess) return e;
  // The streaming kernel needs 16-byte aligned rows and ranges (chunks of
  // whole sub-tiles, from accept_chunking).
  const bool st16 = stream16_ok(a) && a.chunk % kSub == 0;
  if (a.l_dtype == 0)
    e = st16 ? launch_stream16<false>(a, s) : launch_rowstat<uint16_t>(a, s);
  else if (a.l_dtype == 1)
    e = st16 ? launch_stream16<true>(a, s) : launch_rowstat<_Float16>(a, s);
  else
    e = launch_rowstat<float>(a, s);
  if (e != hipSuccess) return e;
  if (ev1 != nullptr && (e = hipEventRecord(ev1, s)) != hipSuccess) return e;
  return launch_walk(a, s);
}

hipError_t launch_walk(const AcceptArgs& a, hipStream_t s) {
  const int threads = walk_threads(a);
  hipLaunchKernelGGL(accept_walk_kernel, dim3((unsigned)a.T), dim3(threads), accept_walk_lds_bytes(a.M), s, a);
  return hipGetLastError();
}

}  // namespace dsv
