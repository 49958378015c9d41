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

#include "dsv_internal.h"

namespace dsv {

namespace {

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634074f;
constexpr float kLn2 = 0.69314718055994530942f;
constexpr int kRowThreads = 256;

struct ArgMax {
  float v;
  int i;
};

// a ranks before b: larger value, NaN above all numbers, ties -> lower index.
__device__ __forceinline__ bool am_better(float av, int ai, float bv, int bi) {
  const bool an = av != av, bn = bv != bv;
  if (an || bn) return an && (!bn || ai < bi);
  if (av != bv) return av > bv;
  return ai < bi;
}

struct Soft {
  float m;  // max of y*log2e
  float l;  // sum 2^(z - m)
  float s;  // sum y * 2^(z - m)
};

__device__ __forceinline__ Soft soft_merge(Soft a, Soft b) {
  if (a.m == kNegInf) return b;
  if (b.m == kNegInf) return a;
  const float m = fmaxf(a.m, b.m);
  const float fa = __builtin_amdgcn_exp2f(a.m - m), fb = __builtin_amdgcn_exp2f(b.m - m);
  return Soft{m, a.l * fa + b.l * fb, a.s * fa + b.s * fb};
}

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
          sm.s = fmaf(xs[e] * a.inv_temp, p, sm.s);
        }
      }
    }
  };

  const bool aligned = ((reinterpret_cast<uintptr_t>(base + lo) & 15) == 0);
  if (aligned) {
    const int64_t nvec = (hi - lo) / VEC;
    for (int64_t vi = threadIdx.x; vi < nvec; vi += kRowThreads) {
      const u32x4 raw = *reinterpret_cast<const u32x4*>(base + lo + vi * VEC);
      float xs[VEC];
      const LT* el = reinterpret_cast<const LT*>(&raw);
#pragma unroll
      for (int e = 0; e < VEC; ++e) xs[e] = to_f<LT>(el[e]);
      consume(xs, VEC, lo + vi * VEC);
    }
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
// Stage A for 16-bit logits (bf16 / f16), rows 16-byte aligned.
//
// A 16-bit float maps to an unsigned key that orders like the value:
// key = bits ^ (bits < 0 ? 0xFFFF : 0x8000) (sign-magnitude -> offset), so
// the argmax is "largest key, then lowest index".  Keys are formed two per
// dword with packed 16-bit ops (v_pk_ashrrev_i16 / v_pk_max_u16), the chunk's
// maximum key is reduced over the workgroup, and a second pass over the
// register-resident data finds the first index holding it (a thread that has
// a hit - rare - locates it with a scalar scan).  A chunk containing a NaN
// takes an exact slow path in which every NaN gets the largest key (torch
// ranks NaN above all numbers, first index wins).  Typical statistics reuse
// the chunk maximum as m, so one exp2, two FMAs and an add per element remain.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef short i16x2 __attribute__((ext_vector_type(2)));

constexpr int kVecPerThread = 8;  // 16-byte vectors per thread (chunk <= 256 * 8 * 8 elements)

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

template <bool F16, bool TYPICAL>
__global__ void __launch_bounds__(kRowThreads) accept_rowstat16_kernel(const AcceptArgs a) {
  constexpr uint32_t kNanAbove = F16 ? 0x7C00u : 0x7F80u;  // |bits| above: NaN
  constexpr uint32_t kNegInfBits = F16 ? 0xFC00u : 0xFF80u;
  constexpr int kNw = kRowThreads / 64;
  const int c = blockIdx.x;
  const int64_t row = blockIdx.y;  // t * M + i
  const int t = (int)(row / a.M), i = (int)(row % a.M);
  const uint16_t* base = reinterpret_cast<const uint16_t*>(a.logits) + (int64_t)t * a.l_st + (int64_t)i * a.l_sm;
  const int64_t lo = (int64_t)c * a.chunk;
  const int n = (int)(min(lo + a.chunk, a.V) - lo);
  const int nvec = n >> 3;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  __shared__ uint32_t red_u[kNw];
  __shared__ float red_l[kNw], red_s[kNw];

  // Vector v of this thread covers chunk elements [8 * (tid + 256 v), +8);
  // vectors past the chunk hold -inf (they come after every real element).
  const uint32_t pad = kNegInfBits | (kNegInfBits << 16);
  u32x4 raw[kVecPerThread];
#pragma unroll
  for (int v = 0; v < kVecPerThread; ++v) {
    const int vi = tid + kRowThreads * v;
    raw[v] = vi < nvec ? *reinterpret_cast<const u32x4*>(base + lo + 8 * vi) : u32x4{pad, pad, pad, pad};
  }
  // Elements past the last whole vector (n % 8 of them), one per thread.
  const int ntail = n - 8 * nvec;
  uint32_t tail_bits = kNegInfBits;
  if (tid < ntail) tail_bits = base[lo + 8 * nvec + tid];

  // NaN anywhere in the chunk?
  uint32_t amax = tail_bits & 0x7FFFu;
#pragma unroll
  for (int v = 0; v < kVecPerThread; ++v)
#pragma unroll
    for (int w = 0; w < 4; ++w) amax = pk_max(amax, raw[v][w] & 0x7FFF7FFFu);
  amax = max(amax & 0xFFFFu, amax >> 16);
  const bool chunk_nan = __syncthreads_or(amax > kNanAbove) != 0;

  // Largest key.
  uint32_t kbest = 0;
  if (!chunk_nan) {
#pragma unroll
    for (int v = 0; v < kVecPerThread; ++v)
#pragma unroll
      for (int w = 0; w < 4; ++w) kbest = pk_max(kbest, key2(raw[v][w]));
    kbest = max(kbest & 0xFFFFu, kbest >> 16);
    kbest = max(kbest, key2(tail_bits) & 0xFFFFu);
  } else {
    // Exact path: NaN halves take the largest key.
    auto nkey = [&](uint32_t h) { return (h & 0x7FFFu) > kNanAbove ? 0xFFFFu : (key2(h) & 0xFFFFu); };
#pragma unroll
    for (int v = 0; v < kVecPerThread; ++v)
#pragma unroll
      for (int w = 0; w < 4; ++w) kbest = max(kbest, max(nkey(raw[v][w] & 0xFFFFu), nkey(raw[v][w] >> 16)));
    kbest = max(kbest, nkey(tail_bits));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) kbest = max(kbest, (uint32_t)__shfl_xor((int)kbest, o));
  if (lane == 0) red_u[wv] = kbest;
  __syncthreads();
  uint32_t kstar = red_u[0];
#pragma unroll
  for (int x = 1; x < kNw; ++x) kstar = max(kstar, red_u[x]);
  __syncthreads();

  // A zero maximum: -0 and +0 compare equal (keys 0x7FFF and 0x8000), so
  // both count as hits and the exact scan runs.
  const bool zmax = !chunk_nan && (kstar == 0x7FFFu || kstar == 0x8000u);
  if (zmax) kstar = 0x8000u;

  // First index holding kstar.
  int first = 0x7fffffff;
  {
    auto hkey = [&](uint32_t h) {
      const uint32_t k = chunk_nan && (h & 0x7FFFu) > kNanAbove ? 0xFFFFu : (key2(h) & 0xFFFFu);
      return (zmax && k == 0x7FFFu) ? 0x8000u : k;
    };
    bool hit;
    if (!chunk_nan && !zmax) {
      const uint32_t kk = kstar | (kstar << 16);
      uint32_t accz = 0x00010001u;
#pragma unroll
      for (int v = 0; v < kVecPerThread; ++v)
#pragma unroll
        for (int w = 0; w < 4; ++w) accz &= pk_min(key2(raw[v][w]) ^ kk, 0x00010001u);
      hit = accz != 0x00010001u;
    } else {
      hit = true;
    }
    if (hit) {
      for (int v = 0; v < kVecPerThread && first == 0x7fffffff; ++v) {
        const int vi = tid + kRowThreads * v;
        if (vi >= nvec) break;
        for (int w = 0; w < 8; ++w) {
          const uint32_t h = (raw[v][w >> 1] >> (16 * (w & 1))) & 0xFFFFu;
          if (hkey(h) == kstar) {
            first = 8 * vi + w;
            break;
          }
        }
      }
    }
    if (first == 0x7fffffff && tid < ntail && hkey(tail_bits) == kstar) first = 8 * nvec + tid;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) first = min(first, __shfl_xor(first, o));
  if (lane == 0) red_u[wv] = (uint32_t)first;
  __syncthreads();
  int fbest = (int)red_u[0];
#pragma unroll
  for (int x = 1; x < kNw; ++x) fbest = min(fbest, (int)red_u[x]);

  const float vbest = chunk_nan && kstar == 0xFFFFu ? __builtin_nanf("") : half_to_f<F16>(key_to_bits(kstar));

  // Typical statistics against m = max(x) * log2(e) / T.
  float mz = kNegInf, lsum = 0.f, ssum = 0.f;
  if constexpr (TYPICAL) {
    const float zs = a.inv_temp * kLog2e;
    mz = vbest * zs;
    if (mz != kNegInf) {
      float l = 0.f, sx = 0.f;
#pragma unroll
      for (int v = 0; v < kVecPerThread; ++v)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float x0 = half_to_f<F16>(raw[v][w] & 0xFFFFu), x1 = half_to_f<F16>(raw[v][w] >> 16);
          const float p0 = __builtin_amdgcn_exp2f(fmaf(x0, zs, -mz));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(x1, zs, -mz));
          l += p0 + p1;
          sx = fmaf(x0, p0, fmaf(x1, p1, sx));
        }
      if (tid < ntail) {
        const float x = half_to_f<F16>(tail_bits);
        const float p = __builtin_amdgcn_exp2f(fmaf(x, zs, -mz));
        l += p;
        sx = fmaf(x, p, sx);
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        l += __shfl_xor(l, o);
        sx += __shfl_xor(sx, o);
      }
      __syncthreads();
      if (lane == 0) {
        red_l[wv] = l;
        red_s[wv] = sx;
      }
      __syncthreads();
      lsum = red_l[0];
      ssum = red_s[0];
#pragma unroll
      for (int x = 1; x < kNw; ++x) {
        lsum += red_l[x];
        ssum += red_s[x];
      }
      ssum *= a.inv_temp;
    }
  }
  if (tid == 0) {
    const int64_t o = row * a.nchunk + c;
    a.rstat[o] = make_float4(vbest, __int_as_float((int)(lo + fbest)), mz, lsum);
    if constexpr (TYPICAL) a.rstat2[o] = ssum;
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

  if (i < M) {
    // 1. Combine vocab-chunk statistics of row (t, i).
    const int64_t row = (int64_t)t * M + i;
    float bv = kNegInf;
    int bi = -1;
    Soft sm{kNegInf, 0.f, 0.f};
    for (int c = 0; c < a.nchunk; ++c) {
      const float4 st = a.rstat[row * a.nchunk + c];
      const int ci = __float_as_int(st.y);
      if (ci >= 0 && (bi < 0 || am_better(st.x, ci, bv, bi))) {
        bv = st.x;
        bi = ci;
      }
      if (a.mode == 1) sm = soft_merge(sm, Soft{st.z, st.w, a.rstat2[row * a.nchunk + c]});
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
      int64_t p = a.parent[(int64_t)t * a.p_st + (int64_t)k * a.p_sm];
      if (p == k) p = -1;
      if (p < -1 || p >= M - 1) {
        atomicOr(&s_err, 1);
        p = -1;
      }
      pe = (int)p + 1;
    }
    par[i] = pe;
  }
  __syncthreads();

  // 3. Per-node acceptance test against the parent's distribution.
  if (i < M) {
    int ok = 1;
    if (i > 0) {
      const int p = par[i];
      const int64_t tok = a.draft[(int64_t)t * a.d_st + (int64_t)i * a.d_sm];
      if (a.mode == 0) {
        ok = (tok == (int64_t)nxt[p]);
      } else {
        ok = 0;
        if (tok >= 0 && tok < a.V && lz[p] > 0.f) {
          const int64_t off = (int64_t)t * a.l_st + (int64_t)p * a.l_sm + tok;
          float x;
          if (a.l_dtype == 0)
            x = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(a.logits)[off] << 16);
          else if (a.l_dtype == 1)
            x = (float)reinterpret_cast<const _Float16*>(a.logits)[off];
          else
            x = reinterpret_cast<const float*>(a.logits)[off];
          const float prob = __builtin_amdgcn_exp2f(fmaf(x, a.inv_temp * kLog2e, -mz[p])) / lz[p];
          const float thr = fminf(a.eps, a.alpha * __expf(-hz[p]));
          ok = prob > thr;
        }
      }
    }
    okv[i] = ok;
  }
  __syncthreads();

  // 4. Bounded ancestor closure + masked position value.
  int64_t val = INT64_MIN;
  int vidx = 0x7fffffff;
  if (i < M) {
    int okc = okv[i];
    int node = i;
    for (int h = 0; h < a.max_hops && okc; ++h) {
      node = par[node];
      okc &= okv[node];
    }
    const int64_t pv = a.pos[(int64_t)t * a.pos_st + (int64_t)i * a.pos_sm];
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
      tok = a.draft[(int64_t)t * a.d_st + pid * a.d_sm];
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
hipError_t launch_rowstat16(const AcceptArgs& a, hipStream_t s) {
  dim3 grid((unsigned)a.nchunk, (unsigned)((int64_t)a.T * a.M));
  if (a.mode == 1)
    hipLaunchKernelGGL((accept_rowstat16_kernel<F16, true>), grid, dim3(kRowThreads), 0, s, a);
  else
    hipLaunchKernelGGL((accept_rowstat16_kernel<F16, false>), grid, dim3(kRowThreads), 0, s, a);
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

}  // namespace

size_t accept_walk_lds_bytes(int M) {
  // par, nxt, ok, mz, lz, hz, path: 7*M words, plus reduction scratch.
  return ((size_t)7 * M + 1) / 2 * 8 + 8 + 16 * 8 + 16 * 4 + 64;
}

hipError_t launch_accept(const AcceptArgs& a, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  if (a.T <= 0 || a.M <= 0) return hipSuccess;
  hipError_t e;
  if (ev0 != nullptr && (e = hipEventRecord(ev0, s)) != hipSuccess) return e;
  // 16-bit logits with 16-byte aligned rows and chunks take the packed-key
  // kernel (its chunk must fit 256 threads x 8 vectors of 8 elements).
  const bool al16 = ((uintptr_t)a.logits & 15) == 0 && (a.l_st * 2) % 16 == 0 && (a.l_sm * 2) % 16 == 0 &&
                    (a.chunk * 2) % 16 == 0 && a.chunk <= (int64_t)kRowThreads * kVecPerThread * 8;
  if (a.l_dtype == 0)
    e = al16 ? launch_rowstat16<false>(a, s) : launch_rowstat<uint16_t>(a, s);
  else if (a.l_dtype == 1)
    e = al16 ? launch_rowstat16<true>(a, s) : launch_rowstat<_Float16>(a, s);
  else
    e = launch_rowstat<float>(a, s);
  if (e != hipSuccess) return e;
  if (ev1 != nullptr && (e = hipEventRecord(ev1, s)) != hipSuccess) return e;
  const int threads = ((a.M + 63) / 64) * 64;
  hipLaunchKernelGGL(accept_walk_kernel, dim3((unsigned)a.T), dim3(threads), accept_walk_lds_bytes(a.M), s, a);
  return hipGetLastError();
}

}  // namespace dsv
