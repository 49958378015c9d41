// dsv_sample.hip — kernel 4 in sampling mode on gfx950: the reference's
// multinomial branch of verify_new (draft/tree_verification.py:103-106) with
// the warpers of prepare_logits_processor (:15-32), then the greedy walk over
// the drawn tokens.
//
// Per node row x (vocabulary V), with the logits dtype's rounding:
//   y = x / T (T == 1: y = x); NaN counts as -inf, -0 as +0.
//   Order: descending by (y, index) — among equal values the higher index
//   ranks first, as the warpers' stable ascending sort cut from the low end.
//   Masses q_v = rint(2^(S + (y_v - max y) log2 e)), S = 63 - bitlen(V):
//   exact 64-bit integers, so every top-p decision is an integer comparison.
//   top-p: keep v iff the mass ranked above v < Tq = ceil(P * L / 2^32),
//   L = sum q, P = rint(top_p * 2^32).  top-k: keep y >= the k-th largest y.
//   Draw: argmax over kept v of y_v + G_v (double, lowest index on ties),
//   G_v = -ln(-ln U_v), U_v from Philox4x64-10 (Salmon et al. 2011) with key
//   (seed, 0) and counter (v, node, tree, 0): a Gumbel-max draw from
//   softmax(y) over the kept set.
// The logarithms and 2^x are evaluated with a fixed sequence of double
// operations (no fused multiply-add, no library call), each correctly
// rounded, so the draws are reproducible bit for bit off the GPU.
//
// Kernels:
//   sample_select_kernel  one workgroup per row, only with top-p or top-k:
//       8-bit radix selection over the order keys of y (count-weighted for
//       top-k, mass-weighted for top-p), then over the indices of the tie
//       group at the top-p cut; writes the kept-set bounds of the row.
//   sample_sweep_kernel   one workgroup per (row, vocabulary range): the
//       Gumbel-max draw over the range's kept entries.
//   the walk of dsv_accept.hip combines the ranges' draws and walks.

#include "dsv_internal.h"

namespace dsv {

namespace {

constexpr int kSelThreads = 1024;
constexpr int kSweepThreads = 256;
constexpr float kNegInfF = -__builtin_huge_valf();

// ln(2)^k / k!, k = 0..17, and 1 / (2k + 1), k = 0..11 (correctly rounded).
__constant__ double kExp2C[18] = {
    0x1.0000000000000p+0,  0x1.62e42fefa39efp-1,  0x1.ebfbdff82c58fp-3,  0x1.c6b08d704a0c0p-5,
    0x1.3b2ab6fba4e77p-7,  0x1.5d87fe78a6731p-10, 0x1.430912f86c787p-13, 0x1.ffcbfc588b0c7p-17,
    0x1.62c0223a5c824p-20, 0x1.b5253d395e7c4p-24, 0x1.e4cf5158b8ecap-28, 0x1.e8cac7351bb25p-32,
    0x1.c3bd650fc2986p-36, 0x1.816193166d0f9p-40, 0x1.314964d5878a9p-44, 0x1.c36e843b04022p-49,
    0x1.38e89ae79f8b4p-53, 0x1.98444b41c25a8p-58};
__constant__ double kAtanhC[12] = {
    0x1.0000000000000p+0, 0x1.5555555555555p-2, 0x1.999999999999ap-3, 0x1.2492492492492p-3,
    0x1.c71c71c71c71cp-4, 0x1.745d1745d1746p-4, 0x1.3b13b13b13b14p-4, 0x1.1111111111111p-4,
    0x1.e1e1e1e1e1e1ep-5, 0x1.af286bca1af28p-5, 0x1.8618618618618p-5, 0x1.642c8590b2164p-5};
constexpr double kLn2D = 0x1.62e42fefa39efp-1;
constexpr double kLog2eD = 0x1.71547652b82fep+0;
constexpr double kSqrtHalfD = 0x1.6a09e667f3bcdp-1;

// ln x for finite x > 0: x = m 2^e, m in [sqrt(1/2), sqrt(2)),
// ln m = 2 atanh(s), s = (m - 1) / (m + 1), Horner in s^2.
__device__ __forceinline__ double det_ln(double x) {
#pragma clang fp contract(off)
  int e;
  double m = __builtin_frexp(x, &e);
  if (m < kSqrtHalfD) {
    m = m * 2.0;
    e -= 1;
  }
  const double s = (m - 1.0) / (m + 1.0);
  const double s2 = s * s;
  double p = kAtanhC[11];
#pragma unroll
  for (int k = 10; k >= 0; --k) {
    p = p * s2;
    p = p + kAtanhC[k];
  }
  const double t = s * p;
  return (double)e * kLn2D + (t + t);
}

// 2^u for u <= 0; 0 below -200 and for -inf / NaN.
__device__ __forceinline__ double det_exp2(double u) {
#pragma clang fp contract(off)
  if (!(u >= -200.0)) return 0.0;
  const double n = __builtin_floor(u);
  const double f = u - n;
  double p = kExp2C[17];
#pragma unroll
  for (int k = 16; k >= 0; --k) {
    p = p * f;
    p = p + kExp2C[k];
  }
  return __builtin_ldexp(p, (int)n);
}

// Philox4x64-10, word 0 of the output block.
__device__ __forceinline__ uint64_t philox_word0(uint64_t c0, uint64_t c1, uint64_t c2, uint64_t c3, uint64_t k0,
                                                 uint64_t k1) {
  constexpr uint64_t M0 = 0xD2E7470EE14C6C93ull, M1 = 0xCA5A826395121157ull;
  constexpr uint64_t W0 = 0x9E3779B97F4A7C15ull, W1 = 0xBB67AE8584CAA73Bull;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += W0;
      k1 += W1;
    }
    const uint64_t hi0 = __umul64hi(M0, c0), lo0 = M0 * c0;
    const uint64_t hi1 = __umul64hi(M1, c2), lo1 = M1 * c2;
    const uint64_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
  return c0;
}

// G = -ln(-ln U), U = ((w >> 12) + 0.5) * 2^-52.
__device__ __forceinline__ double gumbel(uint64_t w) {
#pragma clang fp contract(off)
  const double u = ((double)(w >> 12) + 0.5) * 0x1p-52;
  return -det_ln(-det_ln(u));
}

template <typename LT>
__device__ __forceinline__ float raw_to_f(LT x);
template <>
__device__ __forceinline__ float raw_to_f<uint16_t>(uint16_t x) {  // bf16 bits
  return __uint_as_float((uint32_t)x << 16);
}
template <>
__device__ __forceinline__ float raw_to_f<_Float16>(_Float16 x) {
  return (float)x;
}
template <>
__device__ __forceinline__ float raw_to_f<float>(float x) {
  return x;
}

// y of one logit: x / T rounded to the logits dtype (T == 1: x); NaN -> -inf, -0 -> +0.
template <typename LT>
__device__ __forceinline__ float warp_y(LT raw, float T) {
  float y = raw_to_f<LT>(raw);
  if (T != 1.f) {
    y = y / T;  // IEEE division (correctly rounded by default in HIP)
    if constexpr (sizeof(LT) == 2) {
      if constexpr (__is_same(LT, _Float16))
        y = (float)(_Float16)y;
      else
        y = (float)(__bf16)y;
    }
  }
  if (y != y) y = kNegInfF;
  if (y == 0.f) y = 0.f;
  return y;
}

// Order-preserving 32-bit key of y.
__device__ __forceinline__ uint32_t ykey(float y) {
  const uint32_t b = __float_as_uint(y);
  return b ^ ((b >> 31) ? 0xFFFFFFFFu : 0x80000000u);
}

// Fixed-point mass of y given the row maximum m: rint(2^(S + (y - m) log2 e)).
__device__ __forceinline__ uint64_t fixed_mass(float y, float m, int S) {
#pragma clang fp contract(off)
  if (!(m > kNegInfF)) return 0;  // no finite logit: no mass
  if (y == m) return 1ull << S;
  const double d = (double)y - (double)m;
  const double p = det_exp2(d * kLog2eD);
  return (uint64_t)__builtin_rint(__builtin_ldexp(p, S));
}

// Key digits to resolve per logits dtype: bf16 keys vary in bits 31..16,
// f16 (widened) in bits 31..13, f32 in all 32.
template <typename LT>
constexpr int key_digits() {
  return sizeof(LT) == 4 ? 4 : (__is_same(LT, _Float16) ? 3 : 2);
}

// The key bits below the resolved digits are the same for every value of a
// 16-bit dtype of one sign: 0 for keys of positive values, 1 for negative
// ones (their key is the complement of the widened bits).  A resolved prefix
// completed with them is the exact key of its values.
__device__ __forceinline__ uint32_t fill_low(uint32_t prefix, int nd) {
  if (nd >= 4 || (prefix >> 31)) return prefix;
  return prefix | ((1u << (32 - 8 * nd)) - 1u);
}

// Descending scan of a 256-bin histogram by wave 0: the first bin b (from 255
// down) where before(b) + w(b) >= target, before(b) = sum of bins above b.
// Returns b (or -1 when the total stays below the target) and before(b).
__device__ __forceinline__ int scan_desc(const uint64_t* w, uint64_t target, uint64_t& before_out) {
  const int lane = threadIdx.x & 63;
  uint64_t v[4], tot = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[j] = w[255 - (4 * lane + j)];
    tot += v[j];
  }
  // Exclusive prefix over lanes of the lane totals.
  uint64_t incl = tot;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t x = __shfl_up(incl, o);
    if (lane >= o) incl += x;
  }
  uint64_t run = incl - tot;
  int found = -1;
  uint64_t before = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (found < 0 && run + v[j] >= target) {
      found = 255 - (4 * lane + j);
      before = run;
    }
    run += v[j];
  }
  const uint64_t mask = __ballot(found >= 0);
  if (mask == 0) return -1;
  const int first = __builtin_ctzll(mask);
  before_out = __shfl(before, first);
  return __shfl(found, first);
}

template <typename LT>
__global__ void __launch_bounds__(kSelThreads) sample_select_kernel(const AcceptArgs a) {
  const int64_t row = blockIdx.x;
  const int t = (int)(row / a.M), i = (int)(row % a.M);
  const LT* x = reinterpret_cast<const LT*>(a.logits) + (int64_t)t * a.l_st + (int64_t)i * a.l_sm;
  const int V = (int)a.V;
  const int tid = threadIdx.x;
  constexpr int ND = key_digits<LT>();

  __shared__ uint64_t hist[256];
  __shared__ float red_f[kSelThreads / 64];
  __shared__ uint32_t res_u[4];
  __shared__ uint64_t res_q[4];

  // Row maximum of y.
  float m = kNegInfF;
  for (int v = tid; v < V; v += kSelThreads) m = fmaxf(m, warp_y<LT>(x[v], a.temperature));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if ((tid & 63) == 0) red_f[tid >> 6] = m;
  __syncthreads();
  if (tid == 0) {
    float mm = red_f[0];
    for (int w = 1; w < kSelThreads / 64; ++w) mm = fmaxf(mm, red_f[w]);
    red_f[0] = mm;
  }
  __syncthreads();
  m = red_f[0];

  int S = 63;
  for (int vv = V; vv > 0; vv >>= 1) --S;  // 63 - bitlen(V)

  // One radix pass: histogram of digit `shift` over the elements whose key
  // matches `prefix` above that digit (and, for the tie pass, key == tie_key
  // with the index as the digit source), weighted by count or mass.
  auto pass = [&](int shift, uint32_t prefix, bool mass, bool by_index, uint32_t tie_key) {
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    const uint32_t hi_mask = shift >= 24 ? 0u : ~((1u << (shift + 8)) - 1u);
    for (int v = tid; v < V; v += kSelThreads) {
      const float y = warp_y<LT>(x[v], a.temperature);
      const uint32_t k = ykey(y);
      uint32_t src = k;
      if (by_index) {
        if (k != tie_key) continue;
        src = (uint32_t)v;
      }
      if ((src & hi_mask) != (prefix & hi_mask)) continue;
      const int bin = (int)((src >> shift) & 255u);
      atomicAdd(reinterpret_cast<unsigned long long*>(&hist[bin]),
                (unsigned long long)(mass ? fixed_mass(y, m, S) : 1ull));
    }
    __syncthreads();
  };

  // top-k: the k-th largest key (1-based rank, with multiplicity).
  uint32_t tk = 0;
  if (a.top_k > 0 && a.top_k < V) {
    uint32_t prefix = 0;
    uint64_t rank = (uint64_t)a.top_k;
    for (int d = 0; d < ND; ++d) {
      const int shift = 24 - 8 * d;
      pass(shift, prefix, false, false, 0);
      if (tid < 64) {
        uint64_t before = 0;
        const int b = scan_desc(hist, rank, before);
        if (tid == 0) {
          res_u[0] = (uint32_t)max(b, 0);
          res_q[0] = before;
        }
      }
      __syncthreads();
      prefix |= res_u[0] << shift;
      rank -= res_q[0];
      __syncthreads();
    }
    tk = fill_low(prefix, ND);
  }

  // top-p: the key of the last kept element, then the index bound in its tie group.
  uint32_t ystar = 0, istar = 0;
  if (a.top_p_q != 0) {
    uint32_t prefix = 0;
    uint64_t above = 0, Tq = 0, group = 0;
    for (int d = 0; d < ND; ++d) {
      const int shift = 24 - 8 * d;
      pass(shift, prefix, true, false, 0);
      if (d == 0 && tid < 64) {
        // Total mass L and the threshold Tq = ceil(P * L / 2^32).
        uint64_t s = hist[4 * tid] + hist[4 * tid + 1] + hist[4 * tid + 2] + hist[4 * tid + 3];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
        if (tid == 0) {
          const uint64_t P = a.top_p_q;
          const uint64_t lo = P * s, hi = __umul64hi(P, s);
          const uint64_t lo2 = lo + 0xFFFFFFFFull;
          const uint64_t hi2 = hi + (lo2 < lo ? 1ull : 0ull);
          res_q[1] = (lo2 >> 32) | (hi2 << 32);
        }
      }
      __syncthreads();
      Tq = res_q[1];
      if (tid < 64) {
        uint64_t before = 0;
        const int b = scan_desc(hist, Tq > above ? Tq - above : 0, before);
        if (tid == 0) {
          // Without a crossing (L == 0: no finite logit) nothing is kept.
          res_u[0] = (uint32_t)(b < 0 ? 255 : b);
          res_u[1] = b < 0 ? 1u : 0u;
          res_q[0] = before;
          res_q[2] = b < 0 ? 0 : hist[b];  // mass of the chosen bin
        }
      }
      __syncthreads();
      prefix |= res_u[0] << shift;
      above += res_q[0];
      const bool none = res_u[1] != 0;
      __syncthreads();
      if (none) {
        prefix = 0xFFFFFFFFu;
        break;
      }
    }
    ystar = prefix == 0xFFFFFFFFu ? prefix : fill_low(prefix, ND);
    if (ystar != 0xFFFFFFFFu) {
      // Tie group of the cut key: its size c and per-element mass q*.
      float ys;
      {
        const uint32_t b = ystar ^ ((ystar >> 31) ? 0x80000000u : 0xFFFFFFFFu);
        ys = __uint_as_float(b);
      }
      const uint64_t qs = fixed_mass(ys, m, S);
      // Group size: count pass on the exact key (every index in bin 0).
      pass(24, 0, false, true, ystar);
      if (tid < 64) {
        uint64_t c = hist[4 * tid] + hist[4 * tid + 1] + hist[4 * tid + 2] + hist[4 * tid + 3];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o);
        if (tid == 0) res_q[3] = c;
      }
      __syncthreads();
      group = res_q[3];
      __syncthreads();
      // Index-bit passes cover bitlen(V - 1) bits: the kept members are the
      // n_keep highest indices, n_keep = #{j < c : above + j q* < Tq}.
      uint64_t n_keep = group;
      if (qs > 0) {
        const uint64_t need = (Tq - above + qs - 1) / qs;
        n_keep = need < group ? need : group;
      }
      if (n_keep < group) {
        int ib = 0;
        for (int vv = V - 1; vv > 0; vv >>= 1) ++ib;
        const int nd_i = (ib + 7) / 8;
        uint32_t ipre = 0;
        uint64_t rank = n_keep;
        for (int d = nd_i - 1; d >= 0; --d) {
          const int shift = 8 * d;
          pass(shift, ipre, false, true, ystar);
          if (tid < 64) {
            uint64_t before = 0;
            const int b = scan_desc(hist, rank, before);
            if (tid == 0) {
              res_u[0] = (uint32_t)max(b, 0);
              res_q[0] = before;
            }
          }
          __syncthreads();
          ipre |= res_u[0] << shift;
          rank -= res_q[0];
          __syncthreads();
        }
        istar = ipre;
      }
    }
  }
  if (tid == 0) a.sel[row] = make_uint4(tk, ystar, istar, 0u);
}

// Gumbel-max draw over one vocabulary range of one row.
template <typename LT>
__global__ void __launch_bounds__(kSweepThreads) sample_sweep_kernel(const AcceptArgs a) {
  const int c = blockIdx.x;
  const int64_t row = blockIdx.y;
  const int t = (int)(row / a.M), i = (int)(row % a.M);
  const LT* x = reinterpret_cast<const LT*>(a.logits) + (int64_t)t * a.l_st + (int64_t)i * a.l_sm;
  const int64_t lo = (int64_t)c * a.chunk, hi = min(lo + a.chunk, a.V);
  uint32_t tk = 0, ystar = 0, istar = 0;
  if (a.sel != nullptr) {
    const uint4 s = a.sel[row];
    tk = s.x;
    ystar = s.y;
    istar = s.z;
  }
  double best = -__builtin_huge_val();
  int bi = -1;
  for (int64_t v = lo + threadIdx.x; v < hi; v += kSweepThreads) {
    const float y = warp_y<LT>(x[v], a.temperature);
    if (!(y > kNegInfF)) continue;
    const uint32_t k = ykey(y);
    if (k < tk || k < ystar || (k == ystar && (uint32_t)v < istar)) continue;
    const double g = gumbel(philox_word0((uint64_t)v, (uint64_t)i, (uint64_t)t, 0ull, a.seed, 0ull));
    const double z = (double)y + g;
    if (bi < 0 || z > best) {
      best = z;
      bi = (int)v;
    }
  }
  // Reduction: larger z, then lower index; -1 = nothing kept.
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const double ob = __shfl_xor(best, o);
    const int oi = __shfl_xor(bi, o);
    if (oi >= 0 && (bi < 0 || ob > best || (ob == best && oi < bi))) {
      best = ob;
      bi = oi;
    }
  }
  __shared__ double sb[kSweepThreads / 64];
  __shared__ int si[kSweepThreads / 64];
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sb[w] = best;
    si[w] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < kSweepThreads / 64; ++k)
      if (si[k] >= 0 && (bi < 0 || sb[k] > best || (sb[k] == best && si[k] < bi))) {
        best = sb[k];
        bi = si[k];
      }
    const uint64_t zb = __builtin_bit_cast(uint64_t, best);
    a.rstat[row * a.nchunk + c] =
        make_float4(__uint_as_float((uint32_t)zb), __uint_as_float((uint32_t)(zb >> 32)), __int_as_float(bi), 0.f);
  }
}

template <typename LT>
hipError_t launch_sample_t(const AcceptArgs& a, hipStream_t s) {
  const unsigned rows = (unsigned)((int64_t)a.T * a.M);
  if (a.sel != nullptr) hipLaunchKernelGGL(sample_select_kernel<LT>, dim3(rows), dim3(kSelThreads), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(sample_sweep_kernel<LT>, dim3((unsigned)a.nchunk, rows), dim3(kSweepThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_sample(const AcceptArgs& a, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  if (a.T <= 0 || a.M <= 0) return hipSuccess;
  hipError_t e;
  if (ev0 != nullptr && (e = hipEventRecord(ev0, s)) != hipSuccess) return e;
  if (a.l_dtype == 0)
    e = launch_sample_t<uint16_t>(a, s);
  else if (a.l_dtype == 1)
    e = launch_sample_t<_Float16>(a, s);
  else
    e = launch_sample_t<float>(a, s);
  if (e != hipSuccess) return e;
  if (ev1 != nullptr && (e = hipEventRecord(ev1, s)) != hipSuccess) return e;
  return launch_walk(a, s);
}

}  // namespace dsv
