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
//   G_v = -ln(-ln U_v), U_v = (w + 0.5) 2^-32 with w the output word v & 3 of
//   Philox4x32-10 (Salmon et al. 2011) at key (seed mod 2^32, seed >> 32) and
//   counter (v >> 2, node, tree, 0): a Gumbel-max draw from softmax(y) over
//   the kept set, one generator call per four vocabulary entries.
// The logarithms and 2^x are evaluated with a fixed sequence of double
// operations (no fused multiply-add, no library call), each correctly
// rounded, so the draws are reproducible bit for bit off the GPU.
//
// Kernels:
//   sample_select_kernel  one workgroup per row, only with top-p or top-k.
//       Pass 1: the row maximum m (packed integer extremes of the logits'
//       bits).  Pass 2: exact y, the fp32 sum of 2^a (a = (y - m) log2 e) over
//       the row, and per wave a region of the entries with a >= -g (g lowered
//       and the region compacted when it would overflow).  The narrowest head
//       {a > -theta} within the regions that carries the top-p mass (or holds
//       k) is taken from them and sorted; rows whose regions do not hold it
//       count a histogram of a and gather a head in further passes.  top-k is
//       the head's k-th key; top-p takes the head's exact masses and bounds L
//       from the fp32 sum: the cut is exact when it lands on the same entry
//       for every L in those bounds, inside the head.  The draw over the kept
//       head entries is the row's result.  Other rows (flat rows, a large k,
//       an undecided cut, NaN or +inf logits) are left to the radix kernel
//       (status 2, with m).
//   sample_radix_kernel   one workgroup per row left open: 8-bit radix
//       selection over the order keys of y (count-weighted for top-k,
//       mass-weighted for top-p); the kept set (keys at or above both bounds)
//       is gathered into LDS, where the index bound in the cut's tie group and
//       the draw are taken when it fits; otherwise the bound comes from index
//       passes over the row and the sweep draws.
//   sample_sweep_kernel   one workgroup per (row, vocabulary range) of the
//       rows still open (f32 rows without top-p / top-k when rows are fewer
//       than CUs):
//       the Gumbel-max draw over the range's kept entries.  Against a
//       wave-shared lower bound lb of the range's maximum z, an entry whose
//       1 - U exceeds an upper bound of e^(y - lb) cannot reach lb (one 2^x
//       per entry from x * fl(1/T)); the few others take the exact warper,
//       the keep test and an fp32 estimate of z (within 2^-14 of it), which
//       leaves the exact double evaluation to the entries that can still win.
//   sample_temp_kernel    temperature alone (f32 logits: with at least as
//       many rows as CUs): one workgroup per row, or up to 8 when rows are
//       few; the maximum entry's exact z bounds the row's maximum z from the
//       start, groups are screened on their raw bits against the smallest
//       logit that can still reach the bound, and the groups kept are queued
//       per wave and drawn 64 at a time (the sweep's screen and draw).
//   the walk of dsv_accept.hip combines the ranges' draws and walks.

#include "dsv_internal.h"

namespace dsv {

namespace {

constexpr int kRadixThreads = 1024;
constexpr int kSweepThreads = 256;
constexpr float kNegInfF = -__builtin_huge_valf();
constexpr int kCap = 4096;   // candidates the select kernel's fast path sorts in LDS
// Head thresholds of the select kernel, in log2 units of a = (y - m) log2 e
// (the head {a > -theta_j}): the floats whose bits are (250 + j) << 22, i.e.
// 2^e and 1.5 * 2^e from 1/4 to 48.
constexpr int kNTheta = 16;
__constant__ float kTheta[kNTheta] = {0.25f, 0.375f, 0.5f, 0.75f, 1.f, 1.5f, 2.f, 3.f,
                                      4.f,   6.f,    8.f,  12.f,  16.f, 24.f, 32.f, 48.f};
// Upper bound of the fp32 Gumbel estimate: U <= 1 - 2^-33 gives G < 22.9.
constexpr float kGumbelMax = 23.f;
// Margin of the fp32 estimate of z = y + G: the estimate is within 2^-14 of
// the double value (hardware log2 to about 1 ulp, fp32 rounding of U, 1 - U,
// -ln U and the sum); the margin is 2^-7 plus 2^-20 of |z|.
constexpr float kZMargin = 0x1p-7f;
constexpr float kZMarginRel = 0x1p-20f;

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

// Philox4x32-10: the four output words of counter (c0, c1, c2, c3), key (k0, k1).
__device__ __forceinline__ uint4 philox4x32(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                                            uint32_t k1) {
  constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += W0;
      k1 += W1;
    }
    // One 32 x 32 -> 64-bit product each (v_mad_u64_u32).
    const uint64_t p0 = (uint64_t)M0 * c0, p1 = (uint64_t)M1 * c2;
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
    c0 = n0;
    c1 = (uint32_t)p1;
    c2 = n2;
    c3 = (uint32_t)p0;
  }
  return make_uint4(c0, c1, c2, c3);
}

__device__ __forceinline__ uint32_t word_of(const uint4& w, int e) {
  return e == 0 ? w.x : (e == 1 ? w.y : (e == 2 ? w.z : w.w));
}

// The draw's random word of vocabulary entry v of row (tree t, node i).
__device__ __forceinline__ uint32_t draw_word(int64_t v, int i, int t, uint64_t seed) {
  const uint4 w = philox4x32((uint32_t)(v >> 2), (uint32_t)i, (uint32_t)t, 0u, (uint32_t)seed, (uint32_t)(seed >> 32));
  return word_of(w, (int)(v & 3));
}

// G = -ln(-ln U), U = (w + 0.5) * 2^-32, in double (the definition).  Not
// inlined: the filters leave it to few entries, and one copy keeps the
// kernels small.
__device__ __noinline__ double gumbel(uint32_t w) {
#pragma clang fp contract(off)
  const double u = ((double)w + 0.5) * 0x1p-32;
  return -det_ln(-det_ln(u));
}

// fp32 estimate of gumbel(w).  -ln U from U for U < 1/2, else from
// x = 1 - U = (~w + 0.5) 2^-32 (a series below 2^-7), so that -ln U keeps its
// relative accuracy as U approaches 1.
__device__ __forceinline__ float gumbel_est(uint32_t w) {
  float e;
  if (w < 0x80000000u) {
    e = -__logf(((float)w + 0.5f) * 0x1p-32f);
  } else {
    const float x = ((float)(~w) + 0.5f) * 0x1p-32f;
    e = x < 0x1p-7f ? x * (1.f + x * (0.5f + x * (1.f / 3.f))) : -__logf(1.f - x);
  }
  return -__logf(e);
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

// The temperature warper's constants.
struct Warp {
  float T, rT;  // T and fl(1 / T)
};
__device__ __forceinline__ Warp make_warp(float T) { return Warp{T, 1.f / T}; }

// NaN counts as -inf, -0 as +0.
__device__ __forceinline__ float clean_y(float y) {
  if (y != y) y = kNegInfF;
  if (y == 0.f) y = 0.f;
  return y;
}

template <typename LT>
__device__ __forceinline__ float round_lt(float y) {
  if constexpr (__is_same(LT, _Float16))
    return (float)(_Float16)y;
  else if constexpr (__is_same(LT, uint16_t))
    return (float)(__bf16)y;
  else
    return y;
}

// y of one logit: x / T (IEEE division, correctly rounded by default in HIP)
// rounded to the logits dtype (T == 1: x); NaN -> -inf, -0 -> +0.
template <typename LT>
__device__ __forceinline__ float warp_yf(float y, const Warp& w) {
  if (w.T != 1.f) y = round_lt<LT>(y / w.T);
  return clean_y(y);
}
template <typename LT>
__device__ __forceinline__ float warp_y(LT raw, const Warp& w) {
  return warp_yf<LT>(raw_to_f<LT>(raw), w);
}

// warp_y of N values held as floats.  For 16-bit logits q = x * fl(1/T) lies
// within 3 fp32 ulp of the correctly rounded quotient; both round to the same
// 16-bit value unless q is within 8 ulp of a rounding midpoint or outside the
// dtype's normal range, and only there (for the wave: only when some lane has
// such an entry) the division decides.
template <typename LT, int N>
__device__ __forceinline__ void warp_vec(float (&y)[N], const Warp& w) {
  if (w.T != 1.f) {
    if constexpr (sizeof(LT) == 2) {
      constexpr bool kF16 = __is_same(LT, _Float16);
      constexpr int LOW = kF16 ? 13 : 16;  // fp32 mantissa bits below the 16-bit type's
      constexpr uint32_t MID = 1u << (LOW - 1);
      constexpr float kLo = kF16 ? 0x1p-14f : 0x1p-100f, kHi = kF16 ? 32768.f : 0x1p100f;
      float q[N];
      bool unsafe[N], any = false;
#pragma unroll
      for (int e = 0; e < N; ++e) {
        q[e] = y[e] * w.rT;
        const uint32_t low = __float_as_uint(q[e]) & ((1u << LOW) - 1u);
        const float aq = fabsf(q[e]);
        unsafe[e] = !((low > MID + 8u || low + 8u < MID) && aq >= kLo && aq <= kHi);
        any |= unsafe[e];
      }
      if (__ballot(any) != 0ull) {
#pragma unroll
        for (int e = 0; e < N; ++e)
          if (unsafe[e]) q[e] = y[e] / w.T;
      }
#pragma unroll
      for (int e = 0; e < N; ++e) y[e] = round_lt<LT>(q[e]);
    } else {
#pragma unroll
      for (int e = 0; e < N; ++e) y[e] = y[e] / w.T;
    }
  }
#pragma unroll
  for (int e = 0; e < N; ++e) y[e] = clean_y(y[e]);
}

// The logit of dtype LT whose value is f (f is such a value).
template <typename LT>
__device__ __forceinline__ LT f_to_raw(float f) {
  if constexpr (__is_same(LT, uint16_t))
    return (uint16_t)(__float_as_uint(f) >> 16);
  else
    return (LT)f;
}

// Order-preserving 32-bit key of y.
__device__ __forceinline__ uint32_t ykey(float y) {
  const uint32_t b = __float_as_uint(y);
  return b ^ ((b >> 31) ? 0xFFFFFFFFu : 0x80000000u);
}

// The 16-byte vector of logits at v0 when it is whole and the row is 16-byte
// aligned (otherwise zero: unpack_vec then reads the entries one by one).
template <typename LT>
__device__ __forceinline__ u32x4 fetch_vec(const LT* x, int64_t v0, int64_t hi, bool aligned) {
  constexpr int N = 16 / sizeof(LT);
  return (aligned && v0 + N <= hi) ? *reinterpret_cast<const u32x4*>(x + v0) : u32x4{0, 0, 0, 0};
}

// N = 16 / sizeof(LT) consecutive logits from v0 as floats (entries at or
// past hi read as -inf), from fetch_vec's vector r.
template <typename LT>
__device__ __forceinline__ void unpack_vec(const LT* x, int64_t v0, int64_t hi, bool aligned, const u32x4& r,
                                           float (&y)[16 / sizeof(LT)]) {
  constexpr int N = 16 / sizeof(LT);
  if (aligned && v0 + N <= hi) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (sizeof(LT) == 4) {
        y[e] = __uint_as_float(r[e]);
      } else {
        y[2 * e] = raw_to_f<LT>(__builtin_bit_cast(LT, (uint16_t)(r[e] & 0xFFFFu)));
        y[2 * e + 1] = raw_to_f<LT>(__builtin_bit_cast(LT, (uint16_t)(r[e] >> 16)));
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < N; ++e) y[e] = v0 + e < hi ? raw_to_f<LT>(x[v0 + e]) : kNegInfF;
  }
}

// y of loaded logits: the warper (WARP) or NaN -> -inf and -0 -> +0 only.
template <typename LT, bool WARP, int N>
__device__ __forceinline__ void finish_y(float (&y)[N], const Warp& T) {
  if constexpr (WARP) {
    warp_vec<LT, N>(y, T);
  } else {
#pragma unroll
    for (int e = 0; e < N; ++e) y[e] = clean_y(y[e]);
  }
}

// Runs f(v0, y) over [lo, hi) in vectors of N entries (lo a multiple of N):
// the threads of a block take consecutive vectors, two vectors per thread and
// iteration, and the next iteration's two loads are issued before f runs on
// this one's, so that a thread keeps up to four vector loads in flight.
// Every lane of a wave runs the same iterations, so f may use wave ballots
// and shuffles.  WARP = false hands f the logits themselves (NaN as -inf),
// RAW = true the logits as loaded.  A wave's iterations whose vectors are all
// whole (aligned rows) take unconditional loads; the rest read entry by entry
// where needed.
template <typename LT, int NT, bool WARP = true, bool RAW = false, typename F>
__device__ __forceinline__ void row_sweep(const LT* x, int64_t lo, int64_t hi, const Warp& T, F&& f) {
  constexpr int N = 16 / sizeof(LT);
  constexpr int64_t kStep = (int64_t)2 * NT * N;
  constexpr int64_t kSpan = (int64_t)(NT + 64) * N;  // a wave's two vectors lie in [b0, b0 + kSpan)
  const bool aligned = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  const int lane = threadIdx.x & 63;
  int64_t b0 = lo + (int64_t)(threadIdx.x & ~63) * N;  // uniform over the wave
  auto run = [&](int64_t v0, const u32x4& r) {
    float y[N];
    unpack_vec<LT>(x, v0, v0 + N, true, r, y);
    if constexpr (!RAW) finish_y<LT, WARP>(y, T);
    f(v0, y);
  };
  if (aligned && b0 + kSpan <= hi) {
    const LT* p = x + b0 + (int64_t)lane * N;
    u32x4 ra = *reinterpret_cast<const u32x4*>(p), rb = *reinterpret_cast<const u32x4*>(p + NT * N);
    for (;;) {
      const bool more = b0 + kStep + kSpan <= hi;  // uniform over the wave
      u32x4 na, nb;
      if (more) {
        na = *reinterpret_cast<const u32x4*>(p + kStep);
        nb = *reinterpret_cast<const u32x4*>(p + kStep + NT * N);
      }
      run(b0 + (int64_t)lane * N, ra);
      run(b0 + (int64_t)lane * N + (int64_t)NT * N, rb);
      b0 += kStep;
      p += kStep;
      if (!more) break;
      ra = na;
      rb = nb;
    }
  }
  for (; b0 < hi; b0 += kStep) {
    const int64_t v0 = b0 + (int64_t)lane * N, v1 = v0 + (int64_t)NT * N;
    float ya[N], yb[N];
    unpack_vec<LT>(x, v0, hi, aligned, fetch_vec<LT>(x, v0, hi, aligned), ya);
    unpack_vec<LT>(x, v1, hi, aligned, fetch_vec<LT>(x, v1, hi, aligned), yb);
    if constexpr (!RAW) {
      finish_y<LT, WARP>(ya, T);
      finish_y<LT, WARP>(yb, T);
    }
    f(v0, ya);
    f(v1, yb);
  }
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

// The y of an order key (inverse of ykey).
__device__ __forceinline__ float key_to_y(uint32_t k) {
  return __uint_as_float(k ^ ((k >> 31) ? 0x80000000u : 0xFFFFFFFFu));
}

// Tq = ceil(P * L / 2^32) with a 128-bit product.
__device__ __forceinline__ uint64_t tq_of(uint64_t P, uint64_t L) {
  const uint64_t lo = P * L, hi = __umul64hi(P, L);
  const uint64_t lo2 = lo + 0xFFFFFFFFull;
  const uint64_t hi2 = hi + (lo2 < lo ? 1ull : 0ull);
  return (lo2 >> 32) | (hi2 << 32);
}

// Block argmax of (z, index): larger z, then lower index; -1 = none.  Every
// thread calls it; thread 0 gets the result.
__device__ __forceinline__ void block_argmax(double& best, int& bi, double* sb, int* si, int nthreads) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const double ob = __shfl_xor(best, o);
    const int oi = __shfl_xor(bi, o);
    if (oi >= 0 && (bi < 0 || ob > best || (ob == best && oi < bi))) {
      best = ob;
      bi = oi;
    }
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sb[w] = best;
    si[w] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < nthreads / 64; ++k)
      if (si[k] >= 0 && (bi < 0 || sb[k] > best || (sb[k] == best && si[k] < bi))) {
        best = sb[k];
        bi = si[k];
      }
  }
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

// ---- select kernel helpers ----------------------------------------------------

// Bits of the logits dtype read as signed integers: non-negative values order
// as their integers and negative ones in reverse, so the integer maximum is the
// largest non-negative value and the integer minimum the negative value
// closest to zero.  kInf / kNegInf: the integers of +inf and -inf.
template <typename LT>
struct IntOrder;
template <>
struct IntOrder<uint16_t> {
  static constexpr int kInf = 0x7F80, kNegInf = -0x80;
};
template <>
struct IntOrder<_Float16> {
  static constexpr int kInf = 0x7C00, kNegInf = -0x400;
};
template <>
struct IntOrder<float> {
  static constexpr int kInf = 0x7F800000, kNegInf = -0x800000;
};

typedef short s16x2 __attribute__((ext_vector_type(2)));

// The logit whose bits read as the signed integer b.
template <typename LT>
__device__ __forceinline__ float int_to_f(int b) {
  if constexpr (sizeof(LT) == 4)
    return __int_as_float(b);
  else
    return raw_to_f<LT>(__builtin_bit_cast(LT, (uint16_t)b));
}

// This thread's maximum of the row's logits (NaN counts as -inf) over the
// vectors row_sweep would hand it: two integer extremes per packed word, then
// the float they stand for.  A thread that met a positive NaN (it would pass
// for the maximum) redoes its vectors entry by entry.
template <typename LT, int NT>
__device__ __forceinline__ float thread_max(const LT* x, int64_t hi) {
  constexpr int N = 16 / sizeof(LT);
  constexpr int64_t kStep = (int64_t)NT * N;
  using IO = IntOrder<LT>;
  const bool aligned = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  const int64_t first = (int64_t)threadIdx.x * N;
  auto word = [&](int64_t v0, int w) -> uint32_t {  // entries past hi read as -inf
    if constexpr (sizeof(LT) == 4) {
      return v0 + w < hi ? __builtin_bit_cast(uint32_t, x[v0 + w]) : (uint32_t)IO::kNegInf;
    } else {
      const uint32_t ninf = (uint32_t)IO::kNegInf & 0xFFFFu;
      const uint32_t lo = v0 + 2 * w < hi ? (uint32_t)__builtin_bit_cast(uint16_t, x[v0 + 2 * w]) : ninf;
      const uint32_t hi16 = v0 + 2 * w + 1 < hi ? (uint32_t)__builtin_bit_cast(uint16_t, x[v0 + 2 * w + 1]) : ninf;
      return lo | (hi16 << 16);
    }
  };
  int hmax, hmin;
  if constexpr (sizeof(LT) == 4) {
    int pmax = INT32_MIN, nmin = INT32_MAX;
    auto take = [&](const u32x4& r) {
      pmax = max(max(pmax, (int)r[0]), max((int)r[1], max((int)r[2], (int)r[3])));
      nmin = min(min(nmin, (int)r[0]), min((int)r[1], min((int)r[2], (int)r[3])));
    };
    int64_t v0 = first;
    for (; aligned && v0 + 3 * kStep + N <= hi; v0 += 4 * kStep) {
      u32x4 r[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) r[u] = *reinterpret_cast<const u32x4*>(x + v0 + u * kStep);
#pragma unroll
      for (int u = 0; u < 4; ++u) take(r[u]);
    }
    for (; v0 < hi; v0 += kStep) {
      u32x4 r;
      if (aligned && v0 + N <= hi)
        r = *reinterpret_cast<const u32x4*>(x + v0);
      else
        r = u32x4{word(v0, 0), word(v0, 1), word(v0, 2), word(v0, 3)};
      take(r);
    }
    hmax = pmax;
    hmin = nmin;
  } else {
    s16x2 pmax = {(short)-32768, (short)-32768}, nmin = {(short)32767, (short)32767};
    auto take = [&](const u32x4& r) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t rw = r[w];  // (a bit cast of the element itself reads element 0)
        const s16x2 s = __builtin_bit_cast(s16x2, rw);
        pmax = __builtin_elementwise_max(pmax, s);
        nmin = __builtin_elementwise_min(nmin, s);
      }
    };
    int64_t v0 = first;
    for (; aligned && v0 + 3 * kStep + N <= hi; v0 += 4 * kStep) {
      u32x4 r[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) r[u] = *reinterpret_cast<const u32x4*>(x + v0 + u * kStep);
#pragma unroll
      for (int u = 0; u < 4; ++u) take(r[u]);
    }
    for (; v0 < hi; v0 += kStep) {
      u32x4 r;
      if (aligned && v0 + N <= hi)
        r = *reinterpret_cast<const u32x4*>(x + v0);
      else
        r = u32x4{word(v0, 0), word(v0, 1), word(v0, 2), word(v0, 3)};
      take(r);
    }
    hmax = max((int)pmax.x, (int)pmax.y);
    hmin = min((int)nmin.x, (int)nmin.y);
  }
  if (hmax > IO::kInf) {  // a positive NaN: entry by entry, NaN as -inf
    float m = kNegInfF;
    for (int64_t v0 = first; v0 < hi; v0 += kStep)
      for (int e = 0; e < N && v0 + e < hi; ++e) m = fmaxf(m, clean_y(raw_to_f<LT>(x[v0 + e])));
    return m;
  }
  if (hmax >= 0) return int_to_f<LT>(hmax);
  if (hmin <= IO::kNegInf) return int_to_f<LT>(hmin);
  return kNegInfF;  // no entries, or only negative NaNs
}

// warp_vec without clean_y (NaN stays NaN, -0 stays -0), for 16-bit logits:
// y = x / T rounded to the dtype, from q = x * fl(1/T).  q lies within 3 fp32
// ulp of the correctly rounded quotient (for bf16 also among the subnormals,
// whose spacing is that of the smallest binade and whose bf16 rounding reads
// the same low 16 bits), so both round to the same 16-bit value unless q is
// within 8 ulp of a rounding midpoint; the division decides there and, for
// f16, outside its normal range.
template <typename LT, int N>
__device__ __forceinline__ void warp_vec_raw(float (&y)[N], const Warp& w) {
  if constexpr (sizeof(LT) == 2) {
    constexpr bool kF16 = __is_same(LT, _Float16);
    constexpr int LOW = kF16 ? 13 : 16;
    constexpr uint32_t MID = 1u << (LOW - 1);
    float q[N];
    bool unsafe[N], any = false;
#pragma unroll
    for (int e = 0; e < N; ++e) {
      q[e] = y[e] * w.rT;
      const uint32_t low = __float_as_uint(q[e]) & ((1u << LOW) - 1u);
      bool u = low - (MID - 8u) <= 16u;
      if constexpr (kF16) {
        const float aq = fabsf(q[e]);
        u |= !(aq >= 0x1p-14f && aq <= 32768.f);
      }
      unsafe[e] = u;
      any |= u;
    }
    if (__ballot(any) != 0ull) {
#pragma unroll
      for (int e = 0; e < N; ++e)
        if (unsafe[e]) q[e] = y[e] / w.T;
    }
#pragma unroll
    for (int e = 0; e < N; ++e) y[e] = round_lt<LT>(q[e]);
  } else {
#pragma unroll
    for (int e = 0; e < N; ++e) y[e] = y[e] / w.T;
  }
}

// The bits of the smallest logit x (in the dtype's order, NaN excluded) whose
// warped y is at least thr; thr is not NaN, so +inf qualifies.  The warper
// is monotone, so {x : y(x) >= thr} = {x >= result}.  Wave-parallel search
// over the order keys: each round the 64 lanes test 64 evenly spaced keys.
// Every lane of the wave calls it and gets the result.
template <typename LT>
__device__ __forceinline__ uint32_t x_threshold_bits(float thr, const Warp& w) {
  constexpr bool k16 = sizeof(LT) == 2;
  const uint32_t sign = k16 ? 0x8000u : 0x80000000u, all = k16 ? 0xFFFFu : 0xFFFFFFFFu;
  const uint32_t inf = (uint32_t)IntOrder<LT>::kInf, ninf = ((uint32_t)IntOrder<LT>::kNegInf) & all;
  auto key_of = [&](uint32_t b) { return (b & sign) ? (b ^ all) : (b ^ sign); };
  auto bits_of = [&](uint32_t k) { return (k & sign) ? (k ^ sign) : (k ^ all); };
  auto passes = [&](uint32_t k) {
    const uint32_t b = bits_of(k);
    return warp_yf<LT>(int_to_f<LT>((int)b), w) >= thr;
  };
  const int lane = threadIdx.x & 63;
  uint64_t lo = key_of(ninf), hi = key_of(inf);  // the answer lies in [lo, hi]
  while (lo < hi) {
    const uint64_t step = (hi - lo + 64) / 64;
    const uint64_t p = min(lo + (uint64_t)(lane + 1) * step - 1, hi);
    const uint64_t bal = __ballot(passes((uint32_t)p));
    const int l = __builtin_ctzll(bal);  // the last lane tests hi, which passes
    const uint64_t nhi = min(lo + (uint64_t)(l + 1) * step - 1, hi);
    lo = l == 0 ? lo : lo + (uint64_t)l * step;
    hi = nhi;
  }
  return bits_of((uint32_t)lo);
}
template <typename LT>
__device__ __forceinline__ float x_threshold(float thr, const Warp& w) {
  return int_to_f<LT>((int)x_threshold_bits<LT>(thr, w));
}

// Histogram bins of a = (y - m) log2 e, read off |a|'s bits (exponent and first
// mantissa bit): bin 0 holds |a| < kTheta[0], bin j (1..15) kTheta[j-1] <= |a|
// < kTheta[j], bin 16 the rest (and NaN).
constexpr int kBins = kNTheta + 1;
// The statistics pass also keeps, per wave, the entries with a >= -g in a
// region of kPre / waves entries: g starts at kPreG0 and drops by 2 (the
// region compacted) whenever the region would overflow, down to kPreGMin.
// a is the same fp32 expression wherever it is evaluated, and monotone in y,
// so {a >= -theta} is a head of the order, held by the regions when theta <=
// the smallest g of the waves.
constexpr float kPreG0 = 16.f, kPreGMin = 2.f;
constexpr int kPre = 2048;  // entries of the regions of a block

// Four waves per SIMD (at most 128 VGPRs): two 512-thread rows share a CU.
template <typename LT, int NT>
__global__ void __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4))) sample_select_kernel(const AcceptArgs a) {
  static_assert(kCap % NT == 0, "candidates split evenly over the threads");
  constexpr int kWaves = NT / 64;
  constexpr int kHistWords = kWaves * kBins * 64;
  constexpr int kPreCap = kPre / kWaves;  // entries of a wave's region of pre
  static_assert(kHistWords >= 2 * kCap && kCap >= 2 * NT, "the candidates (and a sorted copy of up to NT) fit where the histograms were");
  const int64_t row = blockIdx.x;
  const int t = (int)(row / a.M), i = (int)(row % a.M);
  const LT* x = reinterpret_cast<const LT*>(a.logits) + (int64_t)t * a.l_st + (int64_t)i * a.l_sm;
  const int V = (int)a.V;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6;
  const Warp wp = make_warp(a.temperature);
  constexpr int NV = 16 / sizeof(LT);

  // hist: the per-lane histograms of the histogram pass (rows whose regions
  // do not hold the cut), and the head's candidates ((key << 32) | index).
  // pre: the waves' regions of entries near the maximum, (index << 32) | bits
  // of y.
  __shared__ __align__(16) uint32_t hist[kHistWords];
  __shared__ __align__(16) uint64_t pre[kPre];
  uint64_t* cand = reinterpret_cast<uint64_t*>(hist);
  __shared__ float red_f[kWaves];
  __shared__ uint32_t pre_n[kWaves];
  __shared__ float pre_g[kWaves];
  __shared__ float wbin_q[kWaves][kBins];
  __shared__ uint32_t wbin_c[kWaves][kBins];
  __shared__ uint32_t cnt_th[kNTheta];
  __shared__ uint32_t ncand, nk_lo, nk_hi;
  __shared__ int jsel[3];
  __shared__ float xthr_s;
  __shared__ uint64_t red_q[kWaves];
  __shared__ double red_d[kWaves];
  __shared__ int red_i[kWaves];

  // Row maximum of y: the warper is monotone, so it is the warped maximum
  // logit (xm).
  float m = thread_max<LT, NT>(x, V);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if (lane == 0) red_f[wv] = m;
  __syncthreads();
  float xm = red_f[0];
  for (int w = 1; w < kWaves; ++w) xm = fmaxf(xm, red_f[w]);
  m = xm > kNegInfF ? warp_y<LT>(f_to_raw<LT>(xm), wp) : kNegInfF;

  int S = 63;
  for (int vv = V; vv > 0; vv >>= 1) --S;  // 63 - bitlen(V)

  const int64_t kk = (a.top_k > 0 && a.top_k < V) ? a.top_k : 0;
  const bool use_p = a.top_p_q != 0;
  // The row's draw, written by thread 0 as range 0's result (the other
  // ranges report none); the sweep then skips the row.
  auto finish = [&](double z, int idx) {
    const uint64_t zb = __builtin_bit_cast(uint64_t, z);
    for (int c = 0; c < a.nchunk; ++c)
      a.rstat[row * a.nchunk + c] =
          c == 0 ? make_float4(__uint_as_float((uint32_t)zb), __uint_as_float((uint32_t)(zb >> 32)), __int_as_float(idx), 0.f)
                 : make_float4(0.f, 0.f, __int_as_float(-1), 0.f);
    a.sel[row] = make_uint4(0u, 0u, 0u, 1u);
  };
  if (!(m > kNegInfF)) {  // no finite logit: nothing is kept (token 0)
    if (tid == 0) finish(0.0, -1);
    return;
  }
  if (!use_p && kk == 0) {  // top-k of at least V: everything is kept
    if (tid == 0) a.sel[row] = make_uint4(0u, 0u, 0u, 0u);
    return;
  }
  if (!(m < -kNegInfF)) {  // +inf maximum: the radix kernel's exact masses
    if (tid == 0) a.sel[row] = make_uint4(__float_as_uint(m), 0u, 0u, 2u);
    return;
  }

  // ---- statistics: exact y, the fp32 sum of 2^a, the entries near m ---------
  for (int q = tid; q < kWaves * kBins; q += NT) {
    wbin_c[q / kBins][q % kBins] = 0;
    wbin_q[q / kBins][q % kBins] = 0.f;
  }
  if (tid == 0) {
    ncand = 0;
    nk_lo = 0;
    nk_hi = 0;
  }
  __syncthreads();
  const float mc = m * 0x1.715476p+0f;
  // a of a logit's warped value: the one fp32 expression used for every decision on a.
  auto a_of = [&](float y) { return fmaf(y, 0x1.715476p+0f, -mc); };
  uint64_t* pw = pre + wv * kPreCap;
  // Per-wave bins of the appended entries (count of bin b at wbin_c[wv][b],
  // fp32 mass at wbin_q[wv][b]); bins past the final bound also count entries
  // the compaction dropped, and are not used.
  uint32_t pcnt = 0;   // entries in this wave's region (the same in every lane)
  float gw = kPreG0;   // this wave's bound (the same in every lane); below kPreGMin: given up
  float lsum = 0.f;    // top-p: sum of 2^a over the row (fp32)
  // Keeps the region's entries with a >= -gw, in order (the wave's lanes read
  // a chunk before they write below it).
  auto compact = [&]() {
    uint32_t nk = 0;
    for (uint32_t s0 = 0; s0 < pcnt; s0 += 64) {
      const uint32_t q = s0 + (uint32_t)lane;
      const uint64_t cv = q < pcnt ? pw[q] : 0ull;
      const bool keep = q < pcnt && a_of(__uint_as_float((uint32_t)cv)) >= -gw;
      const uint64_t bal = __ballot(keep);
      if (keep) pw[nk + (uint32_t)__popcll(bal & ((1ull << lane) - 1ull))] = cv;
      nk += (uint32_t)__popcll(bal);
    }
    pcnt = nk;
  };
  row_sweep<LT, NT, false, true>(x, 0, V, wp, [&](int64_t v0, const float(&xv)[NV]) {
    float y[NV], ar[NV];
#pragma unroll
    for (int e = 0; e < NV; ++e) y[e] = xv[e];
    if (wp.T != 1.f) warp_vec_raw<LT, NV>(y, wp);
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      ar[e] = a_of(y[e]);
      if (use_p) lsum += __builtin_amdgcn_exp2f(ar[e]);  // NaN y: the sum is NaN
    }
    // This vector's entries near the maximum, appended to the wave's region
    // (the bound lowered first while they would overflow it).
    uint64_t bal[NV];
    uint32_t tot = 0;
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      bal[e] = __ballot(ar[e] >= -gw);
      tot += (uint32_t)__popcll(bal[e]);
    }
    if (tot != 0u && gw >= kPreGMin) {
      while (pcnt + tot > (uint32_t)kPreCap && gw >= kPreGMin) {
        gw -= 2.f;
        compact();
        tot = 0;
#pragma unroll
        for (int e = 0; e < NV; ++e) {
          bal[e] = __ballot(ar[e] >= -gw);
          tot += (uint32_t)__popcll(bal[e]);
        }
      }
      if (gw >= kPreGMin) {
#pragma unroll
        for (int e = 0; e < NV; ++e) {
          if (bal[e] != 0ull) {
            if ((bal[e] >> lane) & 1ull) {
              pw[pcnt + (uint32_t)__popcll(bal[e] & ((1ull << lane) - 1ull))] =
                  ((uint64_t)(uint32_t)(v0 + e) << 32) | __float_as_uint(y[e]);
              const uint32_t b = min(max((__float_as_uint(ar[e]) >> 22) & 0x1FFu, 249u), 249u + kNTheta) - 249u;
              atomicAdd(&wbin_c[wv][b], 1u);
              atomicAdd(&wbin_q[wv][b], __builtin_amdgcn_exp2f(ar[e]));
            }
            pcnt += (uint32_t)__popcll(bal[e]);
          }
        }
      }
    }
  });
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) lsum += __shfl_xor(lsum, o);
  if (lane == 0) {
    red_f[wv] = lsum;
    pre_n[wv] = pcnt;
    pre_g[wv] = gw;
  }
  __syncthreads();
  float L = 0.f, gcov = kPreG0;  // the regions hold every entry with a >= -gcov
  for (int w = 0; w < kWaves; ++w) {
    L += red_f[w];
    gcov = fminf(gcov, pre_g[w]);
  }
  if (use_p && !(L == L)) {  // NaN logits (NaN counts as -inf): the radix kernel
    if (tid == 0) a.sel[row] = make_uint4(__float_as_uint(m), 0u, 0u, 2u);
    return;
  }
  const float need = (float)a.top_p_q * 0x1p-32f * L * (1.f + 0x1p-8f);
  // Counts and fp32 masses of the regions' entries per bin of a (bin 0: |a| <
  // kTheta[0], bin j: kTheta[j-1] <= |a| < kTheta[j], read off |a|'s exponent
  // and first mantissa bit); with gcov >= kTheta[j], bins 0..j of the regions
  // are the whole head {a > -kTheta[j]}.
  if (wv == 0) {
    // The narrowest head within gcov whose fp32 mass reaches top_p of the
    // total (top-k alone: holding k), marked kNTheta + j (taken from the
    // regions): lane j sums bin j over the waves, then inclusive prefix sums.
    float hq = 0.f;
    uint32_t hc = 0;
    if (lane < kNTheta) {
      for (int w = 0; w < kWaves; ++w) {
        hq += wbin_q[w][lane];
        hc += wbin_c[w][lane];
      }
    }
#pragma unroll
    for (int o = 1; o < kNTheta; o <<= 1) {
      const float q2 = __shfl_up(hq, o);
      const uint32_t c2 = __shfl_up(hc, o);
      if (lane >= o) {
        hq += q2;
        hc += c2;
      }
    }
    const bool reach = lane < kNTheta && gcov >= kPreGMin && kTheta[lane < kNTheta ? lane : 0] <= gcov &&
                       (use_p ? hq >= need : hc >= (uint64_t)kk);
    const uint64_t bal = __ballot(reach);
    if (lane == 0) {
      jsel[0] = bal != 0ull ? kNTheta + __builtin_ctzll(bal) : -1;
      jsel[1] = -2;  // the histogram's heads: not counted yet
    }
  }
  __syncthreads();

  // Histogram of a over the row, for the rows whose regions do not hold the
  // cut: per-lane counts in LDS (hist), then jsel[1..2]: top-k alone, the
  // narrowest head holding k; top-p, first the narrowest head whose mass
  // surely reaches top_p of the total (an entry of bin j has mass above
  // 2^-kTheta[j]), then the widest head that fits.
  auto histogram_heads = [&]() {
    for (int q = tid; q < kHistWords; q += NT) hist[q] = 0;
    if (tid < kNTheta) cnt_th[tid] = 0;
    __syncthreads();
    uint32_t* hb = hist + wv * kBins * 64 + lane - 249 * 64;  // bin b9 - 249 of this lane at hb[b9 * 64]
    row_sweep<LT, NT, false, true>(x, 0, V, wp, [&](int64_t, const float(&xv)[NV]) {
      float y[NV];
#pragma unroll
      for (int e = 0; e < NV; ++e) y[e] = xv[e];
      if (wp.T != 1.f) warp_vec_raw<LT, NV>(y, wp);
#pragma unroll
      for (int e = 0; e < NV; ++e) {
        const uint32_t b9 = min(max((__float_as_uint(a_of(y[e])) >> 22) & 0x1FFu, 249u), 249u + kNTheta);
        atomicAdd(hb + b9 * 64, 1u);
      }
    });
    __syncthreads();
    uint32_t c = 0, cth[kNTheta];
#pragma unroll
    for (int j = 0; j < kNTheta; ++j) {
      c += hb[(249 + j) * 64];
      cth[j] = c;
    }
#pragma unroll
    for (int j = 0; j < kNTheta; ++j) {
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) cth[j] += __shfl_xor(cth[j], o);
    }
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < kNTheta; ++j) atomicAdd(&cnt_th[j], cth[j]);
    }
    __syncthreads();
    if (tid == 0) {
      int j0 = -1, j1 = -1;
      if (use_p) {
        float head = 0.f;
        for (int j = 0; j < kNTheta && cnt_th[j] <= (uint32_t)kCap; ++j) {
          head += (float)(cnt_th[j] - (j > 0 ? cnt_th[j - 1] : 0u)) * exp2f(-kTheta[j]);
          if (j0 < 0 && head >= need) j0 = j;
          j1 = j;
        }
        if (j0 < 0 || j0 == j1) {
          j0 = j1;
          j1 = -1;
        }
      } else {
        for (int j = 0; j < kNTheta && j0 < 0; ++j)
          if (cnt_th[j] >= (uint64_t)kk && cnt_th[j] <= (uint32_t)kCap) j0 = j;
      }
      jsel[1] = j0;
      jsel[2] = j1;
      ncand = 0;
      nk_lo = 0;
      nk_hi = 0;
    }
    __syncthreads();
  };

  // Attempt 0: the regions' head; attempts 1, 2: the histogram's heads.
  for (int att = 0; att < 3; ++att) {
    if (att == 1 && jsel[1] == -2) histogram_heads();
    const int js = jsel[att];
    if (js < 0) {
      if (att == 0) continue;
      break;
    }
    if (att == 2 && tid == 0) {
      ncand = 0;
      nk_lo = 0;
      nk_hi = 0;
    }
    if (att == 2) __syncthreads();
    if (js >= kNTheta) {
      // From the waves' regions: the head {a > -kTheta[j]} (bins 0..j).
      const float ath = -kTheta[js - kNTheta];
      for (int q0 = 0; q0 < kPre; q0 += NT) {
        const int q = q0 + tid;
        const uint64_t pv = pre[q];
        const float yq = __uint_as_float((uint32_t)pv);
        const bool c = (uint32_t)(q % kPreCap) < pre_n[q / kPreCap] && a_of(yq) > ath;
        const uint64_t cv = ((uint64_t)ykey(yq == 0.f ? 0.f : yq) << 32) | (pv >> 32);
        const uint64_t bal = __ballot(c);
        if (bal != 0ull) {
          uint32_t base = 0;
          if (lane == 0) base = atomicAdd(&ncand, (uint32_t)__popcll(bal));
          base = __shfl(base, 0);
          if (c) cand[base + (uint32_t)__popcll(bal & ((1ull << lane) - 1ull))] = cv;
        }
      }
    } else {
      // A pass over the row for the head {y >= thr}: by the warper's monotony,
      // {x >= x_thr} on the logits.
      const float thr = m - kTheta[js] * 0x1.62e430p-1f;
      if (wv == 0) {
        const float xt = x_threshold<LT>(thr, wp);
        if (lane == 0) xthr_s = xt;
      }
      __syncthreads();
      const float xthr = xthr_s;
      row_sweep<LT, NT, false, true>(x, 0, V, wp, [&](int64_t v0, const float(&xv)[NV]) {
        bool any = false;
#pragma unroll
        for (int e = 0; e < NV; ++e) any |= xv[e] >= xthr;
        if (__ballot(any) == 0ull) return;
#pragma unroll
        for (int e = 0; e < NV; ++e) {
          const bool c = xv[e] >= xthr;
          const uint64_t bal = __ballot(c);
          if (bal != 0ull) {
            uint32_t base = 0;
            if (lane == 0) base = atomicAdd(&ncand, (uint32_t)__popcll(bal));
            base = __shfl(base, 0);
            if (c) {
              const uint32_t slot = base + (uint32_t)__popcll(bal & ((1ull << lane) - 1ull));
              if (slot < (uint32_t)kCap) cand[slot] = ((uint64_t)ykey(warp_yf<LT>(xv[e], wp)) << 32) | (uint32_t)(v0 + e);
            }
          }
        }
      });
    }
    __syncthreads();
    const int n = min((int)ncand, kCap);
    // The counts chose the threshold; the gathered count decides whether the
    // head fits and holds k entries.
    const bool fits = (int)ncand <= kCap && (use_p || (int64_t)ncand >= kk);
    // Sorted descending: up to NT entries by rank (keys are distinct: they
    // carry the index) into cand[NT, 2 NT); more by a bitonic sort in place,
    // padded with zero keys to a power of two.
    const uint64_t* keys = cand;
    if (n <= NT) {
      uint64_t* out = cand + NT;  // above the n <= NT candidates
      if (tid < n) {
        const uint64_t mine = cand[tid];
        int rank = 0;
#pragma unroll 8
        for (int j = 0; j < n; ++j) rank += cand[j] > mine ? 1 : 0;
        out[rank] = mine;
      }
      keys = out;
    } else {
      int npad = 2;
      while (npad < n) npad <<= 1;
      for (int q = n + tid; q < npad; q += NT) cand[q] = 0ull;
      __syncthreads();
      // Each stage's npad / 2 pairs (q, q | j2), q with bit j2 clear: a
      // thread loads two pairs before comparing (the pairs of a stage are
      // disjoint), so that their LDS round trips overlap.
      for (int k2 = 2; k2 <= npad; k2 <<= 1)
        for (int j2 = k2 >> 1; j2 > 0; j2 >>= 1) {
          const int lj = __builtin_ctz(j2);
          for (int p0 = tid; p0 < npad / 2; p0 += 2 * NT) {
            const bool h1 = p0 + NT < npad / 2;
            const int p1 = h1 ? p0 + NT : p0;  // (without a second pair: the first again, not stored)
            const int q0 = ((p0 >> lj) << (lj + 1)) | (p0 & (j2 - 1));
            const int q1 = ((p1 >> lj) << (lj + 1)) | (p1 & (j2 - 1));
            const uint64_t u0 = cand[q0], w0 = cand[q0 | j2];
            const uint64_t u1 = cand[q1], w1 = cand[q1 | j2];
            if (((q0 & k2) == 0) ? (u0 < w0) : (u0 > w0)) {
              cand[q0] = w0;
              cand[q0 | j2] = u0;
            }
            if (h1 && (((q1 & k2) == 0) ? (u1 < w1) : (u1 > w1))) {
              cand[q1] = w1;
              cand[q1 | j2] = u1;
            }
          }
          __syncthreads();
        }
    }
    __syncthreads();
    // top-k: the k-th key when the candidates hold k (else every candidate
    // passes top-k, and the cut comes from top-p inside the candidates).
    const uint32_t tk = (kk > 0 && n >= kk) ? (uint32_t)(keys[kk - 1] >> 32) : 0u;
    int nkeep = n;
    bool ok = fits;
    if (use_p && ok) {
      // Exact masses along the order (thread tid holds entries ept * tid ..
      // + ept - 1) and their exclusive prefix sums.
      constexpr int EPT = kCap / NT;
      const int ept = (n + NT - 1) / NT;
      uint64_t qv[EPT], tot = 0;
#pragma unroll
      for (int u = 0; u < EPT; ++u) {
        const int e = ept * tid + u;
        qv[u] = (u < ept && e < n) ? fixed_mass(key_to_y((uint32_t)(keys[e] >> 32)), m, S) : 0ull;
        tot += qv[u];
      }
      uint64_t incl = tot;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint64_t y2 = __shfl_up(incl, o);
        if (lane >= o) incl += y2;
      }
      if (lane == 63) red_q[wv] = incl;
      __syncthreads();
      uint64_t wbase = 0, H = 0;
      for (int w = 0; w < kWaves; ++w) {
        if (w < wv) wbase += red_q[w];
        H += red_q[w];
      }
      // L = sum of the exact masses, bounded from the fp32 sum of 2^a over the
      // row: relative error below (summands per thread + 8 + waves) 2^-24
      // from the sum, 2^-16 from the hardware 2^x and the rounding of a
      // (|a| <= 64; smaller masses are within the integer slack), and 2^-22 |m|
      // from the rounding of m log2 e; each mass's integer rounding adds V.
      const double Lq = (double)L * __builtin_ldexp(1.0, S);
      const double eps = ((double)((V + NT - 1) / NT) + 8.0 + kWaves) * 0x1p-24 + 0x1p-16 +
                         0x1p-22 * __builtin_fabs((double)m);
      // Every mass is at most 2^S and V * 2^S < 2^63, so L < 2^63: the upper
      // bound is capped there (and still converts to uint64 exactly).
      const double llo = __builtin_fmax(0.0, Lq * (1.0 - eps) - (double)V);
      const double lhi = __builtin_fmin(Lq * (1.0 + eps) + (double)V + 1.0, 0x1p63);
      const uint64_t L_lo = max(H, (uint64_t)__builtin_floor(llo));
      const uint64_t L_hi = max(H, (uint64_t)__builtin_ceil(lhi));
      const uint64_t tq_lo = tq_of(a.top_p_q, L_lo);
      const uint64_t tq_hi = tq_of(a.top_p_q, L_hi);
      uint32_t cl = 0, ch = 0;
      uint64_t above = wbase + incl - tot;
#pragma unroll
      for (int u = 0; u < EPT; ++u) {
        if (u < ept && ept * tid + u < n) {
          cl += above < tq_lo;
          ch += above < tq_hi;
        }
        above += qv[u];
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        cl += __shfl_xor(cl, o);
        ch += __shfl_xor(ch, o);
      }
      if (lane == 0) {
        atomicAdd(&nk_lo, cl);
        atomicAdd(&nk_hi, ch);
      }
      __syncthreads();
      // Decided: the first non-candidate (mass H above it) is dropped for
      // every L in the bounds, and so is the same head of the candidates.
      ok = L_lo <= L_hi && H >= tq_hi && nk_lo == nk_hi;
      nkeep = (int)nk_hi;
    }
    if (ok) {
      double bz = -__builtin_huge_val();
      int bi = -1;
      for (int q = tid; q < n; q += NT) {
        const uint64_t cv = keys[q];
        const uint32_t key = (uint32_t)(cv >> 32);
        const int v = (int)(uint32_t)cv;
        if (q < nkeep && key >= tk) {
          const double z = (double)key_to_y(key) + gumbel(draw_word(v, i, t, a.seed));
          if (bi < 0 || z > bz || (z == bz && v < bi)) {
            bz = z;
            bi = v;
          }
        }
      }
      block_argmax(bz, bi, red_d, red_i, NT);
      if (tid == 0) finish(bz, bi);
      return;
    }
    __syncthreads();
  }

  // ---- not decided here: the radix kernel takes the row (status 2, with m) --
  if (tid == 0) a.sel[row] = make_uint4(__float_as_uint(m), 0u, 0u, 2u);
}

// Radix selection for the rows the select kernel left open (status 2): the
// top-k key, the top-p cut key and, in the cut's tie group, the index bound;
// the kept set is then gathered and drawn here when it fits in LDS, else the
// bounds go to the sweep kernel.
template <typename LT>
__global__ void __launch_bounds__(kRadixThreads) sample_radix_kernel(const AcceptArgs a) {
  const int64_t row = blockIdx.x;
  const uint4 st = a.sel[row];
  if (st.w != 2u) return;
  const int t = (int)(row / a.M), i = (int)(row % a.M);
  const LT* x = reinterpret_cast<const LT*>(a.logits) + (int64_t)t * a.l_st + (int64_t)i * a.l_sm;
  const int V = (int)a.V;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  constexpr int ND = key_digits<LT>();
  constexpr int NV = 16 / sizeof(LT);
  const Warp wp = make_warp(a.temperature);
  const float m = __uint_as_float(st.x);  // the row maximum of y, from the select kernel
  int S = 63;
  for (int vv = V; vv > 0; vv >>= 1) --S;  // 63 - bitlen(V)
  const int64_t kk = (a.top_k > 0 && a.top_k < V) ? a.top_k : 0;
  const bool use_p = a.top_p_q != 0;
  (void)kk;

  __shared__ uint64_t hist[256];
  __shared__ uint32_t res_u[4];
  __shared__ uint64_t res_q[4];
  __shared__ uint64_t cand[kCap];
  __shared__ uint32_t ncand, nk_lo;
  __shared__ double red_d[kRadixThreads / 64];
  __shared__ int red_i[kRadixThreads / 64];
  auto finish = [&](double z, int idx) {
    const uint64_t zb = __builtin_bit_cast(uint64_t, z);
    for (int c = 0; c < a.nchunk; ++c)
      a.rstat[row * a.nchunk + c] =
          c == 0 ? make_float4(__uint_as_float((uint32_t)zb), __uint_as_float((uint32_t)(zb >> 32)), __int_as_float(idx), 0.f)
                 : make_float4(0.f, 0.f, __int_as_float(-1), 0.f);
    a.sel[row] = make_uint4(0u, 0u, 0u, 1u);
  };

  // ---- radix selection over the whole row -------------------------------------

  // One radix pass: histogram of digit `shift` over the elements whose key
  // matches `prefix` above that digit (and, for the tie pass, key == tie_key
  // with the index as the digit source), weighted by count or mass.
  auto pass = [&](int shift, uint32_t prefix, bool mass, bool by_index, uint32_t tie_key) {
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    const uint32_t hi_mask = shift >= 24 ? 0u : ~((1u << (shift + 8)) - 1u);
    row_sweep<LT, kRadixThreads>(x, 0, V, wp, [&](int64_t v0, const float(&y)[NV]) {
#pragma unroll
      for (int e = 0; e < NV; ++e) {
        const uint32_t k = ykey(y[e]);
        const uint32_t src = by_index ? (uint32_t)(v0 + e) : k;
        const bool valid = v0 + e < V && (!by_index || k == tie_key) && (src & hi_mask) == (prefix & hi_mask);
        if (valid)
          atomicAdd(reinterpret_cast<unsigned long long*>(&hist[(src >> shift) & 255u]),
                    (unsigned long long)(mass ? fixed_mass(y[e], m, S) : 1ull));
      }
    });
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

  // top-p: the key of the last kept element (ystar), then the index bound in
  // its tie group (istar).
  uint32_t ystar = 0, istar = 0;
  uint64_t above = 0, Tq = 0;
  if (use_p) {
    uint32_t prefix = 0;
    for (int d = 0; d < ND; ++d) {
      const int shift = 24 - 8 * d;
      if (d > 0 && d == ND - 1) {
        // The last digit completes the key: every bin holds one value of y,
        // so its mass is its count times that value's mass.
        pass(shift, prefix, false, false, 0);
        if (tid < 256 && hist[tid] != 0ull)
          hist[tid] *= fixed_mass(key_to_y(fill_low(prefix | ((uint32_t)tid << shift), ND)), m, S);
        __syncthreads();
      } else {
        pass(shift, prefix, true, false, 0);
      }
      if (d == 0 && tid < 64) {
        // Total mass L and the threshold Tq = ceil(P * L / 2^32).
        uint64_t s = hist[4 * tid] + hist[4 * tid + 1] + hist[4 * tid + 2] + hist[4 * tid + 3];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
        if (tid == 0) res_q[1] = tq_of(a.top_p_q, s);
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
  }
  if (ystar == 0xFFFFFFFFu) {  // nothing is kept
    if (tid == 0) a.sel[row] = make_uint4(tk, ystar, 0u, 0u);
    return;
  }
  // Mass q* of one member of the cut's tie group, and how many of the group
  // (its highest indices) the cut keeps: n_keep = #{j : above + j q* < Tq}.
  const uint64_t qs = use_p ? fixed_mass(key_to_y(ystar), m, S) : 0ull;
  auto keep_of = [&](uint64_t group) -> uint64_t {
    if (!use_p || qs == 0) return group;
    const uint64_t need = (Tq - above + qs - 1) / qs;
    return need < group ? need : group;
  };
  // The index bound among the tie members: the rank-th largest index, digit
  // by digit (8-bit digits over bitlen(V - 1) bits); count(shift, prefix)
  // fills hist with the digit counts of the members that match prefix above.
  auto index_bound = [&](uint64_t rank, auto&& count) -> uint32_t {
    int ib = 0;
    for (int vv = V - 1; vv > 0; vv >>= 1) ++ib;
    uint32_t ipre = 0;
    for (int d = (ib + 7) / 8 - 1; d >= 0; --d) {
      const int shift = 8 * d;
      count(shift, ipre);
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
    return ipre;
  };

  // ---- the kept set in LDS: every entry with key >= max(tk, ystar) ----------
  // When it fits, the tie bound and the draw are taken here; otherwise the
  // bounds go to the sweep kernel.
  {
    const uint32_t lower = max(tk, ystar);
    uint32_t* list = reinterpret_cast<uint32_t*>(cand);  // kList indices
    constexpr int kList = 2 * kCap;
    if (tid == 0) ncand = 0;
    __syncthreads();
    row_sweep<LT, kRadixThreads>(x, 0, V, wp, [&](int64_t v0, const float(&y)[NV]) {
      bool any = false;
#pragma unroll
      for (int e = 0; e < NV; ++e) any |= v0 + e < V && ykey(y[e]) >= lower;
      if (__ballot(any) == 0ull) return;
#pragma unroll
      for (int e = 0; e < NV; ++e) {
        const bool c = v0 + e < V && ykey(y[e]) >= lower;
        const uint64_t bal = __ballot(c);
        if (bal != 0ull) {
          uint32_t base = 0;
          if (lane == 0) base = atomicAdd(&ncand, (uint32_t)__popcll(bal));
          base = __shfl(base, 0);
          if (c) {
            const uint32_t slot = base + (uint32_t)__popcll(bal & ((1ull << lane) - 1ull));
            if (slot < (uint32_t)kList) list[slot] = (uint32_t)(v0 + e);
          }
        }
      }
    });
    __syncthreads();
    const int nl = (int)ncand;
    if (nl <= kList) {
      auto key_at = [&](int q) { return ykey(warp_y<LT>(x[list[q]], wp)); };
      if (use_p && ystar >= tk) {
        uint32_t g = 0;
        for (int q = tid; q < nl; q += kRadixThreads) g += key_at(q) == ystar ? 1u : 0u;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) g += __shfl_xor(g, o);
        if (tid == 0) nk_lo = 0;
        __syncthreads();
        if (lane == 0) atomicAdd(&nk_lo, g);
        __syncthreads();
        const uint64_t group = nk_lo;
        const uint64_t n_keep = keep_of(group);
        if (n_keep < group)
          istar = index_bound(n_keep, [&](int shift, uint32_t ipre) {
            if (tid < 256) hist[tid] = 0;
            __syncthreads();
            const uint32_t hi_mask = shift >= 24 ? 0u : ~((1u << (shift + 8)) - 1u);
            for (int q = tid; q < nl; q += kRadixThreads) {
              const uint32_t v = list[q];
              if (key_at(q) == ystar && (v & hi_mask) == (ipre & hi_mask))
                atomicAdd(reinterpret_cast<unsigned long long*>(&hist[(v >> shift) & 255u]), 1ull);
            }
            __syncthreads();
          });
      }
      double bz = -__builtin_huge_val();
      int bi = -1;
      for (int q = tid; q < nl; q += kRadixThreads) {
        const int v = (int)list[q];
        const float y = warp_y<LT>(x[v], wp);
        const uint32_t k = ykey(y);
        if (k >= tk && (k > ystar || (k == ystar && (uint32_t)v >= istar))) {
          const double z = (double)y + gumbel(draw_word(v, i, t, a.seed));
          if (bi < 0 || z > bz || (z == bz && v < bi)) {
            bz = z;
            bi = v;
          }
        }
      }
      block_argmax(bz, bi, red_d, red_i, kRadixThreads);
      if (tid == 0) finish(bz, bi);
      return;
    }
  }

  // ---- the kept set is too large: tie bound by passes over the row, then the
  // sweep draws with the bounds ------------------------------------------------
  if (use_p && ystar >= tk) {
    // Group size: count pass on the exact key (every index in bin 0).
    pass(24, 0, false, true, ystar);
    if (tid < 64) {
      uint64_t c = hist[4 * tid] + hist[4 * tid + 1] + hist[4 * tid + 2] + hist[4 * tid + 3];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o);
      if (tid == 0) res_q[3] = c;
    }
    __syncthreads();
    const uint64_t group = res_q[3];
    __syncthreads();
    const uint64_t n_keep = keep_of(group);
    if (n_keep < group)
      istar = index_bound(n_keep, [&](int shift, uint32_t ipre) { pass(shift, ipre, false, true, ystar); });
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
  const Warp wp = make_warp(a.temperature);
  uint32_t tk = 0, ystar = 0, istar = 0;
  if (a.sel != nullptr) {
    const uint4 s = a.sel[row];
    if (s.w != 0) return;  // drawn by the select kernel
    tk = s.x;
    ystar = s.y;
    istar = s.z;
  }
  const uint32_t k0 = (uint32_t)a.seed, k1 = (uint32_t)(a.seed >> 32);
  double best = -__builtin_huge_val();
  int bi = -1;
  float lb = kNegInfF;   // wave-uniform lower bound of the range's maximum z
  float lbl = kNegInfF;  // this lane's share of it
  // ya = x * fl(1/T) is within 2^-8 |ya| + 2^-25 of y (the division rounded to
  // the logits dtype; y = x when T == 1); yh = ya + 2^-7 |ya| bounds y from
  // above, up to 2^-25.
  const float rT = wp.T != 1.f ? wp.rT : 1.f;
  // Every lane of a wave runs the same iterations (the bound is shared by
  // shuffles); a vector of NV entries is NV / 4 generator groups.
  constexpr int NV = 16 / sizeof(LT);
  row_sweep<LT, kSweepThreads, false, true>(x, lo, hi, wp, [&](int64_t v0, const float(&xv)[NV]) {
    bool upd = false;
#pragma unroll
    for (int gq = 0; gq < NV / 4; ++gq) {
      const int64_t g = v0 + 4 * gq;
      float yh[4];
      float ym = kNegInfF;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float ya = xv[4 * gq + e] * rT;
        float h = fmaf(fabsf(ya), 0x1p-7f, ya);  // NaN for x = -inf or NaN: such entries are screened exactly
        // f16: a quotient at or above 65520 rounds to +inf.
        if constexpr (__is_same(LT, _Float16)) h = h >= 65520.f ? __builtin_huge_valf() : h;
        yh[e] = h;
        ym = fmaxf(ym, h);
      }
      // G < kGumbelMax: a group whose largest y cannot reach the bound holds
      // no winner and needs no generator call.
      if (!(ym + kGumbelMax >= lb)) continue;
      const uint4 w4 = philox4x32((uint32_t)(g >> 2), (uint32_t)i, (uint32_t)t, 0u, k0, k1);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w = word_of(w4, e);
        // Screen: 1 - U <= -ln U, so 1 - U > e^(y - lb) gives
        // G = -ln(-ln U) < lb - y, i.e. z < lb: not the maximum.  Both sides
        // are scaled by 2^32: ~w (rounded to fp32, within 2^-24 of it) is at
        // most 2^32 (1 - U) = ~w + 1/2, and tq is at least 2^32 e^(y - lb)
        // (an exponent margin of 2^-9 covers y's 2^-25, the rounding of the
        // argument for every |yh - lb| where 2^x neither overflows nor
        // underflows, and the hardware 2^x).  NaN passes.
        const float tq = __builtin_amdgcn_exp2f(fmaf(yh[e] - lb, 0x1.715476p+0f, 32.f + 0x1p-9f));
        if ((float)(~w) > tq) continue;
        // The exact y and the keep test, then the fp32 estimate of z.
        const float yy = warp_yf<LT>(xv[4 * gq + e], wp);
        const uint32_t k = ykey(yy);
        if (!(yy > kNegInfF && k >= tk && (k > ystar || (k == ystar && (uint32_t)(g + e) >= istar)))) continue;
        const float zf = yy + gumbel_est(w);
        const float mg = kZMargin + fabsf(zf) * kZMarginRel;
        lbl = fmaxf(lbl, zf - mg);
        upd = true;
        if (zf + mg >= lb) {
          // Within the margin of the bound: the exact draw (entries of a
          // lane come in increasing index, so a tie keeps the first).
          const double z = (double)yy + gumbel(w);
          if (bi < 0 || z > best) {
            best = z;
            bi = (int)(g + e);
          }
        }
      }
    }
    if (__ballot(upd) != 0ull) {
      float wl = lbl;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) wl = fmaxf(wl, __shfl_xor(wl, o));
      lb = wl;
    }
  });
  __shared__ double sb[kSweepThreads / 64];
  __shared__ int si[kSweepThreads / 64];
  block_argmax(best, bi, sb, si, kSweepThreads);
  if (threadIdx.x == 0) {
    const uint64_t zb = __builtin_bit_cast(uint64_t, best);
    a.rstat[row * a.nchunk + c] =
        make_float4(__uint_as_float((uint32_t)zb), __uint_as_float((uint32_t)(zb >> 32)), __int_as_float(bi), 0.f);
  }
}

// The 16-byte vector of logits at v0 as loaded; entries at or past hi read
// as -inf.
template <typename LT>
__device__ __forceinline__ u32x4 load_words(const LT* x, int64_t v0, int64_t hi, bool aligned) {
  constexpr int N = 16 / sizeof(LT);
  if (aligned && v0 + N <= hi) return *reinterpret_cast<const u32x4*>(x + v0);
  uint32_t w[4];
  if constexpr (sizeof(LT) == 4) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = v0 + e < hi ? __builtin_bit_cast(uint32_t, x[v0 + e]) : (uint32_t)IntOrder<LT>::kNegInf;
  } else {
    constexpr uint32_t ninf = (uint32_t)IntOrder<LT>::kNegInf & 0xFFFFu;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t lo = v0 + 2 * e < hi ? (uint32_t)__builtin_bit_cast(uint16_t, x[v0 + 2 * e]) : ninf;
      const uint32_t up = v0 + 2 * e + 1 < hi ? (uint32_t)__builtin_bit_cast(uint16_t, x[v0 + 2 * e + 1]) : ninf;
      w[e] = lo | (up << 16);
    }
  }
  return u32x4{w[0], w[1], w[2], w[3]};
}

// row_sweep's order and loads over [lo, hi), handing f(v0, r) the vector's
// words as loaded instead of floats.
template <typename LT, int NT, typename F>
__device__ __forceinline__ void row_sweep_words(const LT* x, int64_t lo, int64_t hi, F&& f) {
  constexpr int N = 16 / sizeof(LT);
  constexpr int64_t kStep = (int64_t)2 * NT * N;
  constexpr int64_t kSpan = (int64_t)(NT + 64) * N;  // a wave's two vectors lie in [b0, b0 + kSpan)
  const bool aligned = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  const int lane = threadIdx.x & 63;
  int64_t b0 = lo + (int64_t)(threadIdx.x & ~63) * N;  // uniform over the wave
  if (aligned && b0 + kSpan <= hi) {
    const LT* p = x + b0 + (int64_t)lane * N;
    u32x4 ra = *reinterpret_cast<const u32x4*>(p), rb = *reinterpret_cast<const u32x4*>(p + NT * N);
    for (;;) {
      const bool more = b0 + kStep + kSpan <= hi;  // uniform over the wave
      u32x4 na, nb;
      if (more) {
        na = *reinterpret_cast<const u32x4*>(p + kStep);
        nb = *reinterpret_cast<const u32x4*>(p + kStep + NT * N);
      }
      f(b0 + (int64_t)lane * N, ra);
      f(b0 + (int64_t)lane * N + (int64_t)NT * N, rb);
      b0 += kStep;
      p += kStep;
      if (!more) break;
      ra = na;
      rb = nb;
    }
  }
  for (; b0 < hi; b0 += kStep) {
    const int64_t v0 = b0 + (int64_t)lane * N, v1 = v0 + (int64_t)NT * N;
    const u32x4 ra = load_words<LT>(x, v0, hi, aligned), rb = load_words<LT>(x, v1, hi, aligned);
    f(v0, ra);
    f(v1, rb);
  }
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Temperature alone: one workgroup per row, or up to 8 when the rows are
// few, each drawing over a run of the row's vocabulary ranges.
// Pass 1 (over the whole row, in every workgroup) takes signed integer
// extremes of the logits' bits (packed 16-bit ones for 16-bit logits): among
// non-negative bits the integer order is the float order, among negative
// bits the reverse, so the largest non-negative integer is the largest
// logit when there is one, else the smallest integer is.  Each extreme (each
// half of a packed one) of a thread keeps the vector where it last
// changed, so the row's largest logit comes with a vector that holds it; that
// entry's exact z (it is kept, as every finite entry is) bounds the row's
// maximum z from below (lb) from the start, for every wave.  Positive NaNs
// never stand for the maximum (a thread that met one offers only its
// negative side); any entry found is a valid bound.
// Pass 2 keeps a group of four only if one of its logits x has
// y(x) >= lb - kGumbelMax (as G < kGumbelMax), tested on the bits h against
// the smallest such logit xt (the warper is monotone): int(h) >= int(xt) for
// a non-negative xt, else uint(h) <= uint(xt), at the dtype's width; negative
// NaNs never pass.  The groups kept are queued per wave in LDS (index and
// raw words) and drawn 64 at a time, one per lane, with the sweep's screen,
// estimate and exact draw.  xt is recomputed
// when lb has risen by 4 (a lower xt only keeps more groups).
constexpr int kTempThreads = 512;

template <typename LT>
__global__ void __launch_bounds__(kTempThreads) __attribute__((amdgpu_waves_per_eu(4))) sample_temp_kernel(const AcceptArgs a) {
  using IO = IntOrder<LT>;
  constexpr bool k32 = sizeof(LT) == 4;
  constexpr int NV = 16 / sizeof(LT), kGV = NV / 4, kWv = kTempThreads / 64;
  constexpr int kQ = 64 * (kGV + 1);  // queue entries per wave
  const int64_t row = blockIdx.x;
  const int t = (int)(row / a.M), i = (int)(row % a.M);
  const LT* x = reinterpret_cast<const LT*>(a.logits) + (int64_t)t * a.l_st + (int64_t)i * a.l_sm;
  const int64_t V = a.V;
  const Warp wp = make_warp(a.temperature);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t k0 = (uint32_t)a.seed, k1 = (uint32_t)(a.seed >> 32);
  // This workgroup's vocabulary ranges [c0, c1) of the row's a.nchunk: the
  // row's gridDim.y workgroups take consecutive runs of G ranges.
  const int G = (a.nchunk + (int)gridDim.y - 1) / (int)gridDim.y;
  const int c0 = min((int)blockIdx.y * G, a.nchunk), c1 = min(c0 + G, a.nchunk);
  const int64_t lo = (int64_t)c0 * a.chunk, hi = min(V, (int64_t)c1 * a.chunk);
  __shared__ int64_t red_k[kWv];
  __shared__ int red_p[kWv];
  __shared__ float lb0_s;
  __shared__ uint4 qbuf[kWv][kQ];              // 16-bit: (index, words); 32-bit: the words
  __shared__ uint32_t qidx[kWv][k32 ? kQ : 1];  // 32-bit: the index
  __shared__ double sb[kWv];
  __shared__ int si[kWv];

  // ---- pass 1: the largest logit and a vector that holds it ------------------------
  // hm, hn: the thread's largest and smallest integer (of the bits), at the
  // vectors hp, hq.
  int hm, hn, hp, hq;
  if constexpr (k32) {
    int pmax = INT32_MIN, nmin = INT32_MAX, pp = -1, np = -1;
    row_sweep_words<LT, kTempThreads>(x, 0, V, [&](int64_t v0, const u32x4& r) {
      const uint32_t a0 = r[0], a1 = r[1], a2 = r[2], a3 = r[3];
      const int vmax = max(max((int)a0, (int)a1), max((int)a2, (int)a3));
      const int vmin = min(min((int)a0, (int)a1), min((int)a2, (int)a3));
      if (vmax > pmax) {
        pmax = vmax;
        pp = (int)v0;
      }
      if (vmin < nmin) {
        nmin = vmin;
        np = (int)v0;
      }
    });
    hm = pmax;
    hp = pp;
    hn = nmin;
    hq = np;
  } else {
    s16x2 pmax = {(short)-32768, (short)-32768}, nmin = {(short)32767, (short)32767};
    int px = -1, py = -1, nx = -1, ny = -1;
    row_sweep_words<LT, kTempThreads>(x, 0, V, [&](int64_t v0, const u32x4& r) {
      s16x2 s[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t rw = r[w];  // (a bit cast of the element itself reads element 0)
        s[w] = __builtin_bit_cast(s16x2, rw);
      }
      const s16x2 vmax = __builtin_elementwise_max(__builtin_elementwise_max(s[0], s[1]), __builtin_elementwise_max(s[2], s[3]));
      const s16x2 vmin = __builtin_elementwise_min(__builtin_elementwise_min(s[0], s[1]), __builtin_elementwise_min(s[2], s[3]));
      const s16x2 pn = __builtin_elementwise_max(pmax, vmax), nn = __builtin_elementwise_min(nmin, vmin);
      if (pn.x != pmax.x) px = (int)v0;
      if (pn.y != pmax.y) py = (int)v0;
      if (nn.x != nmin.x) nx = (int)v0;
      if (nn.y != nmin.y) ny = (int)v0;
      pmax = pn;
      nmin = nn;
    });
    hm = pmax.x >= pmax.y ? (int)pmax.x : (int)pmax.y;
    hp = pmax.x >= pmax.y ? px : py;
    hn = nmin.x <= nmin.y ? (int)nmin.x : (int)nmin.y;
    hq = nmin.x <= nmin.y ? nx : ny;
  }
  // The thread's candidate as one ordered key: 2^32 + bits for a
  // non-negative logit, -int(bits) for a negative one (-inf included), -1 for
  // none.
  int64_t key = -1;
  int kp = -1;
  if (hm >= 0 && hm <= IO::kInf) {
    key = (1ll << 32) + hm;
    kp = hp;
  } else if (hn <= IO::kNegInf) {
    key = -(int64_t)hn;
    kp = hq;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const int64_t ok = __shfl_xor(key, o);
    const int op = __shfl_xor(kp, o);
    if (ok > key || (ok == key && op < kp)) {
      key = ok;
      kp = op;
    }
  }
  if (lane == 0) {
    red_k[wv] = key;
    red_p[wv] = kp;
  }
  __syncthreads();
  double best = -__builtin_huge_val();
  int bi = -1;
  if (tid == 0) {
    int64_t gk = red_k[0];
    int gp = red_p[0];
    for (int w = 1; w < kWv; ++w)
      if (red_k[w] > gk || (red_k[w] == gk && red_p[w] < gp)) {
        gk = red_k[w];
        gp = red_p[w];
      }
    float lb0 = kNegInfF;
    int e = -1;  // an entry of vector gp with those bits
    if (gk >= 0 && gp >= 0) {
      uint32_t bits = gk >= (1ll << 32) ? (uint32_t)(gk - (1ll << 32)) : (uint32_t)(-gk);
      if constexpr (!k32) bits &= 0xFFFFu;
      for (int q = 0; q < NV && e < 0; ++q) {
        if (gp + q >= V) break;
        uint32_t b;
        if constexpr (k32)
          b = __builtin_bit_cast(uint32_t, x[gp + q]);
        else
          b = (uint32_t)__builtin_bit_cast(uint16_t, x[gp + q]);
        if (b == bits) e = q;
      }
    }
    if (e >= 0) {
      // Its exact z.
      const int64_t v = gp + e;
      const float yv = warp_y<LT>(x[v], wp);
      const double z = (double)yv + gumbel(draw_word(v, i, t, a.seed));
      best = z;
      bi = (int)v;
      // A float at or below z (z rounded to nearest is within half an ulp).
      lb0 = (float)z;
      if ((double)lb0 > z) lb0 = lb0 - fabsf(lb0) * 0x1p-23f - 0x1p-126f;
    }
    lb0_s = lb0;
  }
  __syncthreads();

  // ---- pass 2: the groups that can reach the bound, queued and drawn ---------------
  float lb = lb0_s, lbl = kNegInfF;
  // The screen (uniform over the wave): tneg and the operand tpk, uint(xt) + 1
  // or int(xt) - 1 (16-bit: in both halves), for the lb of lb_t.
  int tneg = 1;
  uint32_t tpk = 0;
  float lb_t = kNegInfF;
  auto set_threshold = [&]() {
    // At most lb - kGumbelMax: the two roundings are within 2^-23 |lb|.
    const float thr = (lb > kNegInfF && lb < -kNegInfF) ? (lb - kGumbelMax) - fabsf(lb) * 0x1p-21f : lb;
    const uint32_t xb = x_threshold_bits<LT>(thr, wp);
    const bool neg = (xb & (k32 ? 0x80000000u : 0x8000u)) != 0u;
    const uint32_t c = neg ? xb + 1u : xb - 1u;
    tneg = __builtin_amdgcn_readfirstlane(neg ? 1 : 0);
    tpk = __builtin_amdgcn_readfirstlane(k32 ? c : ((c & 0xFFFFu) | (c << 16)));
    lb_t = lb;
  };
  // 16-bit logits: a group is two words.
  auto screen = [&](uint32_t w0, uint32_t w1) -> bool {
    if (tneg) {
      const u16x2 m = __builtin_elementwise_min(__builtin_bit_cast(u16x2, w0), __builtin_bit_cast(u16x2, w1));
      return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(m, __builtin_bit_cast(u16x2, tpk))) != tpk;
    }
    const s16x2 m = __builtin_elementwise_max(__builtin_bit_cast(s16x2, w0), __builtin_bit_cast(s16x2, w1));
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(m, __builtin_bit_cast(s16x2, tpk))) != tpk;
  };
  auto group = [&](int64_t g, const float (&x4)[4], bool& upd) {
    const uint4 w4 = philox4x32((uint32_t)(g >> 2), (uint32_t)i, (uint32_t)t, 0u, k0, k1);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t w = word_of(w4, e);
      const float ya = x4[e] * wp.rT;
      float yh = fmaf(fabsf(ya), 0x1p-7f, ya);  // NaN for x = -inf or NaN: screened exactly
      if constexpr (__is_same(LT, _Float16)) yh = yh >= 65520.f ? __builtin_huge_valf() : yh;
      // The sweep kernel's screen: 1 - U <= -ln U (see there).
      const float tq = __builtin_amdgcn_exp2f(fmaf(yh - lb, 0x1.715476p+0f, 32.f + 0x1p-9f));
      if ((float)(~w) > tq) continue;
      const float yy = warp_yf<LT>(x4[e], wp);
      if (!(yy > kNegInfF)) continue;
      const float zf = yy + gumbel_est(w);
      const float mg = kZMargin + fabsf(zf) * kZMarginRel;
      lbl = fmaxf(lbl, zf - mg);
      upd = true;
      if (zf + mg >= lb) {
        const double z = (double)yy + gumbel(w);
        if (bi < 0 || z > best || (z == best && (int)(g + e) < bi)) {
          best = z;
          bi = (int)(g + e);
        }
      }
    }
  };
  uint4* qw = qbuf[wv];
  uint32_t* qi = qidx[wv];
  uint32_t qn = 0;  // queued groups (the same in every lane)
  auto drain = [&](uint32_t n) {  // groups [0, n), one per lane
    for (uint32_t s0 = 0; s0 < n; s0 += 64) {
      bool upd = false;
      if (s0 + (uint32_t)lane < n) {
        const uint4 it = qw[s0 + lane];
        if constexpr (k32) {
          const float x4[4] = {__uint_as_float(it.x), __uint_as_float(it.y), __uint_as_float(it.z),
                               __uint_as_float(it.w)};
          group((int64_t)qi[s0 + lane], x4, upd);
        } else {
          const float x4[4] = {raw_to_f<LT>(__builtin_bit_cast(LT, (uint16_t)(it.y & 0xFFFFu))),
                               raw_to_f<LT>(__builtin_bit_cast(LT, (uint16_t)(it.y >> 16))),
                               raw_to_f<LT>(__builtin_bit_cast(LT, (uint16_t)(it.z & 0xFFFFu))),
                               raw_to_f<LT>(__builtin_bit_cast(LT, (uint16_t)(it.z >> 16)))};
          group((int64_t)it.x, x4, upd);
        }
      }
      if (__ballot(upd) != 0ull) {
        float wl = lbl;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) wl = fmaxf(wl, __shfl_xor(wl, o));
        lb = fmaxf(lb, wl);
      }
    }
  };
  set_threshold();
  row_sweep_words<LT, kTempThreads>(x, lo, hi, [&](int64_t v0, const u32x4& r) {
    if constexpr (k32) {
      const uint32_t a0 = r[0], a1 = r[1], a2 = r[2], a3 = r[3];
      const bool pass = tneg ? min(min(a0, a1), min(a2, a3)) < tpk
                             : max(max((int)a0, (int)a1), max((int)a2, (int)a3)) > (int)tpk;
      const uint64_t bal = __ballot(pass);
      if (bal != 0ull) {
        if (pass) {
          const uint32_t q = qn + (uint32_t)__popcll(bal & ((1ull << lane) - 1ull));
          qw[q] = make_uint4(a0, a1, a2, a3);
          qi[q] = (uint32_t)v0;
        }
        qn += (uint32_t)__popcll(bal);
      }
    } else {
#pragma unroll
      for (int gq = 0; gq < kGV; ++gq) {
        const uint32_t w0 = r[2 * gq], w1 = r[2 * gq + 1];
        const bool pass = screen(w0, w1);
        const uint64_t bal = __ballot(pass);
        if (bal != 0ull) {
          if (pass)
            qw[qn + (uint32_t)__popcll(bal & ((1ull << lane) - 1ull))] = make_uint4((uint32_t)(v0 + 4 * gq), w0, w1, 0u);
          qn += (uint32_t)__popcll(bal);
        }
      }
    }
    if (qn >= 64u) {
      const uint32_t full = qn & ~63u, rest = qn - full;
      drain(full);
      // The rest (fewer than 64, at positions 64 and above) to the front.
      uint4 it = make_uint4(0u, 0u, 0u, 0u);
      uint32_t ix = 0;
      if ((uint32_t)lane < rest) {
        it = qw[full + lane];
        if constexpr (k32) ix = qi[full + lane];
      }
      if ((uint32_t)lane < rest) {
        qw[lane] = it;
        if constexpr (k32) qi[lane] = ix;
      }
      qn = rest;
      if (lb > lb_t + 4.f) set_threshold();
    }
  });
  drain(qn);
  block_argmax(best, bi, sb, si, kTempThreads);
  if (tid == 0) {
    // The draw over this workgroup's ranges (and the bound's entry, which
    // every workgroup of the row may report) as range c0's result.
    const uint64_t zb = __builtin_bit_cast(uint64_t, best);
    for (int c = c0; c < c1; ++c)
      a.rstat[row * a.nchunk + c] =
          c == c0 ? make_float4(__uint_as_float((uint32_t)zb), __uint_as_float((uint32_t)(zb >> 32)), __int_as_float(bi), 0.f)
                  : make_float4(0.f, 0.f, __int_as_float(-1), 0.f);
  }
}

template <typename LT>
hipError_t launch_sample_t(const AcceptArgs& a, hipStream_t s) {
  const unsigned rows = (unsigned)((int64_t)a.T * a.M);
  if (a.sel != nullptr) {
    // One workgroup per row: 1024 threads when the rows leave CUs idle, else
    // 512, so that each CU holds two rows and their serial phases overlap.
    if ((int64_t)rows >= 2 * (int64_t)(a.cus > 0 ? a.cus : 256))
      hipLaunchKernelGGL((sample_select_kernel<LT, 512>), dim3(rows), dim3(512), 0, s, a);
    else
      hipLaunchKernelGGL((sample_select_kernel<LT, 1024>), dim3(rows), dim3(1024), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(sample_radix_kernel<LT>, dim3(rows), dim3(kRadixThreads), 0, s, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (a.sel == nullptr) {  // temperature alone
    // One workgroup per row when the rows fill the CUs twice, else up to 8
    // per row, each on a run of the row's ranges (each one's pass 1 reads the
    // whole row).  f32 rows are twice the bytes: with fewer rows than CUs the
    // sweep kernel draws them.
    const int64_t cus = a.cus > 0 ? a.cus : 256;
    int64_t wpr = 2 * cus / (int64_t)rows;
    wpr = wpr < 1 ? 1 : (wpr > 8 ? 8 : wpr);
    wpr = wpr > a.nchunk ? a.nchunk : wpr;
    if (sizeof(LT) == 2 || (int64_t)rows >= cus) {
      const int64_t G = (a.nchunk + wpr - 1) / wpr;
      hipLaunchKernelGGL(sample_temp_kernel<LT>, dim3(rows, (unsigned)((a.nchunk + G - 1) / G)), dim3(kTempThreads), 0,
                         s, a);
      return hipGetLastError();
    }
  }
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
