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
//       The row maximum m; counts of d = m - y in a ladder of buckets (read
//       off d's bits); the narrowest head {d <= theta} (at most kCap
//       entries) that surely carries the top-p mass, or holds k entries, is
//       gathered into LDS and sorted.  top-k is the head's k-th key; top-p
//       takes the head's exact masses and bounds the rest of L by an fp32
//       sum: the cut is exact when it lands on the same entry for every L in
//       those bounds, inside the head.  The draw over the kept head entries is
//       the row's result.  Other rows (flat rows, a large k, an undecided
//       cut) are left to the radix kernel (status 2, with m).
//   sample_radix_kernel   one workgroup per row left open: 8-bit radix
//       selection over the order keys of y (count-weighted for top-k,
//       mass-weighted for top-p); the kept set (keys at or above both bounds)
//       is gathered into LDS, where the index bound in the cut's tie group and
//       the draw are taken when it fits; otherwise the bound comes from index
//       passes over the row and the sweep draws.
//   sample_sweep_kernel   one workgroup per (row, vocabulary range) of the
//       rows still open (all rows without top-p / top-k):
//       the Gumbel-max draw over the range's kept entries.  Against a
//       wave-shared lower bound lb of the range's maximum z, an entry whose
//       1 - U exceeds an upper bound of e^(y - lb) cannot reach lb (one 2^x
//       per entry from x * fl(1/T)); the few others take the exact warper,
//       the keep test and an fp32 estimate of z (within 2^-14 of it), which
//       leaves the exact double evaluation to the entries that can still win.
//   the walk of dsv_accept.hip combines the ranges' draws and walks.

#include "dsv_internal.h"

namespace dsv {

namespace {

constexpr int kRadixThreads = 1024;
constexpr int kSweepThreads = 256;
constexpr float kNegInfF = -__builtin_huge_valf();
constexpr int kCap = 4096;   // candidates the select kernel's fast path sorts in LDS
// Ladder of candidate thresholds m - y <= theta_j: the floats whose bits are
// (250 + j) << 22, i.e. 2^e and 1.5 * 2^e from 1/4 to 48.
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
// RAW = true the logits as loaded.
template <typename LT, int NT, bool WARP = true, bool RAW = false, typename F>
__device__ __forceinline__ void row_sweep(const LT* x, int64_t lo, int64_t hi, const Warp& T, F&& f) {
  constexpr int N = 16 / sizeof(LT);
  constexpr int64_t kStep = (int64_t)2 * NT * N;
  const bool aligned = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  const int lane = threadIdx.x & 63;
  int64_t b0 = lo + (int64_t)(threadIdx.x & ~63) * N;  // uniform over the wave
  if (b0 >= hi) return;
  u32x4 ra = fetch_vec<LT>(x, b0 + (int64_t)lane * N, hi, aligned);
  u32x4 rb = fetch_vec<LT>(x, b0 + (int64_t)lane * N + (int64_t)NT * N, hi, aligned);
  for (; b0 < hi; b0 += kStep) {
    const int64_t v0 = b0 + (int64_t)lane * N, v1 = v0 + (int64_t)NT * N;
    u32x4 na = u32x4{0, 0, 0, 0}, nb = u32x4{0, 0, 0, 0};
    if (b0 + kStep < hi) {
      na = fetch_vec<LT>(x, v0 + kStep, hi, aligned);
      nb = fetch_vec<LT>(x, v1 + kStep, hi, aligned);
    }
    float ya[N], yb[N];
    unpack_vec<LT>(x, v0, hi, aligned, ra, ya);
    unpack_vec<LT>(x, v1, hi, aligned, rb, yb);
    if constexpr (!RAW) {
      finish_y<LT, WARP>(ya, T);
      finish_y<LT, WARP>(yb, T);
    }
    f(v0, ya);
    f(v1, yb);
    ra = na;
    rb = nb;
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

template <typename LT, int NT>
__global__ void __launch_bounds__(NT) sample_select_kernel(const AcceptArgs a) {
  static_assert(kCap % NT == 0, "candidates split evenly over the threads");
  const int64_t row = blockIdx.x;
  const int t = (int)(row / a.M), i = (int)(row % a.M);
  const LT* x = reinterpret_cast<const LT*>(a.logits) + (int64_t)t * a.l_st + (int64_t)i * a.l_sm;
  const int V = (int)a.V;
  const int tid = threadIdx.x;
  constexpr int ND = key_digits<LT>();
  const Warp wp = make_warp(a.temperature);

  __shared__ float red_f[NT / 64];

  // Row maximum of y: the warper is monotone, so it is the warped maximum
  // logit (xm).
  float m = kNegInfF;
  constexpr int NV = 16 / sizeof(LT);
  row_sweep<LT, NT, false>(x, 0, V, wp, [&](int64_t, const float(&y)[NV]) {
#pragma unroll
    for (int e = 0; e < NV; ++e) m = fmaxf(m, y[e]);
  });
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if ((tid & 63) == 0) red_f[tid >> 6] = m;
  __syncthreads();
  if (tid == 0) {
    float mm = red_f[0];
    for (int w = 1; w < NT / 64; ++w) mm = fmaxf(mm, red_f[w]);
    red_f[0] = mm;
  }
  __syncthreads();
  const float xm = red_f[0];
  m = xm > kNegInfF ? warp_y<LT>(f_to_raw<LT>(xm), wp) : kNegInfF;

  int S = 63;
  for (int vv = V; vv > 0; vv >>= 1) --S;  // 63 - bitlen(V)

  const int lane = tid & 63, wv = tid >> 6;
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

  // ---- fast path --------------------------------------------------------------
  __shared__ uint64_t cand[kCap];  // (key << 32) | index, sorted descending
  __shared__ uint32_t cnt_th[kNTheta];
  __shared__ uint32_t ncand, nk_lo, nk_hi;
  __shared__ int jsel[2];
  __shared__ uint32_t n_eq;
  __shared__ float red_l[NT / 64];
  __shared__ uint64_t red_q[NT / 64];
  __shared__ double red_d[NT / 64];
  __shared__ int red_i[NT / 64];

  if (tid < kNTheta) cnt_th[tid] = 0;
  if (tid == 0) {
    ncand = 0;
    nk_lo = 0;
    nk_hi = 0;
    n_eq = 0;
  }
  __syncthreads();
  // Counts of d = (xm - x) / T (fp32, equal to m - y when T == 1; close to
  // it otherwise, the gather below checks the count) per bucket b: d <= theta_0 (b = 0),
  // theta_(b-1) < d <= theta_b (b = 1..15), read off d's bits (exponent and
  // first mantissa bit); a lane keeps them as 8-bit fields of two words (at
  // most 16 * 8 entries between flushes).
  {
    uint32_t cth[kNTheta];
#pragma unroll
    for (int j = 0; j < kNTheta; ++j) cth[j] = 0;
    uint64_t pk0 = 0, pk1 = 0;
    int calls = 0;
    float lsum = 0.f;  // top-p: sum of e^-d (fp32), for the choice of the head
    uint32_t eq = 0;   // entries at the maximum (d == 0, mass 1 each)
    auto flush = [&]() {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        cth[j] += (uint32_t)(pk0 >> (8 * j)) & 0xFFu;
        cth[j + 8] += (uint32_t)(pk1 >> (8 * j)) & 0xFFu;
      }
      pk0 = 0;
      pk1 = 0;
    };
    row_sweep<LT, NT, false>(x, 0, V, wp, [&](int64_t, const float(&y)[NV]) {
#pragma unroll
      for (int e = 0; e < NV; ++e) {
        const float d = (xm - y[e]) * wp.rT;
        const int b = min(max((((int)__float_as_uint(d) - 1) >> 22) - 249, 0), kNTheta);
        const uint64_t inc = 1ull << (8 * (b & 7));
        pk0 += b < 8 ? inc : 0ull;
        pk1 += (b >= 8 && b < kNTheta) ? inc : 0ull;
        if (use_p) {
          lsum += __builtin_amdgcn_exp2f(d * -1.44269504088896341f);
          eq += d == 0.f ? 1u : 0u;
        }
      }
      if (++calls == 16) {
        flush();
        calls = 0;
      }
    });
    flush();
    // Cumulative: cth[j] = #{d <= theta_j}; then the block's sums.
#pragma unroll
    for (int j = 1; j < kNTheta; ++j) cth[j] += cth[j - 1];
#pragma unroll
    for (int j = 0; j < kNTheta; ++j) {
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) cth[j] += __shfl_xor(cth[j], o);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      lsum += __shfl_xor(lsum, o);
      eq += __shfl_xor(eq, o);
    }
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < kNTheta; ++j) atomicAdd(&cnt_th[j], cth[j]);
      atomicAdd(&n_eq, eq);
      red_l[wv] = lsum;
    }
  }
  __syncthreads();
  if (tid == 0) {
    // top-k alone: the narrowest head holding k.  top-p: first the narrowest
    // head whose mass surely reaches top_p of the estimated total (entries at
    // the maximum count 1, the others e^-theta of their bucket's bound), then
    // the widest head that fits.
    int j0 = -1, j1 = -1;
    if (use_p) {
      float L = 0.f;
      for (int w = 0; w < NT / 64; ++w) L += red_l[w];
      const float need = (float)a.top_p_q * 0x1p-32f * L * (1.f + 0x1p-8f);
      float head = (float)n_eq + (float)(cnt_th[0] - n_eq) * __expf(-kTheta[0]);
      for (int j = 0; j < kNTheta && cnt_th[j] <= (uint32_t)kCap; ++j) {
        if (j > 0) head += (float)(cnt_th[j] - cnt_th[j - 1]) * __expf(-kTheta[j]);
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
    jsel[0] = j0;
    jsel[1] = j1;
  }
  __syncthreads();
  for (int att = 0; att < 2 && jsel[att] >= 0; ++att) {
    if (att > 0) {
      if (tid == 0) {
        ncand = 0;
        nk_lo = 0;
        nk_hi = 0;
      }
      __syncthreads();
    }
    const float ts = kTheta[jsel[att]];
    // Gather the candidates; sum the fp32 masses of the others.
    float tail = 0.f;
    row_sweep<LT, NT>(x, 0, V, wp, [&](int64_t v0, const float(&y)[NV]) {
      bool any = false;
#pragma unroll
      for (int e = 0; e < NV; ++e) {
        const bool c = m - y[e] <= ts;  // a head of the order (monotone in y)
        any |= c;
        if (use_p && !c) tail += __builtin_amdgcn_exp2f((y[e] - m) * 1.44269504088896341f);
      }
      if (__ballot(any) == 0ull) return;
#pragma unroll
      for (int e = 0; e < NV; ++e) {
        const bool c = m - y[e] <= ts;
        const uint64_t bal = __ballot(c);
        if (bal != 0ull) {
          uint32_t base = 0;
          if (lane == 0) base = atomicAdd(&ncand, (uint32_t)__popcll(bal));
          base = __shfl(base, 0);
          if (c) {
            const uint32_t slot = base + (uint32_t)__popcll(bal & ((1ull << lane) - 1ull));
            if (slot < (uint32_t)kCap) cand[slot] = ((uint64_t)ykey(y[e]) << 32) | (uint32_t)(v0 + e);
          }
        }
      }
    });
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) tail += __shfl_xor(tail, o);
    if (lane == 0) red_f[wv] = tail;
    __syncthreads();
    const int n = min((int)ncand, kCap);
    // The counts (of the unwarped logits when T != 1) chose the threshold;
    // the gathered count decides whether the head fits and holds k entries.
    const bool fits = (int)ncand <= kCap && (use_p || (int64_t)ncand >= kk);
    float tail_all = 0.f;
    for (int w = 0; w < NT / 64; ++w) tail_all += red_f[w];
    // Bitonic sort, descending, padded with zero keys to a power of two.
    int npad = 2;
    while (npad < n) npad <<= 1;
    for (int q = n + tid; q < npad; q += NT) cand[q] = 0ull;
    __syncthreads();
    for (int k2 = 2; k2 <= npad; k2 <<= 1)
      for (int j2 = k2 >> 1; j2 > 0; j2 >>= 1) {
        for (int q = tid; q < npad; q += NT) {
          const int l = q ^ j2;
          if (l > q) {
            const uint64_t u = cand[q], w = cand[l];
            if (((q & k2) == 0) ? (u < w) : (u > w)) {
              cand[q] = w;
              cand[l] = u;
            }
          }
        }
        __syncthreads();
      }
    // top-k: the k-th key when the candidates hold k (else every candidate
    // passes top-k, and the cut comes from top-p inside the candidates).
    const uint32_t tk = (kk > 0 && n >= kk) ? (uint32_t)(cand[kk - 1] >> 32) : 0u;
    int nkeep = n;
    bool ok = fits;
    if (use_p && ok) {
      // Exact masses along the order (thread tid holds entries EPT * tid ..
      // + EPT - 1) and their exclusive prefix sums.
      constexpr int EPT = kCap / NT;
      uint64_t qv[EPT], tot = 0;
#pragma unroll
      for (int u = 0; u < EPT; ++u) {
        const int e = EPT * tid + u;
        qv[u] = e < n ? fixed_mass(key_to_y((uint32_t)(cand[e] >> 32)), m, S) : 0ull;
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
      for (int w = 0; w < NT / 64; ++w) {
        if (w < wv) wbase += red_q[w];
        H += red_q[w];
      }
      // L = H + (masses outside the candidates), bounded from the fp32 sum.
      const double tr = (double)tail_all * __builtin_ldexp(1.0, S);
      const double tlo = __builtin_fmax(0.0, tr * (1.0 - 0x1p-12) - (double)V);
      const double thi = __builtin_fmin(tr * (1.0 + 0x1p-12) + (double)V + 1.0, 0x1p62);
      const uint64_t tq_lo = tq_of(a.top_p_q, H + (uint64_t)__builtin_floor(tlo));
      const uint64_t tq_hi = tq_of(a.top_p_q, H + (uint64_t)__builtin_ceil(thi));
      uint32_t cl = 0, ch = 0;
      uint64_t above = wbase + incl - tot;
#pragma unroll
      for (int u = 0; u < EPT; ++u) {
        if (EPT * tid + u < n) {
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
      ok = H >= tq_hi && nk_lo == nk_hi;
      nkeep = (int)nk_hi;
    }
    if (ok) {
      double bz = -__builtin_huge_val();
      int bi = -1;
      for (int q = tid; q < n; q += NT) {
        const uint64_t cv = cand[q];
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
