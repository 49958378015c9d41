// dsv_append.hip — tree K/V append with RoPE into the cache, on gfx950.
//
// The tree tokens' projected keys and values enter the cache at logical
// tokens [start, start + M): keys rotated by RoPE, values as they are; the
// queries can be rotated in the same launch.  RoPE follows the reference's
// op sequence in the model dtype (llama_target_model.py:452-473 and
// :408-427, applied at :768-783): out = x * cos + rotate_half(x) * sin with
// rotate_half(x) = cat(-x[D/2:], x[:D/2]), each product and the sum rounded
// to the 16-bit dtype (round to nearest even), as torch's elementwise ops on
// bf16/f16 tensors do.  The cache is a page pool half [P, Hk, page, D] behind
// a page table, or a dense [Hk, S, D] cache (KVCache.cat of
// runtime/cache_state.py:52-66 and the per-token PagedKVCache.write_kv of
// core/kv_cache/paged_kv.py:168-223 in the reference).
//
// One thread per pair of 16-byte chunks (8 elements each) D/2 apart in a
// token row: it loads both chunks (each is the other's rotate_half partner)
// and the token's cos/sin chunks before it stores either, so a row rotated
// in place (q_out == q) never reads a chunk another thread has written.

#include "dsv_internal.h"

namespace dsv {

namespace {

template <bool F16>
__device__ __forceinline__ float h2f(uint16_t h) {
  if constexpr (F16) return (float)__builtin_bit_cast(_Float16, h);
  return __uint_as_float((uint32_t)h << 16);
}
template <bool F16>
__device__ __forceinline__ uint16_t f2h(float x) {
  if constexpr (F16) return __builtin_bit_cast(uint16_t, (_Float16)x);
  return __builtin_bit_cast(uint16_t, (__bf16)x);
}

// One 8-element chunk of x * cos + rotate_half(x) * sin, with the dtype's
// rounding after each product and after the sum.
template <bool F16>
__device__ __forceinline__ u32x4 rope8(u32x4 x, u32x4 part, u32x4 c, u32x4 s, bool first_half) {
  // No contraction: a product rounded to the dtype must not fuse into the
  // sum (an FMA through the float widening would skip that rounding).
#pragma clang fp contract(off)
  u32x4 out;
  // rotate_half: -x[e + D/2] for e < D/2, x[e - D/2] above; the negation
  // flips the 16-bit sign bits (exact, like negating the widened value).
  if (first_half) part ^= u32x4{0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t o = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float xv = h2f<F16>((uint16_t)(x[w] >> (16 * h)));
      const float pv = h2f<F16>((uint16_t)(part[w] >> (16 * h)));
      const float cv = h2f<F16>((uint16_t)(c[w] >> (16 * h))), sv = h2f<F16>((uint16_t)(s[w] >> (16 * h)));
      const float a = h2f<F16>(f2h<F16>(xv * cv));
      const float b = h2f<F16>(f2h<F16>(pv * sv));
      o |= (uint32_t)f2h<F16>(a + b) << (16 * h);
    }
    out[w] = o;
  }
  return out;
}

template <bool F16>
__global__ void __launch_bounds__(256) kv_append_kernel(const AppendArgs a) {
  const int half = a.D / 16;  // chunk pairs per row
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  // Rows: [0, M*Hk) keys, [M*Hk, 2*M*Hk) values, then M*H query rows.
  const int64_t nkv = (int64_t)a.M * a.Hk;
  const int64_t rows = 2 * nkv + (a.q != nullptr ? (int64_t)a.M * a.H : 0);
  if (idx >= rows * half) return;
  const int64_t row = idx / half;
  const int c0 = (int)(idx - row * half), c1 = c0 + half;

  int kind, i, h;  // 0 key, 1 value, 2 query; token i, head h
  if (row < nkv) {
    kind = 0;
    i = (int)(row / a.Hk);
    h = (int)(row % a.Hk);
  } else if (row < 2 * nkv) {
    kind = 1;
    i = (int)((row - nkv) / a.Hk);
    h = (int)((row - nkv) % a.Hk);
  } else {
    kind = 2;
    i = (int)((row - 2 * nkv) / a.H);
    h = (int)((row - 2 * nkv) % a.H);
  }
  const uint16_t* src = kind == 0 ? a.k : (kind == 1 ? a.v : a.q);
  const int64_t s_m = kind == 0 ? a.k_sm : (kind == 1 ? a.v_sm : a.q_sm);
  const int64_t s_h = kind == 0 ? a.k_sh : (kind == 1 ? a.v_sh : a.q_sh);
  const uint16_t* xr = src + i * s_m + h * s_h;
  u32x4 x0 = *reinterpret_cast<const u32x4*>(xr + c0 * 8);
  u32x4 x1 = *reinterpret_cast<const u32x4*>(xr + c1 * 8);
  if (kind != 1 && a.cos != nullptr) {
    const uint16_t* cr = a.cos + i * a.cs_m;
    const uint16_t* sr = a.sin + i * a.sn_m;
    const u32x4 cs0 = *reinterpret_cast<const u32x4*>(cr + c0 * 8), cs1 = *reinterpret_cast<const u32x4*>(cr + c1 * 8);
    const u32x4 sn0 = *reinterpret_cast<const u32x4*>(sr + c0 * 8), sn1 = *reinterpret_cast<const u32x4*>(sr + c1 * 8);
    const u32x4 y0 = rope8<F16>(x0, x1, cs0, sn0, true);
    const u32x4 y1 = rope8<F16>(x1, x0, cs1, sn1, false);
    x0 = y0;
    x1 = y1;
  }
  uint16_t* dst;
  if (kind == 2) {
    dst = a.q_out + i * a.qo_sm + h * a.qo_sh;
  } else {
    uint16_t* base = kind == 0 ? a.k_dst : a.v_dst;
    const int64_t t = a.start + i;
    if (a.pt != nullptr) {
      int64_t pg = a.pt_i64 ? reinterpret_cast<const int64_t*>(a.pt)[t >> a.ps_shift]
                            : (int64_t) reinterpret_cast<const int32_t*>(a.pt)[t >> a.ps_shift];
      pg = pg < 0 ? 0 : (pg >= a.n_phys ? a.n_phys - 1 : pg);
      const int64_t sp = kind == 0 ? a.kd_sp : a.vd_sp;
      dst = base + pg * sp + h * (kind == 0 ? a.kd_sh : a.vd_sh) + (t & ((1ll << a.ps_shift) - 1)) * (kind == 0 ? a.kd_st : a.vd_st);
    } else {
      dst = base + h * (kind == 0 ? a.kd_sh : a.vd_sh) + t * (kind == 0 ? a.kd_st : a.vd_st);
    }
  }
  *reinterpret_cast<u32x4*>(dst + c0 * 8) = x0;
  *reinterpret_cast<u32x4*>(dst + c1 * 8) = x1;
}

}  // namespace

hipError_t launch_append(const AppendArgs& a, hipStream_t s) {
  const int64_t rows = 2 * (int64_t)a.M * a.Hk + (a.q != nullptr ? (int64_t)a.M * a.H : 0);
  const int64_t n = rows * (a.D / 16);
  if (n <= 0) return hipSuccess;
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  if (a.f16)
    hipLaunchKernelGGL(kv_append_kernel<true>, grid, block, 0, s, a);
  else
    hipLaunchKernelGGL(kv_append_kernel<false>, grid, block, 0, s, a);
  return hipGetLastError();
}

}  // namespace dsv
