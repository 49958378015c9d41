// dsv_merge.hip — kernel 3: log-sum-exp merge of split-K partials on gfx950.
//
// One wave64 per output row (batch, KV head, packed row).  Split s left a
// normalised bf16 row O_s and (m_s, l_s) = (running max in log2 units, sum of
// exponentials relative to it).  With M* = max_s m_s and
// w_s = l_s * 2^(m_s - M*), the merged row is O = sum_s w_s O_s / sum_s w_s and
// LSE = ln2 * (M* + log2 sum_s w_s).
// Lanes are split into (split group, 16-byte column chunk): every lane keeps
// its splits' (m, l) and 16-byte partial loads in flight together, then the
// split groups are reduced across lanes with DPP-class shuffles.
// This is the S-way generalisation of the reference's 2-way combine
// out = O_tree*(1-w) + O_prefix*w with w = sigmoid(lse_prefix - lse_tree)
// (runtime/tree_attention.py:535-539, llama_target_model.py:862-866), done in
// fp32 registers instead of three bf16 elementwise passes.  The kernel also
// produces the natural-log LSE and, when a prefix LSE is given, the
// reference's weight = sigmoid(prefix_lse - lse) for tree_attention_forward.

#include "dsv_internal.h"

namespace dsv {

namespace {

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kLn2 = 0.69314718055994530942f;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ void store_val(void* base, int dtype, int64_t off, float x) {
  if (dtype == 2) {
    reinterpret_cast<float*>(base)[off] = x;
  } else if (dtype == 0) {
    reinterpret_cast<__bf16*>(base)[off] = (__bf16)x;
  } else {
    reinterpret_cast<_Float16*>(base)[off] = (_Float16)x;
  }
}

// Lanes are (split group sg, 16-byte column chunk tc).  Splits are taken in
// chunks of SG * SPL: a lane loads the (m, l) pairs and the partial-row chunks
// of its SPL splits of the chunk at once (one memory round trip per chunk),
// then the chunk's weights are formed against the running maximum.
template <int D, int SPL>
__global__ void __launch_bounds__(256) lse_merge_kernel(const MergeArgs a) {
  constexpr int TPR = D / 8;        // 16-byte column chunks per row
  constexpr int SG = 64 / TPR;      // split groups per wave
  constexpr int CHUNK = SG * SPL;
  const int lane = threadIdx.x & 63;
  const int tc = lane % TPR, sg = lane / TPR;
  // Dispatch ids go round-robin over the 8 XCDs; remap so that XCD x merges
  // a contiguous eighth of the rows.  Kernel 1 hands out contiguous eighths of
  // its (batch, KV head, split) order the same way, so the rows of a (batch,
  // KV head) tend to be merged on the XCD whose L2 their partials went through
  // (exactly so for 8 KV heads and batch 1).
  const int nb = gridDim.x;
  const int bx = ((nb & 7) == 0) ? (blockIdx.x & 7) * (nb >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  // The row index is uniform over the wave and below 2^31 (the host checks):
  // its decomposition is 32-bit scalar arithmetic.
  const int row = __builtin_amdgcn_readfirstlane(bx * 4 + (threadIdx.x >> 6));
  const int64_t nrows = (int64_t)a.B * a.Hk * a.R;
  if (row >= nrows) return;
  const int q = row / a.R;
  const int r = row - q * a.R;
  const int b = q / a.Hk;
  const int kvh = q - b * a.Hk;

  float mrun = kNegInf;  // running maximum (log2 units), uniform over the wave
  float lsum = 0.f;      // this lane's share of sum_s w_s (per split group)
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  for (int s0 = 0; s0 < a.s_total; s0 += CHUNK) {
    float2 st[SPL];
    u32x4 raw[SPL];
#pragma unroll
    for (int i = 0; i < SPL; ++i) {
      const int s = s0 + sg + SG * i;
      if (s < a.s_total) {
        st[i] = a.ml[s * nrows + row];
        raw[i] = *reinterpret_cast<const u32x4*>(a.opart + (s * nrows + row) * D + tc * 8);
      } else {
        st[i] = make_float2(kNegInf, 0.f);
        raw[i] = u32x4{0, 0, 0, 0};
      }
    }
    float mc = kNegInf;
#pragma unroll
    for (int i = 0; i < SPL; ++i) mc = fmaxf(mc, st[i].x);
#pragma unroll
    for (int o = TPR; o < 64; o <<= 1) mc = fmaxf(mc, __shfl_xor(mc, o));
    const float mnew = fmaxf(mrun, mc);
    if (mnew == kNegInf) continue;  // nothing visible yet
    if (mnew != mrun) {
      const float al = (mrun == kNegInf) ? 0.f : __builtin_amdgcn_exp2f(mrun - mnew);
      lsum *= al;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] *= al;
      mrun = mnew;
    }
#pragma unroll
    for (int i = 0; i < SPL; ++i) {
      const float w = (st[i].x == kNegInf) ? 0.f : __builtin_amdgcn_exp2f(st[i].x - mrun) * st[i].y;
      lsum += w;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[2 * e] = fmaf(w, bf16_lo(raw[i][e]), acc[2 * e]);
        acc[2 * e + 1] = fmaf(w, bf16_hi(raw[i][e]), acc[2 * e + 1]);
      }
    }
  }
  // Sum over split groups (lanes with the same tc).
#pragma unroll
  for (int o = TPR; o < 64; o <<= 1) {
    lsum += __shfl_xor(lsum, o);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += __shfl_xor(acc[e], o);
  }
  const float L = lsum;
  const float invL = L > 0.f ? 1.f / L : 0.f;

  const int g = r / a.M;
  const int mi = r - g * a.M;
  const int m = a.row_perm ? min(max(a.row_perm[mi], 0), a.M - 1) : mi;
  const int h = kvh * a.G + g;
  if (sg == 0) {
    const int64_t obase = (int64_t)b * a.o_sb + (int64_t)m * a.o_sm + (int64_t)h * a.o_sh + tc * 8;
    if (a.out_dtype != 2 && ((reinterpret_cast<uintptr_t>(a.out) + 2 * obase) & 15) == 0) {
      // 16-bit output, 16-byte aligned: the lane's 8 values in one store.
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = acc[2 * e] * invL, x1 = acc[2 * e + 1] * invL;
        w[e] = a.out_dtype == 0
                   ? ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x0) | ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x1) << 16))
                   : ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x0) | ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x1) << 16));
      }
      *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(a.out) + obase) = u32x4{w[0], w[1], w[2], w[3]};
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) store_val(a.out, a.out_dtype, obase + e, acc[e] * invL);
    }
  }
  if (lane == 0) {
    const float lse = (L > 0.f) ? (mrun + __log2f(L)) * kLn2 : kNegInf;
    if (a.lse != nullptr) a.lse[(int64_t)b * a.l_sb + (int64_t)m * a.l_sm + (int64_t)h * a.l_sh] = lse;
    if (a.weight != nullptr) {
      const float pl = a.plse[(int64_t)b * a.p_sb + (int64_t)m * a.p_sm + (int64_t)h * a.p_sh];
      const float wgt = 1.f / (1.f + __expf(-(pl - lse)));
      store_val(a.weight, a.w_dtype, (int64_t)b * a.w_sb + (int64_t)m * a.w_sm + (int64_t)h * a.w_sh, wgt);
    }
  }
}

}  // namespace

hipError_t launch_merge(const MergeArgs& a, hipStream_t s) {
  const int64_t nrows = (int64_t)a.B * a.Hk * a.R;
  if (nrows <= 0) return hipSuccess;
  if (nrows >= ((int64_t)1 << 31) - 4) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((nrows + 3) / 4));
  if (a.D == 128)
    hipLaunchKernelGGL((lse_merge_kernel<128, 8>), grid, dim3(256), 0, s, a);
  else if (a.D == 64)
    hipLaunchKernelGGL((lse_merge_kernel<64, 4>), grid, dim3(256), 0, s, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace dsv
