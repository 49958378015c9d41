// dsv_merge.hip — kernel 3: log-sum-exp merge of split-K partials on gfx950.
//
// One wave64 per output row (batch, KV head, packed row).  Lane s holds the
// statistics (m_s, l_s) of split s; the wave computes M* = max_s m_s and
// L = sum_s 2^(m_s - M*) l_s with cross-lane reductions, turns each split
// into a coefficient c_s = 2^(m_s - M*) / L, then streams the partial rows
// (coalesced 256-byte reads per split) and accumulates O = sum_s c_s O_s.
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

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

__device__ __forceinline__ void store_val(void* base, int dtype, int64_t off, float x) {
  if (dtype == 2) {
    reinterpret_cast<float*>(base)[off] = x;
  } else if (dtype == 0) {
    reinterpret_cast<__bf16*>(base)[off] = (__bf16)x;
  } else {
    reinterpret_cast<_Float16*>(base)[off] = (_Float16)x;
  }
}

__global__ void __launch_bounds__(256) lse_merge_kernel(const MergeArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t nrows = (int64_t)a.B * a.Hk * a.R;
  if (row >= nrows) return;
  const int r = (int)(row % a.R);
  const int kvh = (int)((row / a.R) % a.Hk);
  const int b = (int)(row / ((int64_t)a.R * a.Hk));
  const int64_t split_stride = nrows;  // rows per split

  // Pass 1: global max over splits.
  float mloc = kNegInf;
  for (int s = lane; s < a.s_total; s += 64) mloc = fmaxf(mloc, a.ml[s * split_stride + row].x);
  const float mstar = wave_max(mloc);

  // Pass 2: total weight.
  float lloc = 0.f;
  if (mstar != kNegInf) {
    for (int s = lane; s < a.s_total; s += 64) {
      const float2 st = a.ml[s * split_stride + row];
      if (st.x != kNegInf) lloc += __builtin_amdgcn_exp2f(st.x - mstar) * st.y;
    }
  }
  const float L = wave_sum(lloc);
  const float invL = L > 0.f ? 1.f / L : 0.f;

  // Pass 3: weighted sum of partial rows; coefficients broadcast per split.
  constexpr int kMaxPer = 4;  // D <= 256
  float acc[kMaxPer];
#pragma unroll
  for (int i = 0; i < kMaxPer; ++i) acc[i] = 0.f;
  for (int s0 = 0; s0 < a.s_total; s0 += 64) {
    float c = 0.f;
    const int s = s0 + lane;
    if (s < a.s_total && mstar != kNegInf) {
      const float mx = a.ml[s * split_stride + row].x;
      if (mx != kNegInf) c = __builtin_amdgcn_exp2f(mx - mstar) * invL;
    }
    const int n = min(64, a.s_total - s0);
    for (int j = 0; j < n; ++j) {
      const float cj = __shfl(c, j);
      if (cj == 0.f) continue;
      const float* op = a.opart + ((int64_t)(s0 + j) * split_stride + row) * a.D;
#pragma unroll
      for (int i = 0; i < kMaxPer; ++i) {
        const int d = lane + 64 * i;
        if (d < a.D) acc[i] = fmaf(cj, op[d], acc[i]);
      }
    }
  }

  const int g = r / a.M;
  const int mi = r - g * a.M;
  const int m = a.row_perm ? min(max(a.row_perm[mi], 0), a.M - 1) : mi;
  const int h = kvh * a.G + g;
  const int64_t obase = (int64_t)b * a.o_sb + (int64_t)m * a.o_sm + (int64_t)h * a.o_sh;
#pragma unroll
  for (int i = 0; i < kMaxPer; ++i) {
    const int d = lane + 64 * i;
    if (d < a.D) store_val(a.out, a.out_dtype, obase + d, acc[i]);
  }
  if (lane == 0) {
    const float lse = (L > 0.f) ? (mstar + __log2f(L)) * kLn2 : kNegInf;
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
  hipLaunchKernelGGL(lse_merge_kernel, dim3((unsigned)((nrows + 3) / 4)), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace dsv
