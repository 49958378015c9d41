// dsv_lmhead.hip — lm_head fused with the acceptance statistics, on gfx950.
//
// The target's logits for the tree nodes are lm_head(hidden) = hidden . W^T
// ([R, Dm] x [V, Dm]^T, bf16 in, fp32 accumulate, bf16 out: the reference's
// self.base_model.lm_head, draft/diffspec_model.py:229-231, whose [M, V]
// output verify_new reduces with argmax, draft/tree_verification.py:100-102).
// Here the logits never reach HBM: each workgroup computes a 256-row slice
// of the vocabulary for all (up to 64) hidden rows, rounds every logit to
// bf16 exactly as the reference's bf16 logits are, and reduces its slice to
// the acceptance statistics of kernel 4 (argmax with the lowest index on
// ties; softmax (m, l, s) for typical acceptance) per hidden row.  A combine
// kernel and the tree walk of kernel 4 follow.
//
// The operation streams W once (V * Dm * 2 bytes, 1.05 GB for Llama-3.1-8B)
// and is HBM-bound: at 64 rows it needs 64 flop per byte, a fifth of the
// MFMA ridge.  Layout per workgroup (4 waves):
//   * wave w owns vocabulary rows [64w, 64w + 64) of the slice: two 32-row
//     MFMA blocks (A operand, straight from HBM into registers, two steps of
//     64 elements of Dm in flight ahead of the MFMAs);
//   * the hidden rows (B operand, 64 rows x 64 elements per step) are staged
//     once per workgroup through a double-buffered LDS tile;
//   * v_mfma_f32_32x32x16_bf16, 16 per wave per step.  MFMA sub-step j of a
//     step covers elements [16j, 16j + 16) of the step's 64: lanes 0-31 hold
//     the first 8, lanes 32-63 the next 8, the same on A and B, so one load
//     instruction reads 32 contiguous bytes of each of 32 W rows;
//   * workgroups start their sweep over Dm at different steps (a rotation),
//     which spreads their concurrent W reads over the memory channels.
// Hidden rows beyond R are zero; vocabulary rows beyond V are clamped loads
// whose results are dropped.

#include "dsv_internal.h"
#include "dsv_stats.h"

namespace dsv {

namespace {

constexpr int kWaves = kLmThreads / 64;
constexpr int kKB = 2 * kLmK;                        // bytes of one row per step
constexpr int kHStride = kKB + 16;                   // LDS step tile: bytes per hidden row
constexpr int kTStride = 2 * kLmVocab + 16;          // LDS logits tile: bytes per hidden row
constexpr int kHBytes = kLmRows * kHStride;          // one step tile
constexpr int kSmem = (2 * kHBytes > kLmRows * kTStride) ? 2 * kHBytes : kLmRows * kTStride;
constexpr int kHChunks = kKB / 16 / (kLmThreads / kLmRows);  // 16-byte chunks a thread stages per step
constexpr int kQ = kLmVocab / 4;                     // vocabulary rows per statistics thread
constexpr float kNegInfL = -__builtin_huge_valf();
constexpr float kLog2eL = 1.4426950408889634074f;
static_assert(kLmThreads == 4 * kLmRows, "four statistics threads per hidden row");
static_assert(kLmVocab == kWaves * 32 * kLmRB, "vocabulary rows per workgroup");
static_assert(kQ % 8 == 0, "statistics read 16-byte chunks");

template <int V>
struct IC {
  static constexpr int value = V;
};

__device__ __forceinline__ f32x16 mfma_bf16(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

__device__ __forceinline__ uint32_t bf16_rne(float x) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x);
}

template <bool TYPICAL>
__global__ void __launch_bounds__(kLmThreads, 2) lmhead_stats_kernel(const LmArgs a) {
  constexpr int RB = kLmRB, KS = kLmKS;
  __shared__ __align__(16) uint8_t smem[kSmem];
  uint8_t* const hb0 = smem;
  uint8_t* const hb1 = smem + kHBytes;

  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, lj = lane & 31, lg = lane >> 5;
  const int blk = blockIdx.x;
  const int64_t v0 = (int64_t)blk * kLmVocab;
  const int r0 = blockIdx.y * kLmRows;
  const int S = a.Dm / kLmK;

  // This lane's W rows (clamped into the vocabulary).  MFMA sub-step j of a
  // step covers elements [16j, 16j + 16): lanes 0-31 the first 8, lanes
  // 32-63 the next 8 (the operand layout of v_mfma_f32_32x32x16), so a load
  // instruction reads 32 contiguous bytes of each of 32 rows.
  const uint16_t* wrow[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    int64_t v = v0 + (wid * RB + rb) * 32 + lj;
    v = v < a.V ? v : a.V - 1;
    wrow[rb] = a.w + v * a.ldw + lg * 8;
  }
  // Hidden-row staging: thread -> (row hr, part hc) of a step.
  const int hr = tid >> 2, hc = tid & 3;
  const bool hvalid = r0 + hr < a.R;
  const uint16_t* hrow = a.h + (int64_t)min(r0 + hr, a.R - 1) * a.ldh + hc * (kLmK / 4);

  u32x4 wb[3][RB][KS];
  u32x4 hreg[kHChunks];
  f32x16 acc[RB][2];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) acc[rb][cb] = f32x16{};

  // Workgroups start the reduction at different steps (the sum is taken in a
  // rotated order): at any moment they read different columns of W, whose
  // rows are 2*Dm bytes apart, so the reads spread over the memory channels
  // instead of all landing on the same address bits.
  const int rot = (int)(((int64_t)blk * 7) % S);
  auto col = [&](int s) -> int64_t {
    int x = min(s, S - 1) + rot;
    if (x >= S) x -= S;
    return (int64_t)x * kLmK;
  };
  // Loads past the last step re-read the last one (an L2 hit), so every step
  // issues the same loads and the compiler's wait counts stay exact.
  auto load_w = [&](auto buf_c, int s) {
    constexpr int b = decltype(buf_c)::value;
    const int64_t off = col(s);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int j = 0; j < KS; ++j) wb[b][rb][j] = *reinterpret_cast<const u32x4*>(wrow[rb] + off + 16 * j);
  };
  auto load_h = [&](int s) {
    const int64_t off = col(s);
#pragma unroll
    for (int c = 0; c < kHChunks; ++c) hreg[c] = *reinterpret_cast<const u32x4*>(hrow + off + 8 * c);
  };
  // Rows beyond R stay zero in both buffers (written once below).
  auto store_h = [&](int s) {
    uint8_t* dst = ((s & 1) ? hb1 : hb0) + hr * kHStride + hc * (kKB / 4);
    if (hvalid) {
#pragma unroll
      for (int c = 0; c < kHChunks; ++c) *reinterpret_cast<u32x4*>(dst + 16 * c) = hreg[c];
    }
  };

  // Step s: B operands of h(s) from LDS, loads of h(s+1) and W(s+2) issued,
  // MFMAs on W(s), h(s+1) into the other LDS buffer, one barrier.
  auto step = [&](auto buf_c, int s) {
    constexpr int b = decltype(buf_c)::value;
    const uint8_t* hb = (s & 1) ? hb1 : hb0;
    u32x4 bf[2][KS];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int j = 0; j < KS; ++j)
        bf[cb][j] = *reinterpret_cast<const u32x4*>(hb + (cb * 32 + lj) * kHStride + lg * 16 + 32 * j);
    load_h(s + 1);
    load_w(IC<(b + 2) % 3>{}, s + 2);
#pragma unroll
    for (int j = 0; j < KS; ++j)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) acc[rb][cb] = mfma_bf16(wb[b][rb][j], bf[cb][j], acc[rb][cb]);
    // The wait for h(s+1) (and the W(s+1) loads issued before it) stays
    // behind the MFMAs.
    __builtin_amdgcn_sched_barrier(0);
    store_h(s + 1);
    __syncthreads();
  };

  load_h(0);
  load_w(IC<0>{}, 0);
  load_w(IC<1>{}, 1);
  if (!hvalid) {
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      uint8_t* dst = (x ? hb1 : hb0) + hr * kHStride + hc * (kKB / 4);
#pragma unroll
      for (int c = 0; c < kHChunks; ++c) *reinterpret_cast<u32x4*>(dst + 16 * c) = z;
    }
  }
  store_h(0);
  __syncthreads();
  // Three steps per iteration (one per W register buffer), no conditions in
  // the body; the last S % 3 steps follow.
  int s = 0;
  for (; s + 3 <= S; s += 3) {
    step(IC<0>{}, s);
    step(IC<1>{}, s + 1);
    step(IC<2>{}, s + 2);
  }
  if (s < S) step(IC<0>{}, s);
  if (s + 1 < S) step(IC<1>{}, s + 1);

  // ---- logits tile in LDS: [hidden row][vocab] bf16 (RNE, as the reference's
  // bf16 logits) ---------------------------------------------------------------------
  // Accumulator value e of block (rb, cb) holds vocab row
  // 32*(wid*RB + rb) + 8*(e/4) + 4*lg + e%4 and hidden row cb*32 + lj.
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const f32x16 x = acc[rb][cb];
        const u32x2 val = {bf16_rne(x[4 * q4]) | (bf16_rne(x[4 * q4 + 1]) << 16),
                           bf16_rne(x[4 * q4 + 2]) | (bf16_rne(x[4 * q4 + 3]) << 16)};
        const int vv = (wid * RB + rb) * 32 + 8 * q4 + 4 * lg;
        *reinterpret_cast<u32x2*>(smem + (cb * 32 + lj) * kTStride + vv * 2) = val;
      }
  __syncthreads();

  // ---- statistics: thread (hidden row j, quarter q) over kQ vocab rows ----------
  const int j = tid >> 2, q = tid & 3;
  const int row = r0 + j;
  const int64_t vq = v0 + q * kQ;
  const uint8_t* tr = smem + j * kTStride + q * (2 * kQ);
  ArgMax best{kNegInfL, 0x7fffffff};
  bool have = false;
  Soft sm{kNegInfL, 0.f, 0.f};
  const float zs = a.inv_temp * kLog2eL;
  float xs[kQ];
#pragma unroll
  for (int c = 0; c < kQ / 8; ++c) {
    const u32x4 w4 = *reinterpret_cast<const u32x4*>(tr + 16 * c);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xs[8 * c + 2 * e] = __uint_as_float(w4[e] << 16);
      xs[8 * c + 2 * e + 1] = __uint_as_float(w4[e] & 0xffff0000u);
    }
  }
  const int nv = (int)min<int64_t>(kQ, a.V - vq);  // valid vocab rows of this quarter (may be <= 0)
  float vmax = kNegInfL;
#pragma unroll
  for (int e = 0; e < kQ; ++e) {
    if (e < nv) {
      if (!have || am_better(xs[e], (int)(vq + e), best.v, best.i)) {
        best.v = xs[e];
        best.i = (int)(vq + e);
        have = true;
      }
      if constexpr (TYPICAL) vmax = fmaxf(vmax, xs[e] * zs);
    }
  }
  if constexpr (TYPICAL) {
    if (vmax != kNegInfL) {
      sm.m = vmax;
#pragma unroll
      for (int e = 0; e < kQ; ++e) {
        if (e < nv) {
          const float p = __builtin_amdgcn_exp2f(fmaf(xs[e], zs, -sm.m));
          sm.l += p;
          // 0 log 0 = 0: a -inf logit (p = 0) adds nothing to s.
          if (p > 0.f) sm.s = fmaf(xs[e] * a.inv_temp, p, sm.s);
        }
      }
    }
  }
  // The four quarters of a row are adjacent lanes.
#pragma unroll
  for (int o = 1; o < 4; o <<= 1) {
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
  if (q == 0 && row < a.R) {
    const int64_t o = (int64_t)row * a.nblk + blk;
    a.rstat[o] = make_float4(best.v, __int_as_float(have ? best.i : -1), sm.m, sm.l);
    if constexpr (TYPICAL) a.rstat2[o] = sm.s;
  }

  // ---- optional logits output [R, V] ------------------------------------------------
  if (a.lout != nullptr && row < a.R && nv > 0) {
    uint16_t* dst = a.lout + (int64_t)row * a.lo_sr + vq;
    const uint16_t* src = reinterpret_cast<const uint16_t*>(tr);
    if (nv == kQ && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
#pragma unroll
      for (int c = 0; c < kQ / 8; ++c) reinterpret_cast<u32x4*>(dst)[c] = reinterpret_cast<const u32x4*>(src)[c];
    } else {
      for (int e = 0; e < nv; ++e) dst[e] = src[e];
    }
  }

  // ---- typical: each node's draft-token logit under its parent --------------------
  // Node i of tree t (hidden row t*M + i) needs logit[t*M + parent(i)][draft(i)];
  // the workgroup that holds both that hidden row and that vocabulary row
  // writes it.  parent(i) follows the walk: verify_new's parent_ext
  // (draft/tree_verification.py:120-125), malformed entries mapped to the
  // root (the walk flags them itself).
  if constexpr (TYPICAL) {
    for (int rho = tid; rho < a.R; rho += kLmThreads) {
      const int t = rho / a.M, i = rho - t * a.M;
      if (i == 0) continue;
      int64_t p = a.parent[(int64_t)t * a.p_st + (int64_t)(i - 1) * a.p_sm];
      if (p == i - 1) p = -1;
      if (p < -1 || p >= a.M - 1) p = -1;
      const int prow = t * a.M + (int)p + 1 - r0;
      const int64_t tok = a.draft[(int64_t)t * a.d_st + (int64_t)i * a.d_sm];
      if (prow >= 0 && prow < kLmRows && tok >= v0 && tok < v0 + kLmVocab && tok < a.V) {
        const uint16_t bits = *reinterpret_cast<const uint16_t*>(smem + prow * kTStride + (tok - v0) * 2);
        a.xtok[rho] = __uint_as_float((uint32_t)bits << 16);
      }
    }
  }
}

}  // namespace

int lmhead_blocks(int64_t V) { return (int)((V + kLmVocab - 1) / kLmVocab); }

hipError_t launch_lmhead_accept(const AcceptArgs& acc, const LmArgs& lm, hipStream_t s) {
  if (lm.R <= 0) return hipSuccess;
  const dim3 grid((unsigned)lm.nblk, (unsigned)((lm.R + kLmRows - 1) / kLmRows)), block(kLmThreads);
  if (lm.mode == 1)
    hipLaunchKernelGGL(lmhead_stats_kernel<true>, grid, block, 0, s, lm);
  else
    hipLaunchKernelGGL(lmhead_stats_kernel<false>, grid, block, 0, s, lm);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_accept_from_parts(acc, lm.rstat, lm.rstat2, lm.nblk, s);
}

}  // namespace dsv
