// dsv_attn_f32.hip — kernels 1 and 2 of the tree-verification path for fp32
// Q/K/V on gfx950.
//
// The same split plan, work decomposition, masks and partial format as the
// 16-bit kernel (dsv_attn.hip): one workgroup of 8 waves owns (batch b, KV
// head kvh, block of 256 packed query rows, one key split), each wave 32
// rows; every split writes a normalised bf16 partial O and its (running max,
// sum) for kernel 3 (dsv_merge.hip).  The arithmetic is fp32 throughout: the
// products of both contractions run on the fp32 matrix cores
// (v_mfma_f32_32x32x2_f32, exact fp32 products, fp32 accumulation), the
// softmax and its normaliser in fp32, and P enters the P.V product unrounded.
// This is the reference's fp32 path (runtime/tree_attention.py:439-446 and
// :40-63: fp32 matmul, softmax, logsumexp, fp32 weights times fp32 V).
//
// Per 32-key tile, per wave of 32 rows:
//   S^T[key, row] = sum_d K[key, d] Q[row, d]: 64 MFMAs of 2 d each; lanes
//     0-31 contract d in [0, 64), lanes 32-63 d in [64, 128) (for D = 128),
//     so a lane reads 4 consecutive d of its key with one ds_read_b128.
//   The accumulator layout gives each lane one query row and 16 keys, as in
//   the 16-bit kernel; P is formed in place.
//   O^T[d, row] += sum_key V[key, d] P[key, row]: 16 MFMAs of 2 keys per
//     32-row d tile, each lane supplying its own P values; V is staged
//     transposed in LDS so a lane reads 4 consecutive keys at once.
// K and V tiles go HBM -> registers -> LDS with 16-byte loads, the next
// tile's loads in flight while the current one is computed.
//
// This path serves fp32 inputs (the reference's CPU configuration); the bf16
// path is the one tuned for speed.

#include <hip/hip_ext.h>

#include "dsv_attn_f32_geo.h"
#include "dsv_internal.h"

namespace dsv {

namespace {

constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float xor32_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __builtin_elementwise_maximum(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ int64_t load_index(const void* p, int is64, int64_t i) {
  return is64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t) reinterpret_cast<const int32_t*>(p)[i];
}

__device__ __forceinline__ bool tmask_keep(const AttnArgs& a, int b, int i, int j) {
  const int64_t off = b * a.tm_sb + i * a.tm_sm + j * a.tm_sn;
  switch (a.tmask_dtype) {
    case 2: return reinterpret_cast<const float*>(a.tmask)[off] == 0.0f;            // f32 additive
    case 0:                                                                          // bf16 additive
    case 1: return (reinterpret_cast<const uint16_t*>(a.tmask)[off] & 0x7fff) == 0;  // f16 additive (+-0 keep)
    default: return reinterpret_cast<const uint8_t*>(a.tmask)[off] != 0;             // int8/uint8/bool
  }
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  bf2 r = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, r);
}

template <int D, bool DMASK>
__global__ void __launch_bounds__(512, 1) attn_f32_kernel(const AttnArgs a) {
  using G = GeoF32<D>;
  constexpr int NW = 8;
  constexpr int NT = NW * 64;
  constexpr int KT = G::KT;
  constexpr int HD = D / 2;               // d per lane half in the Q.K^T contraction
  constexpr int DT = D / 32;              // 32-row d tiles of the P.V product
  constexpr int CPT = G::CHUNKS / NT;     // 16-byte chunks per thread per K (or V) tile
  static_assert(CPT * NT == G::CHUNKS, "a tile's chunks split evenly over the threads");
  // LDS: K tile [KT][D + 4], V^T tile [D][KT + 4] (floats; the pads spread
  // the operand reads over the banks), page-table slice, tree bitmask.
  constexpr int KROW = D + 4, VROW = KT + 4;
  constexpr int K_OFF = 0, V_OFF = K_OFF + KT * KROW * 4;
  constexpr int PT_OFF = V_OFF + D * VROW * 4;
  constexpr int VIS_OFF = PT_OFF + kPageLds * 4;
  constexpr int LDS_BYTES = VIS_OFF + kTreeSlots * kTreeMaxW * 8;
  __shared__ __attribute__((aligned(16))) uint8_t smem[LDS_BYTES];
  float* ks = reinterpret_cast<float*>(smem + K_OFF);
  float* vts = reinterpret_cast<float*>(smem + V_OFF);
  int32_t* pt_lds = reinterpret_cast<int32_t*>(smem + PT_OFF);
  uint64_t* vis_lds = reinterpret_cast<uint64_t*>(smem + VIS_OFF);

  const int tid = threadIdx.x;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, lj = lane & 31, lg = lane >> 5;

  // Block -> work item, with the 16-bit kernel's XCD remap.
  const int nblk = gridDim.x;
  int w = ((nblk & 7) == 0) ? (blockIdx.x & 7) * (nblk >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const int rb = w % a.n_rb;
  w /= a.n_rb;
  const int split = w % a.s_total;
  w /= a.s_total;
  const int kvh = w % a.Hk;
  const int b = w / a.Hk;
  const bool is_tree = a.has_tree && split == a.n_splits;
  const KvSrc src = is_tree ? a.tree : a.pre;

  int64_t n_pre_b = a.n_pre;
  if (a.seqlens != nullptr) {
    n_pre_b = load_index(a.seqlens, a.seqlens_i64, b);
    n_pre_b = n_pre_b < 0 ? 0 : (n_pre_b > a.n_pre ? a.n_pre : n_pre_b);
  }
  int64_t kstart, kend;
  if (is_tree) {
    kstart = 0;
    kend = a.M;
  } else {
    kstart = (int64_t)split * a.kps;
    kend = min(kstart + a.kps, n_pre_b);
  }
  const int64_t nkeys = kend - kstart;
  const int ntiles = nkeys > 0 ? (int)((nkeys + KT - 1) / KT) : 0;
  const bool causal = a.causal != 0 && !is_tree;
  const int64_t c0 = n_pre_b - a.M;
  const bool paged = src.pt != nullptr;

  // ---- set-up: page-table slice, tree bitmask (as in the 16-bit kernel) -------
  int64_t pt_lo = 0;
  if (paged && ntiles > 0) {
    pt_lo = (src.key0 + kstart) >> src.ps_shift;
    const int64_t pt_hi = (src.key0 + kend - 1) >> src.ps_shift;
    for (int64_t i = tid; i <= pt_hi - pt_lo; i += NT)
      pt_lds[i] = (int32_t)clamp_page(load_index(src.pt, src.pt_i64, b * src.pt_sb + pt_lo + i), src.n_phys);
  }
  if (is_tree) {
    const int M = a.M;
    int32_t* par_lds = reinterpret_cast<int32_t*>(smem + K_OFF);  // K tile, idle until the first tile
    static_assert(kTreeMaxM * 4 <= KT * KROW * 4, "parent staging fits the K tile");
    if (a.tpar != nullptr) {
      for (int i = tid; i < M; i += NT)
        par_lds[i] = (int32_t)load_index(a.tpar, a.tpar_i64, b * a.tpar_sb + i * a.tpar_sm);
      __syncthreads();
    }
    // Entry lr of the table: the ancestor-or-self bits (kTreeMaxW words, of
    // which the first ceil(M/64) are used) of the node of this block's packed
    // row lr (0 <= lr < 256, row = 256 * rb + lr, node slot mi = row mod M).
    const int W = (M + 63) >> 6;
    const int row_first = rb * (NW * 32);
    for (int lr = tid; lr < kTreeSlots; lr += NT) {
      const int row = row_first + lr;
      if (row >= a.R) break;
      const int mi = row % M;
      // A permutation entry outside [0, M) is clamped, as for the Q rows.
      const int i = a.row_perm ? min(max(a.row_perm[mi], 0), M - 1) : mi;
      uint64_t wd[kTreeMaxW];
#pragma unroll
      for (int x = 0; x < kTreeMaxW; ++x) wd[x] = 0;
      if (a.tpar != nullptr) {
        int node = i;
        for (int step = 0; step < M && node >= 0 && node < M; ++step) {
#pragma unroll
          for (int x = 0; x < kTreeMaxW; ++x)
            if ((node >> 6) == x) wd[x] |= 1ull << (node & 63);
          const int p = par_lds[node];
          if (p == node) break;
          node = p;
        }
      } else {
        for (int j = 0; j < M; ++j) {
          if (tmask_keep(a, b, i, j)) {
#pragma unroll
            for (int x = 0; x < kTreeMaxW; ++x)
              if ((j >> 6) == x) wd[x] |= 1ull << (j & 63);
          }
        }
      }
#pragma unroll
      for (int x = 0; x < kTreeMaxW; ++x)
        if (x < W) vis_lds[lr * kTreeMaxW + x] = wd[x];
    }
  }
  __syncthreads();

  // ---- this wave's query rows: lane (row lj, half lg) holds Q[row, HD*lg .. +HD)
  const int row0 = rb * (NW * 32) + wid * 32;
  const bool wave_active = row0 < a.R;
  const int r_me = row0 + lj;
  const bool rvalid = r_me < a.R;
  float qf[HD];
  int node_of = 0;
  if (rvalid) {
    const int g = r_me / a.M;
    const int mi = r_me - g * a.M;
    const int m = a.row_perm ? min(max(a.row_perm[mi], 0), a.M - 1) : mi;
    node_of = m;
    const float* qp = reinterpret_cast<const float*>(a.q) + b * a.q_sb + (int64_t)m * a.q_sm +
                      (int64_t)(kvh * a.G + g) * a.q_sh + lg * HD;
#pragma unroll
    for (int c = 0; c < HD / 4; ++c) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(qp + 4 * c);
#pragma unroll
      for (int e = 0; e < 4; ++e) qf[4 * c + e] = x[e];
    }
  } else {
#pragma unroll
    for (int c = 0; c < HD; ++c) qf[c] = 0.f;
  }
  const float scale_log2 = a.scale_log2;

  // ---- tile loads: thread tid moves chunks tid + NT * x of the K and V tiles
  const float* kbase = reinterpret_cast<const float*>(src.k);
  const float* vbase = reinterpret_cast<const float*>(src.v);
  f32x4 kreg[CPT], vreg[CPT];
  auto load_tile = [&](int t) {
    const int64_t kb = kstart + (int64_t)t * KT;
#pragma unroll
    for (int x = 0; x < CPT; ++x) {
      const int ch = tid + NT * x;
      const int kk = ch / G::CPR, c4 = ch % G::CPR;
      const int64_t n = f32_key(src, kb, kend, kk);
      const int64_t page = paged ? pt_lds[(n >> src.ps_shift) - pt_lo] : 0;
      kreg[x] = *reinterpret_cast<const f32x4*>(kbase + f32_elem(src, false, b, kvh, n, page, c4));
      vreg[x] = *reinterpret_cast<const f32x4*>(vbase + f32_elem(src, true, b, kvh, n, page, c4));
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int x = 0; x < CPT; ++x) {
      const int ch = tid + NT * x;
      const int kk = ch / G::CPR, c4 = ch % G::CPR;
      *reinterpret_cast<f32x4*>(ks + kk * KROW + 4 * c4) = kreg[x];
#pragma unroll
      for (int e = 0; e < 4; ++e) vts[(4 * c4 + e) * VROW + kk] = vreg[x][e];
    }
  };

  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16{};
  float mx = kNegInf, lsum = 0.f;

  if (ntiles > 0) load_tile(0);
  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();  // every wave is done with the previous tile
    store_tile();
    __syncthreads();
    if (t + 1 < ntiles) load_tile(t + 1);  // in flight during this tile's products
    if (!wave_active) continue;

    // S^T = K . Q^T: A = K[key lj][d], B = Q[row lj][d], d = HD*lg + kstep.
    f32x16 s = f32x16{};
    const float* krow = ks + lj * KROW + lg * HD;
#pragma unroll
    for (int c = 0; c < HD / 4; ++c) {
      const f32x4 kv = *reinterpret_cast<const f32x4*>(krow + 4 * c);
#pragma unroll
      for (int e = 0; e < 4; ++e) s = mfma_f32(kv[e], qf[4 * c + e], s);
    }

    // Keep mask (tail keys, causal, tree visibility, byte mask).  Value v of a
    // lane holds key 8*(v/4) + 4*lg + v%4 of the tile.
    const int64_t kb = kstart + (int64_t)t * KT;
    const bool masked = is_tree || DMASK || causal || kb + KT > kend;
    if (masked) {
      const int64_t ke = causal ? min(kend, c0 + 1 + node_of) : kend;
      uint32_t keep = 0;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int key = 8 * (v >> 2) + 4 * lg + (v & 3);
        keep |= (uint32_t)(kb + key < ke) << v;
      }
      if (is_tree) {
        const uint64_t vw = rvalid ? vis_lds[(wid * 32 + lj) * kTreeMaxW + (t >> 1)] : 0ull;
        const uint32_t vb = (uint32_t)(vw >> ((t & 1) * 32 + 4 * lg));
        keep &= (vb & 0xFu) | ((vb >> 4) & 0xF0u) | ((vb >> 8) & 0xF00u) | ((vb >> 12) & 0xF000u);
      }
      if constexpr (DMASK) {
        const uint8_t* mrow = a.dmask + (int64_t)b * a.dm_sb + (int64_t)node_of * a.dm_sm;
        uint32_t mb = 0;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t n = kb + 8 * (v >> 2) + 4 * lg + (v & 3);
          mb |= (uint32_t)((n < a.dm_n) && (mrow[n * a.dm_sn] != 0)) << v;
        }
        keep &= rvalid ? mb : 0u;
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) s[v] = ((keep >> v) & 1u) ? s[v] : kNegInf;
    }

    // Online softmax in the log2 domain against the exact running maximum
    // (NaN-propagating, like torch.max).
    float mt = s[0];
#pragma unroll
    for (int v = 1; v < 16; ++v) mt = __builtin_elementwise_maximum(mt, s[v]);
    mt = xor32_max(mt) * scale_log2;
    const float mn = __builtin_elementwise_maximum(mx, mt);
    if (mn != mx) {
      const float al = (mx == kNegInf) ? 0.f : __builtin_amdgcn_exp2f(mx - mn);
      lsum *= al;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt] *= al;
      mx = mn;
    }
    const float ms = (mx == kNegInf) ? 0.f : mx;
    float p[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      p[v] = __builtin_amdgcn_exp2f(fmaf(s[v], scale_log2, -ms));
      lsum += p[v];
    }

    // O^T += V^T . P^T: A = V[key][d = 32*dt + lj] (from V^T in LDS), B = P.
    // k-step u covers keys 8*(u/4) + 4*lg + u%4 (this lane's p[u]).
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const float* vrow = vts + (32 * dt + lj) * VROW + 4 * lg;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const f32x4 vv = *reinterpret_cast<const f32x4*>(vrow + 8 * q4);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[dt] = mfma_f32(vv[e], p[4 * q4 + e], acc[dt]);
      }
    }
  }

  // ---- epilogue: normalised bf16 partial + (max, sum) per row ----------------
  if (!wave_active) return;
  const float ltot = xor32_sum(lsum);
  const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
  const int64_t pbase = (((int64_t)split * a.B + b) * a.Hk + kvh) * a.R + row0;
  if (rvalid) {
    uint16_t* op = a.opart + (pbase + lj) * D;
    // Value v of d tile dt holds d = 32*dt + 8*(v/4) + 4*lg + v%4.
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const f32x16 x = acc[dt];
        const u32x2 val = {pack_bf16(x[4 * q4] * inv, x[4 * q4 + 1] * inv),
                           pack_bf16(x[4 * q4 + 2] * inv, x[4 * q4 + 3] * inv)};
        *reinterpret_cast<u32x2*>(op + 32 * dt + 8 * q4 + 4 * lg) = val;
      }
    if (lg == 0) a.ml[pbase + lj] = make_float2(mx, ltot);
  }
}

template <int D, bool DMASK>
hipError_t launch_f32_t(const AttnArgs& a, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  const int64_t nblk = (int64_t)a.B * a.Hk * a.s_total * a.n_rb;
  if (nblk <= 0) return hipSuccess;
  const dim3 grid((unsigned)nblk), block(512);
  if (ev0 != nullptr || ev1 != nullptr)
    hipExtLaunchKernelGGL((attn_f32_kernel<D, DMASK>), grid, block, 0, s, ev0, ev1, 0, a);
  else
    hipLaunchKernelGGL((attn_f32_kernel<D, DMASK>), grid, block, 0, s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_attn_f32(const AttnArgs& a, int D, bool dmask, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  switch (D) {
    case 64: return dmask ? launch_f32_t<64, true>(a, s, ev0, ev1) : launch_f32_t<64, false>(a, s, ev0, ev1);
    case 128: return dmask ? launch_f32_t<128, true>(a, s, ev0, ev1) : launch_f32_t<128, false>(a, s, ev0, ev1);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace dsv
