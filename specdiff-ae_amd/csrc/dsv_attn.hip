// dsv_attn.hip — kernels 1 and 2 of the tree-verification path on gfx950.
//
// One workgroup owns (batch b, KV head kvh, block of 256 query rows, one key
// split).  The 256 rows are the G query heads x M tree nodes that share KV
// head kvh (GQA-native: K/V are never expanded), so every K/V tile staged in
// LDS feeds G*M query rows.  Key splits are either
//   * a prefix split: keys [s*kps, (s+1)*kps) of the prefix, all visible
//     (or filtered by a byte mask for the bundle-verifier contract), or
//   * the tree split: the M tree keys, filtered by an ancestor-or-self bitmask
//     built in LDS from the parent array (or from a dense mask block).
// Each split writes an unnormalised partial (O, running max, running sum);
// kernel 3 (dsv_merge.hip) combines the splits.
//
// Math per 64-key tile, per wave of WR rows (WR = 32 or 64):
//   S^T[key, row] = K[key, :] . Q[row, :]      v_mfma_f32_32x32x16_{bf16,f16}
//   P = exp2(S * log2(e)/sqrt(D) - m_row)      online softmax, lazy rescale
//   O^T[d, row]  += V^T[d, key] . P^T[key,row] v_mfma_f32_32x32x16_{bf16,f16}
// Computing S^T (keys on the MFMA M side) leaves each lane owning one query
// row and 16 keys in the accumulator, which is exactly the B-operand layout
// the P.V product needs, so P never leaves registers.  V is transposed once
// per tile while it is written to LDS, so the P.V A-operand is a single
// 16-byte LDS read per lane.
//
// Reference semantics followed: runtime/tree_attention.py:116-217 (prefix
// O + LSE with an online softmax), :220-292 (tree block), :40-63 (naive tree
// attention), runtime/bundle_verifier.py:26-135 (masked bundle attention).

#include "dsv_internal.h"

namespace dsv {

namespace {

constexpr float kNegInf = -__builtin_huge_valf();
// Lazy-rescale threshold in log2 units: the running max used for the
// exponentials may lag the true max by up to this much (values <= 2^8).
constexpr float kRescaleTau = 8.0f;

template <typename T>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c);

template <>
__device__ __forceinline__ f32x16 mfma32<BF16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16 mfma32<F16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Pack two fp32 values into one dword of two 16-bit values (lo, hi), RNE.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack2<BF16>(float lo, float hi) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  bf2 r = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, r);
}
template <>
__device__ __forceinline__ uint32_t pack2<F16>(float lo, float hi) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  h2 r = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, r);
}

// Combine a value with the one held by lane (lane ^ 32).
__device__ __forceinline__ float xor32_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// Physical 16-byte slot of head-dim index d inside a transposed V row:
// a permutation inside each aligned group of 8, so that 16 consecutive lanes
// reading consecutive d stay conflict-free while the transposing writes of
// 16 lanes with different 8-wide d blocks spread over 8 slots.
__device__ __forceinline__ int vt_phys(int d) { return (d & ~7) | ((d ^ (d >> 3)) & 7); }

__device__ __forceinline__ int64_t load_index(const void* p, int is64, int64_t i) {
  return is64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t) reinterpret_cast<const int32_t*>(p)[i];
}

// Does element (i, j) of a dense tree-mask block keep the key?
__device__ __forceinline__ bool tmask_keep(const AttnArgs& a, int b, int i, int j) {
  const int64_t off = b * a.tm_sb + i * a.tm_sm + j * a.tm_sn;
  switch (a.tmask_dtype) {
    case 2: return reinterpret_cast<const float*>(a.tmask)[off] == 0.0f;          // f32 additive
    case 0: return (reinterpret_cast<const uint16_t*>(a.tmask)[off] & 0x7fff) == 0; // bf16 additive (+-0 keep)
    case 1: return (reinterpret_cast<const uint16_t*>(a.tmask)[off] & 0x7fff) == 0; // f16 additive
    default: return reinterpret_cast<const uint8_t*>(a.tmask)[off] != 0;           // int8/uint8/bool
  }
}

template <typename T, int D, int NW, int WR, bool DMASK>
__global__ void __launch_bounds__(NW * 64, NW / 4) attn_splitk_kernel(const AttnArgs a) {
  constexpr int NT = NW * 64;
  constexpr int KT = kTileKeys;
  constexpr int KS = D / 16;   // k-steps of the Q.K^T product
  constexpr int DT = D / 32;   // 32-row d tiles of the P.V product
  constexpr int CH = D / 8;    // 16-byte chunks per key row
  constexpr int SWZ = (CH < 16 ? CH : 16) - 1;
  constexpr int RT = WR / 32;  // 32-row MFMA tiles per wave
  constexpr int KCH = KT * CH;
  constexpr int KLD = (KCH + NT - 1) / NT;
  constexpr int VPR = (KT / 4) * CH;
  constexpr int VLD = (VPR + NT - 1) / NT;

  __shared__ __attribute__((aligned(16))) uint16_t ks_lds[2][KT * D];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[2][KT * D];
  __shared__ int32_t pt_lds[kPageLds];
  __shared__ uint64_t vis_lds[kTreeMaxM * kTreeMaxW];

  const int tid = threadIdx.x;
  const int wid = tid >> 6, lane = tid & 63, lj = lane & 31, lg = lane >> 5;

  // Block -> work item.  Consecutive dispatch ids go round-robin over the 8
  // XCDs; remap so that neighbouring work items (row blocks of one split)
  // land on the same XCD and share its L2.
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

  int64_t kstart, kend;
  if (is_tree) {
    kstart = 0;
    kend = a.M;
  } else {
    kstart = (int64_t)split * a.kps;
    kend = min(kstart + a.kps, a.n_pre);
  }

  // Stage this split's slice of the page table.
  int64_t pt_lo = 0;
  if (src.pt != nullptr && kend > kstart) {
    pt_lo = (src.key0 + kstart) >> src.ps_shift;
    const int64_t pt_hi = (src.key0 + kend - 1) >> src.ps_shift;
    for (int64_t i = tid; i <= pt_hi - pt_lo; i += NT) {
      // Out-of-range entries are clamped so that no access leaves the pool.
      int64_t pg = load_index(src.pt, src.pt_i64, b * src.pt_sb + pt_lo + i);
      pg = pg < 0 ? 0 : (pg >= src.n_phys ? src.n_phys - 1 : pg);
      pt_lds[i] = (int32_t)pg;
    }
  }

  // Tree split: ancestor-or-self bitmask of every node.
  if (is_tree) {
    const int M = a.M;
    for (int i = tid; i < M; i += NT) {
      uint64_t wd[kTreeMaxW];
#pragma unroll
      for (int x = 0; x < kTreeMaxW; ++x) wd[x] = 0;
      if (a.tpar != nullptr) {
        int node = i;
        for (int step = 0; step < M && node >= 0 && node < M; ++step) {
#pragma unroll
          for (int x = 0; x < kTreeMaxW; ++x)
            if ((node >> 6) == x) wd[x] |= 1ull << (node & 63);
          const int p = (int)load_index(a.tpar, a.tpar_i64, b * a.tpar_sb + node * a.tpar_sm);
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
      for (int x = 0; x < kTreeMaxW; ++x) vis_lds[i * kTreeMaxW + x] = wd[x];
    }
  }
  __syncthreads();

  // This wave's query rows and their Q fragments (B operand of S^T = K.Q^T:
  // lane (row lj, group lg) holds Q[row, 16*ks + 8*lg .. +8]).
  const int row0 = rb * (NW * WR) + wid * WR;
  const bool wave_active = row0 < a.R;
  u32x4 qf[RT][KS];
  int node_of[RT];
  bool rvalid[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int r = row0 + rt * 32 + lj;
    rvalid[rt] = r < a.R;
    node_of[rt] = 0;
    if (rvalid[rt]) {
      const int g = r / a.M;
      const int mi = r - g * a.M;
      // A permutation entry outside [0, M) is clamped: no access leaves q.
      const int m = a.row_perm ? min(max(a.row_perm[mi], 0), a.M - 1) : mi;
      node_of[rt] = m;
      const uint16_t* qp = a.q + b * a.q_sb + (int64_t)m * a.q_sm + (int64_t)(kvh * a.G + g) * a.q_sh + lg * 8;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qf[rt][ks] = ld16(qp + ks * 16);
    } else {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qf[rt][ks] = u32x4{0, 0, 0, 0};
    }
  }

  f32x16 acc[RT][DT];
  float mx[RT], lsum[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    mx[rt] = kNegInf;
    lsum[rt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[rt][dt] = f32x16{};
  }

  // Address of key n (source-relative) in the K or V half of the source.
  auto kv_addr = [&](const uint16_t* base, int64_t sb, int64_t sp, int64_t sh, int64_t st,
                     int64_t n) -> const uint16_t* {
    const int64_t ln = src.key0 + n;
    if (src.pt != nullptr) {
      const int64_t page = pt_lds[(ln >> src.ps_shift) - pt_lo];
      return base + b * sb + page * sp + kvh * sh + (ln & ((1ll << src.ps_shift) - 1)) * st;
    }
    return base + b * sb + ln * st + kvh * sh;
  };

  u32x4 kreg[KLD];
  u32x4 vreg[VLD][4];

  auto load_tile = [&](int64_t kb) {
#pragma unroll
    for (int i = 0; i < KLD; ++i) {
      const int c = tid + i * NT;
      kreg[i] = u32x4{0, 0, 0, 0};
      if (c < KCH) {
        const int key = c / CH, ch = c % CH;
        const int64_t n = kb + key;
        if (n < kend) kreg[i] = ld16(kv_addr(src.k, src.k_sb, src.k_sp, src.k_sh, src.k_st, n) + ch * 8);
      }
    }
#pragma unroll
    for (int i = 0; i < VLD; ++i) {
      const int p = tid + i * NT;
#pragma unroll
      for (int e = 0; e < 4; ++e) vreg[i][e] = u32x4{0, 0, 0, 0};
      if (p < VPR) {
        const int qd = p / CH, dblk = p % CH;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t n = kb + 4 * qd + e;
          if (n < kend) vreg[i][e] = ld16(kv_addr(src.v, src.v_sb, src.v_sp, src.v_sh, src.v_st, n) + dblk * 8);
        }
      }
    }
  };

  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KLD; ++i) {
      const int c = tid + i * NT;
      if (c < KCH) {
        const int key = c / CH, ch = c % CH;
        *reinterpret_cast<u32x4*>(&ks_lds[buf][key * D + ((ch ^ (key & SWZ)) * 8)]) = kreg[i];
      }
    }
#pragma unroll
    for (int i = 0; i < VLD; ++i) {
      const int p = tid + i * NT;
      if (p < VPR) {
        const int qd = p / CH, dblk = p % CH;
        const int sb = qd >> 3;
        const int kk = (qd & 7) * 4;
        const int h = kk >> 4, r = kk & 15;
        const int g = (r >> 2) & 1, e0 = (r >> 3) * 4;
        uint16_t* base = &vt_lds[buf][((sb * 2 + h) * 2 + g) * D * 8 + e0];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int d = dblk * 8 + j;
          const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
          const uint32_t w01 = __builtin_amdgcn_perm(vreg[i][1][j >> 1], vreg[i][0][j >> 1], sel);
          const uint32_t w23 = __builtin_amdgcn_perm(vreg[i][3][j >> 1], vreg[i][2][j >> 1], sel);
          *reinterpret_cast<u32x2*>(base + vt_phys(d) * 8) = u32x2{w01, w23};
        }
      }
    }
  };

  const int64_t nkeys = kend - kstart;
  const int ntiles = nkeys > 0 ? (int)((nkeys + KT - 1) / KT) : 0;

  if (ntiles > 0) {
    load_tile(kstart);
    store_tile(0);
  }
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    const int64_t kb = kstart + (int64_t)t * KT;
    if (t + 1 < ntiles) load_tile(kb + KT);

    bool do_compute = wave_active;
    uint64_t visw[RT];
    if (is_tree) {
      uint64_t any = 0;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        visw[rt] = rvalid[rt] ? vis_lds[node_of[rt] * kTreeMaxW + t] : 0ull;
        any |= visw[rt];
      }
      do_compute = do_compute && (__ballot(any != 0ull) != 0ull);
    }

    if (do_compute) {
      // One 32-key subtile at a time: QK^T, mask, online softmax, PV.
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        // ---- S^T = K . Q^T ----------------------------------------------
        f32x16 st[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) st[rt] = f32x16{};
        const int key = sb * 32 + lj;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int ch = ks * 2 + lg;
          const u32x4 kf = *reinterpret_cast<const u32x4*>(&ks_lds[buf][key * D + ((ch ^ (key & SWZ)) * 8)]);
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) st[rt] = mfma32<T>(kf, qf[rt][ks], st[rt]);
        }

        // ---- masking ----------------------------------------------------
        // Lane (lj, lg) value v holds key sb*32 + 8*(v/4) + 4*lg + v%4.
        if (kb + KT > kend || is_tree || DMASK) {
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const int kt = sb * 32 + 8 * (v >> 2) + 4 * lg + (v & 3);
              const int64_t n = kb + kt;
              bool keep = n < kend;
              if (is_tree) keep = keep && ((visw[rt] >> kt) & 1ull);
              if constexpr (DMASK) {
                const int64_t mb = (int64_t)b * a.dm_sb + (int64_t)node_of[rt] * a.dm_sm;
                keep = keep && (n < a.dm_n) && rvalid[rt] && (a.dmask[mb + n * a.dm_sn] != 0);
              }
              if (!keep) st[rt][v] = kNegInf;
            }
          }
        }

        // ---- online softmax (log2 domain, lazy rescale) -----------------
        float mt[RT];
        bool need = false;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          float m0 = st[rt][0];
#pragma unroll
          for (int v = 1; v < 16; ++v) m0 = fmaxf(m0, st[rt][v]);
          mt[rt] = xor32_max(m0) * a.scale_log2;
          need = need || (mt[rt] > mx[rt] + kRescaleTau);
        }
        if (__ballot(need) != 0ull) {
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            const float mn = fmaxf(mx[rt], mt[rt]);
            const float al = (mn == mx[rt]) ? 1.f : __builtin_amdgcn_exp2f(mx[rt] - mn);
            mx[rt] = mn;
            lsum[rt] *= al;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) acc[rt][dt] *= al;
          }
        }

        u32x4 pk[RT][2];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const float ms = (mx[rt] == kNegInf) ? 0.f : mx[rt];
          float ls = 0.f;
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            float p[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              p[e] = __builtin_amdgcn_exp2f(fmaf(st[rt][hh * 8 + e], a.scale_log2, -ms));
              ls += p[e];
            }
            pk[rt][hh] = u32x4{pack2<T>(p[0], p[1]), pack2<T>(p[2], p[3]), pack2<T>(p[4], p[5]),
                               pack2<T>(p[6], p[7])};
          }
          lsum[rt] += ls;
        }

        // ---- O^T += V^T . P^T -------------------------------------------
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            const int d = dt * 32 + lj;
            const u32x4 vf = *reinterpret_cast<const u32x4*>(
                &vt_lds[buf][(((sb * 2 + hh) * 2 + lg) * D + vt_phys(d)) * 8]);
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) acc[rt][dt] = mfma32<T>(vf, pk[rt][hh], acc[rt][dt]);
          }
        }
      }
    }

    if (t + 1 < ntiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: unnormalised partial + (max, sum) per row ----------------
  if (!wave_active) return;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const float ltot = xor32_sum(lsum[rt]);
    const int r = row0 + rt * 32 + lj;
    if (!rvalid[rt]) continue;
    const int64_t prow = (((int64_t)split * a.B + b) * a.Hk + kvh) * a.R + r;
    float* op = a.opart + prow * D;
    // Accumulator value v of d tile dt holds d = 32*dt + 8*(v/4) + 4*lg + v%4.
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const f32x4 val = {acc[rt][dt][4 * q4 + 0], acc[rt][dt][4 * q4 + 1], acc[rt][dt][4 * q4 + 2],
                           acc[rt][dt][4 * q4 + 3]};
        *reinterpret_cast<f32x4*>(op + dt * 32 + 8 * q4 + 4 * lg) = val;
      }
    }
    if (lg == 0) a.ml[prow] = make_float2(mx[rt], ltot);
  }
}

// Wave layout of a 256-row workgroup: 8 waves x 32 rows (2 waves per SIMD,
// default) or 4 waves x 64 rows (1 wave per SIMD, K/V fragments shared by two
// row tiles).  DSV_ATTN_WAVES=4 selects the latter.
int wave_layout() {
  static int w = [] {
    const char* e = getenv("DSV_ATTN_WAVES");
    return (e != nullptr && atoi(e) == 4) ? 4 : 8;
  }();
  return w;
}

template <typename T, int D, bool DMASK>
hipError_t launch_t(const AttnArgs& a, hipStream_t s) {
  const int64_t nblk = (int64_t)a.B * a.Hk * a.s_total * a.n_rb;
  if (nblk <= 0) return hipSuccess;
  if (wave_layout() == 4)
    hipLaunchKernelGGL((attn_splitk_kernel<T, D, 4, 64, DMASK>), dim3((unsigned)nblk), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((attn_splitk_kernel<T, D, 8, 32, DMASK>), dim3((unsigned)nblk), dim3(512), 0, s, a);
  return hipGetLastError();
}

template <typename T, bool DMASK>
hipError_t launch_d(const AttnArgs& a, int D, hipStream_t s) {
  switch (D) {
    case 64: return launch_t<T, 64, DMASK>(a, s);
    case 128: return launch_t<T, 128, DMASK>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_attn(const AttnArgs& a, int dtype, int D, bool dmask, hipStream_t s) {
  if (dtype == 0) return dmask ? launch_d<BF16, true>(a, D, s) : launch_d<BF16, false>(a, D, s);
  return dmask ? launch_d<F16, true>(a, D, s) : launch_d<F16, false>(a, D, s);
}

}  // namespace dsv
