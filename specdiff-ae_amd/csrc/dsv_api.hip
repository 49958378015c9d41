// dsv_api.hip — C ABI of libdsv.so: argument validation, split planning,
// workspace carving and kernel launches.  Declarations and the reference
// interface each entry point replaces are in include/dsv.h.

#include "dsv.h"
#include "dsv_attn_geo.h"
#include "dsv_check.h"
#include "dsv_internal.h"

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

namespace dsv {
size_t accept_walk_lds_bytes(int M);
}

namespace {

using dsv::AcceptArgs;
using dsv::AttnArgs;
using dsv::AttnExtents;
using dsv::Extent;
using dsv::KvSrc;
using dsv::MergeArgs;

thread_local std::string g_err;
thread_local int g_dry_run = 0;
thread_local int64_t g_dry_checks = 0;

// Byte span of a tensor view from its data pointer (non-negative strides),
// over dimensions [first, ndim).
int64_t span_bytes(const dsv_tensor* t, int first = 0) {
  int64_t s = 1;
  for (int i = first; i < t->ndim; ++i) {
    if (t->shape[i] == 0) return 0;
    s += (t->shape[i] - 1) * t->stride[i];
  }
  static const int es[] = {2, 2, 4, 1, 1, 1, 4, 8};
  return s * ((t->dtype >= 0 && t->dtype <= 7) ? es[t->dtype] : 1);
}

Extent extent_of(const char* name, const dsv_tensor* t) {
  if (t == nullptr || t->ndim == 0 || t->data == nullptr) return Extent{name, 0, 0};
  const uintptr_t lo = (uintptr_t)t->data;
  return Extent{name, lo, lo + (uintptr_t)span_bytes(t)};
}

Extent extent_raw(const char* name, const void* p, int64_t bytes) {
  return Extent{name, (uintptr_t)p, (uintptr_t)p + (uintptr_t)(bytes > 0 ? bytes : 0)};
}

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(DSV_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int elem_size(int dt) {
  switch (dt) {
    case DSV_BF16:
    case DSV_F16: return 2;
    case DSV_F32:
    case DSV_I32: return 4;
    case DSV_I64: return 8;
    case DSV_I8:
    case DSV_U8:
    case DSV_BOOL: return 1;
    default: return 0;
  }
}

const char* dt_name(int dt) {
  static const char* names[] = {"bf16", "f16", "f32", "int8", "uint8", "bool", "int32", "int64"};
  return (dt >= 0 && dt <= 7) ? names[dt] : "?";
}

bool present(const dsv_tensor* t) { return t != nullptr && t->ndim > 0; }

int check_nd(const dsv_tensor* t, const char* name, int ndim) {
  if (t == nullptr || t->ndim != ndim)
    return fail(DSV_ERR_INVALID, "%s must be a %d-d tensor (got %d-d)", name, ndim, t ? t->ndim : -1);
  if (t->data == nullptr) return fail(DSV_ERR_INVALID, "%s has a null data pointer", name);
  if (elem_size(t->dtype) == 0) return fail(DSV_ERR_INVALID, "%s has an unknown dtype %d", name, t->dtype);
  for (int i = 0; i < ndim; ++i) {
    if (t->shape[i] < 0) return fail(DSV_ERR_INVALID, "%s has a negative extent", name);
    if (t->stride[i] < 0) return fail(DSV_ERR_INVALID, "%s has a negative stride", name);
  }
  return DSV_OK;
}

// Attention operand (q, k, v, pages) read with 16-byte vector loads: bf16,
// f16 or f32; innermost stride 1, other strides multiples of 16 bytes,
// 16-byte aligned base.
int check_vec16(const dsv_tensor* t, const char* name, int skip_dim = -1) {
  if (t->dtype != DSV_BF16 && t->dtype != DSV_F16 && t->dtype != DSV_F32)
    return fail(DSV_ERR_UNSUPPORTED, "%s: dtype %s is not supported by the MI355X kernels (bf16, f16 or f32)",
                name, dt_name(t->dtype));
  const int per16 = 16 / elem_size(t->dtype);  // elements per 16 bytes
  if (t->stride[t->ndim - 1] != 1) return fail(DSV_ERR_INVALID, "%s: innermost stride must be 1", name);
  if ((reinterpret_cast<uintptr_t>(t->data) & 15) != 0)
    return fail(DSV_ERR_INVALID, "%s: data pointer must be 16-byte aligned", name);
  for (int i = 0; i < t->ndim - 1; ++i) {
    if (i == skip_dim) continue;
    if (t->shape[i] > 1 && (t->stride[i] % per16) != 0)
      return fail(DSV_ERR_INVALID, "%s: stride[%d]=%lld is not a multiple of %d elements (16 bytes)", name, i,
                  (long long)t->stride[i], per16);
  }
  return DSV_OK;
}

int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

struct Plan {
  int G = 0, R = 0, n_rb = 0, n_splits = 0, s_total = 0;
  int64_t kps = 0;
  size_t opart_bytes = 0, ml_bytes = 0, total = 0;
  const char* err = nullptr;  // sizes beyond the kernels' 32-bit counts (nothing planned)
};

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Splits are sized so that prefix workgroups plus the tree workgroups fill
// every resident workgroup slot of the GPU exactly once.
Plan make_plan(int64_t B, int64_t M, int64_t H, int64_t Hk, int64_t D, int64_t n_keys, int64_t page_size,
               bool has_tree) {
  Plan p;
  const int rows_per_block = dsv::attn_rows_per_block();
  // Row, split and workgroup counts are 32-bit in the kernels and the merge.
  const bool in_range = B <= (1 << 20) && M <= (1 << 24) && H <= (1 << 16) && n_keys <= ((int64_t)1 << 40);
  const int64_t R = in_range ? (H / Hk) * M : 0;
  if (!in_range || R > ((int64_t)1 << 24) || B * Hk * R > ((int64_t)1 << 30)) {
    p.err = "sizes beyond the attention kernels' range (batch <= 2^20, heads <= 65536, keys <= 2^40, query heads / "
            "key heads x rows <= 2^24, batch x query heads x rows <= 2^30)";
    return p;
  }
  p.G = (int)(H / Hk);
  p.R = (int)R;
  p.n_rb = (int)((p.R + rows_per_block - 1) / rows_per_block);
  const int64_t units = B * Hk * p.n_rb;
  if (n_keys > 0) {
    const int64_t slots = (int64_t)device_cus() * dsv::attn_blocks_per_cu();
    const int64_t avail = std::max<int64_t>(slots - (has_tree ? units : 0), units);
    const int64_t s0 = std::max<int64_t>(1, avail / units);
    int64_t kps_max = 16384;
    if (page_size > 0) kps_max = std::min<int64_t>(kps_max, (int64_t)(dsv::kPageLds - 2) * page_size);
    // Whole 32-key tiles per split.
    kps_max = std::max<int64_t>(32, kps_max / 32 * 32);
    int64_t kps = ((n_keys + s0 - 1) / s0 + 31) / 32 * 32;
    kps = std::min(std::max<int64_t>(kps, 32), kps_max);
    p.kps = kps;
    const int64_t ns = (n_keys + kps - 1) / kps;
    if (units * (ns + 1) >= ((int64_t)1 << 31)) {
      p = Plan{};
      p.err = "the key splits need more than 2^31 workgroups";
      return p;
    }
    p.n_splits = (int)ns;
  }
  p.s_total = p.n_splits + (has_tree ? 1 : 0);
  const size_t rows = (size_t)p.s_total * B * Hk * p.R;
  p.opart_bytes = align_up(rows * D * sizeof(uint16_t), 256);
  p.ml_bytes = align_up(rows * sizeof(float2), 256);
  p.total = p.opart_bytes + p.ml_bytes;
  return p;
}

int log2_exact(int64_t x) {
  if (x <= 0 || (x & (x - 1)) != 0) return -1;
  int s = 0;
  while ((1ll << s) < x) ++s;
  return s;
}

// Common checks of q [B, M, H, D] and the output [B, M, H, D].
int check_q_out(const dsv_tensor* q, const dsv_tensor* out) {
  int rc;
  if ((rc = check_nd(q, "q", 4)) != DSV_OK) return rc;
  if ((rc = check_vec16(q, "q")) != DSV_OK) return rc;
  if ((rc = check_nd(out, "out", 4)) != DSV_OK) return rc;
  for (int i = 0; i < 4; ++i)
    if (out->shape[i] != q->shape[i]) return fail(DSV_ERR_INVALID, "out shape must equal q shape");
  if (out->dtype != DSV_BF16 && out->dtype != DSV_F16 && out->dtype != DSV_F32)
    return fail(DSV_ERR_INVALID, "out dtype must be bf16, f16 or f32");
  if (out->stride[3] != 1) return fail(DSV_ERR_INVALID, "out innermost stride must be 1");
  const int64_t D = q->shape[3];
  if (D != 64 && D != 128) return fail(DSV_ERR_UNSUPPORTED, "head_dim %lld is not supported (64 or 128)", (long long)D);
  return DSV_OK;
}

int check_kv_dense(const dsv_tensor* k, const dsv_tensor* v, const dsv_tensor* q, const char* kn, const char* vn) {
  int rc;
  if ((rc = check_nd(k, kn, 4)) != DSV_OK) return rc;
  if ((rc = check_nd(v, vn, 4)) != DSV_OK) return rc;
  if ((rc = check_vec16(k, kn)) != DSV_OK) return rc;
  if ((rc = check_vec16(v, vn)) != DSV_OK) return rc;
  for (int i = 0; i < 4; ++i)
    if (k->shape[i] != v->shape[i]) return fail(DSV_ERR_INVALID, "%s and %s shapes differ", kn, vn);
  if (k->dtype != q->dtype || v->dtype != q->dtype)
    return fail(DSV_ERR_INVALID, "q, %s and %s must share a dtype", kn, vn);
  if (k->shape[0] != q->shape[0]) return fail(DSV_ERR_INVALID, "%s batch differs from q", kn);
  if (k->shape[3] != q->shape[3]) return fail(DSV_ERR_INVALID, "%s head_dim differs from q", kn);
  const int64_t H = q->shape[2], Hk = k->shape[2];
  if (Hk <= 0 || H % Hk != 0)
    return fail(DSV_ERR_INVALID, "query heads (%lld) must be a multiple of key heads (%lld)", (long long)H,
                (long long)Hk);
  return DSV_OK;
}

KvSrc dense_src(const dsv_tensor* k, const dsv_tensor* v, int64_t key0) {
  KvSrc s{};
  s.k = static_cast<const uint16_t*>(k->data);
  s.v = static_cast<const uint16_t*>(v->data);
  s.k_sb = k->shape[0] > 1 ? k->stride[0] : 0;
  s.k_st = k->stride[1];
  s.k_sh = k->stride[2];
  s.v_sb = v->shape[0] > 1 ? v->stride[0] : 0;
  s.v_st = v->stride[1];
  s.v_sh = v->stride[2];
  s.pt = nullptr;
  s.key0 = key0;
  s.k_bytes = span_bytes(k);
  s.v_bytes = span_bytes(v);
  return s;
}

int check_ws(const Plan& p, void* ws, size_t ws_bytes) {
  if (p.err != nullptr) return fail(DSV_ERR_UNSUPPORTED, "%s", p.err);
  if (p.total == 0) return DSV_OK;
  if (ws == nullptr || ws_bytes < p.total)
    return fail(DSV_ERR_WORKSPACE, "workspace of %zu bytes required (got %zu)", p.total, ws_bytes);
  if ((reinterpret_cast<uintptr_t>(ws) & 255) != 0) return fail(DSV_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  return DSV_OK;
}

void fill_common(AttnArgs& a, const dsv_tensor* q, int64_t Hk, const Plan& p, void* ws) {
  a.q = static_cast<const uint16_t*>(q->data);
  a.q_sb = q->stride[0];
  a.q_sm = q->stride[1];
  a.q_sh = q->stride[2];
  a.B = (int)q->shape[0];
  a.M = (int)q->shape[1];
  a.H = (int)q->shape[2];
  a.Hk = (int)Hk;
  a.G = p.G;
  a.R = p.R;
  a.n_rb = p.n_rb;
  a.scale_log2 = (float)(1.4426950408889634 / sqrt((double)q->shape[3]));
  a.n_splits = p.n_splits;
  a.kps = p.kps;
  a.s_total = p.s_total;
  a.opart = static_cast<uint16_t*>(ws);
  a.ml = reinterpret_cast<float2*>(static_cast<char*>(ws) + p.opart_bytes);
}

void fill_merge(MergeArgs& m, const AttnArgs& a, const dsv_tensor* out, int D) {
  m.opart = a.opart;
  m.ml = a.ml;
  m.s_total = a.s_total;
  m.B = a.B;
  m.M = a.M;
  m.H = a.H;
  m.Hk = a.Hk;
  m.G = a.G;
  m.R = a.R;
  m.D = D;
  m.row_perm = a.row_perm;
  m.out = out->data;
  m.out_dtype = out->dtype;
  m.o_sb = out->stride[0];
  m.o_sm = out->stride[1];
  m.o_sh = out->stride[2];
}

// One-shot timing events armed by dsv_set_timing_events (per thread).
thread_local hipEvent_t g_ev_start = nullptr;
thread_local hipEvent_t g_ev_stop = nullptr;

void take_events(hipEvent_t& s, hipEvent_t& e) {
  s = g_ev_start;
  e = g_ev_stop;
  g_ev_start = g_ev_stop = nullptr;
}

// Extents shared by every attention entry point (dry-run checks).
AttnExtents common_extents(const dsv_tensor* q, const dsv_tensor* out, void* ws, const Plan& p) {
  AttnExtents ex;
  ex.q = extent_of("q", q);
  ex.out = extent_of("out", out);
  ex.ws = extent_raw("workspace", ws, (int64_t)p.total);
  return ex;
}

int run(const AttnArgs& a_in, const MergeArgs& m, int dtype, int D, bool dmask, hipStream_t st,
        const AttnExtents& ex) {
  AttnArgs a = a_in;
  a.pre.fast32 = dsv::fast32_ok(a.pre, a.pre.key0 + a.n_pre) ? 1 : 0;
  a.tree.fast32 = a.has_tree && dsv::fast32_ok(a.tree, a.tree.key0 + a.M) ? 1 : 0;
  if (g_dry_run) {
    std::string err;
    int64_t n = 0;
    const int rc = dsv::emulate_attention(a, m, D, dmask, dtype == DSV_F32, ex, err, &n);
    g_dry_checks = n;
    if (rc != 0) return fail(DSV_ERR_INVALID, "dry run: out-of-bounds access: %s", err.c_str());
    return DSV_OK;
  }
  hipEvent_t ev0, ev1;
  take_events(ev0, ev1);
  hipError_t e = dtype == DSV_F32 ? dsv::launch_attn_f32(a, D, dmask, st, ev0, ev1)
                                  : dsv::launch_attn(a, dtype, D, dmask, st, ev0, ev1);
  if (e != hipSuccess) return hip_fail(e, "attention kernel launch");
  e = dsv::launch_merge(m, st);
  if (e != hipSuccess) return hip_fail(e, "merge kernel launch");
  return DSV_OK;
}

int check_byte_mask(const dsv_tensor* mask, int64_t B, int64_t M, const char* name) {
  int rc;
  if ((rc = check_nd(mask, name, 3)) != DSV_OK) return rc;
  if (mask->dtype != DSV_I8 && mask->dtype != DSV_U8 && mask->dtype != DSV_BOOL)
    return fail(DSV_ERR_INVALID, "%s must be int8, uint8 or bool (got %s)", name, dt_name(mask->dtype));
  if (mask->shape[0] != 1 && mask->shape[0] != B) return fail(DSV_ERR_INVALID, "%s batch must be 1 or B", name);
  if (mask->shape[1] != M) return fail(DSV_ERR_INVALID, "%s must have M rows", name);
  return DSV_OK;
}

// Physical page pool view: kv_pages [L, 2, P, Hk, ps, D] -> K and V halves of one layer.
int paged_src(const dsv_tensor* kv_pages, int64_t layer, const dsv_tensor* pt, int64_t B, KvSrc& s,
              int64_t& page_size, int64_t& Hk, int64_t& D, int64_t& capacity) {
  int rc;
  if ((rc = check_nd(kv_pages, "kv_pages", 6)) != DSV_OK) return rc;
  if ((rc = check_vec16(kv_pages, "kv_pages")) != DSV_OK) return rc;
  if (kv_pages->shape[1] != 2) return fail(DSV_ERR_INVALID, "kv_pages dim 1 must be 2 (K, V)");
  if (layer < 0 || layer >= kv_pages->shape[0]) return fail(DSV_ERR_INVALID, "layer_idx out of range");
  page_size = kv_pages->shape[4];
  const int sh = log2_exact(page_size);
  if (sh < 0) return fail(DSV_ERR_UNSUPPORTED, "page_size %lld must be a power of two", (long long)page_size);
  if ((rc = check_nd(pt, "page_table", pt ? pt->ndim : 1)) != DSV_OK) return rc;
  if (pt->ndim != 1 && pt->ndim != 2) return fail(DSV_ERR_INVALID, "page_table must be 1-d or 2-d");
  if (pt->dtype != DSV_I32 && pt->dtype != DSV_I64) return fail(DSV_ERR_INVALID, "page_table must be int32 or int64");
  if (pt->ndim == 2 && pt->shape[0] != B && pt->shape[0] != 1)
    return fail(DSV_ERR_INVALID, "page_table batch must be 1 or B");
  const int64_t npt = pt->shape[pt->ndim - 1];
  if (pt->stride[pt->ndim - 1] != 1) return fail(DSV_ERR_INVALID, "page_table innermost stride must be 1");
  Hk = kv_pages->shape[3];
  D = kv_pages->shape[5];
  const int es = elem_size(kv_pages->dtype);
  const char* base = static_cast<const char*>(kv_pages->data) + layer * kv_pages->stride[0] * es;
  s.k = reinterpret_cast<const uint16_t*>(base);
  s.v = reinterpret_cast<const uint16_t*>(base + kv_pages->stride[1] * es);
  s.k_sb = s.v_sb = 0;
  s.k_sp = s.v_sp = kv_pages->stride[2];
  s.k_sh = s.v_sh = kv_pages->stride[3];
  s.k_st = s.v_st = kv_pages->stride[4];
  s.pt = pt->data;
  s.pt_i64 = pt->dtype == DSV_I64;
  s.ps_shift = sh;
  s.pt_sb = (pt->ndim == 2 && pt->shape[0] > 1) ? pt->stride[0] : 0;
  s.key0 = 0;
  s.n_phys = kv_pages->shape[2];
  s.k_bytes = s.v_bytes = span_bytes(kv_pages, 2);
  capacity = npt * page_size;
  (void)B;
  return DSV_OK;
}

}  // namespace

extern "C" {

int dsv_version(void) { return 1; }

const char* dsv_last_error(void) { return g_err.c_str(); }

int dsv_set_timing_events(void* start_event, void* stop_event) {
  g_ev_start = static_cast<hipEvent_t>(start_event);
  g_ev_stop = static_cast<hipEvent_t>(stop_event);
  return DSV_OK;
}

int dsv_set_dry_run(int enable) {
  g_dry_run = enable != 0;
  return DSV_OK;
}

int64_t dsv_dry_run_checks(void) { return g_dry_checks; }

size_t dsv_attn_workspace_bytes(int64_t B, int64_t M, int64_t H, int64_t Hk, int64_t D, int64_t n_keys,
                                int64_t page_size, int has_tree) {
  if (B <= 0 || M <= 0 || H <= 0 || Hk <= 0 || D <= 0 || H % Hk != 0 || n_keys < 0) return 0;
  return make_plan(B, M, H, Hk, D, n_keys, page_size, has_tree != 0).total;
}

}  // extern "C"

namespace {

// Prefix attention with an optional per-batch length and causal mask: the
// body of dsv_prefix_attention_forward and dsv_flash_attn_with_kvcache.
int prefix_attention(const dsv_tensor* q, const dsv_tensor* k, const dsv_tensor* v, const dsv_tensor* seqlens,
                     int64_t n_keys, int causal, dsv_tensor* out, dsv_tensor* lse, void* workspace,
                     size_t workspace_bytes, void* stream) {
  int rc;
  if ((rc = check_q_out(q, out)) != DSV_OK) return rc;
  if ((rc = check_kv_dense(k, v, q, "k", "v")) != DSV_OK) return rc;
  const int64_t B = q->shape[0], M = q->shape[1], H = q->shape[2], D = q->shape[3];
  const int64_t N = k->shape[1], Hk = k->shape[2];
  if (n_keys < 0) n_keys = N;
  if (n_keys > N) return fail(DSV_ERR_INVALID, "n_keys (%lld) exceeds the key length (%lld)", (long long)n_keys, (long long)N);
  if (present(seqlens)) {
    if ((rc = check_nd(seqlens, "cache_seqlens", 1)) != DSV_OK) return rc;
    if ((seqlens->dtype != DSV_I32 && seqlens->dtype != DSV_I64) || seqlens->shape[0] != B || seqlens->stride[0] != 1)
      return fail(DSV_ERR_INVALID, "cache_seqlens must be a contiguous int32|int64 [B] tensor");
  }
  if (present(lse)) {
    if ((rc = check_nd(lse, "lse", 3)) != DSV_OK) return rc;
    if (lse->dtype != DSV_F32 || lse->shape[0] != B || lse->shape[1] != H || lse->shape[2] != M)
      return fail(DSV_ERR_INVALID, "lse must be float32 [B, H, M]");
  }
  const Plan p = make_plan(B, M, H, Hk, D, n_keys, 0, false);
  if ((rc = check_ws(p, workspace, workspace_bytes)) != DSV_OK) return rc;

  AttnArgs a{};
  fill_common(a, q, Hk, p, workspace);
  a.pre = dense_src(k, v, 0);
  a.n_pre = n_keys;
  if (present(seqlens)) {
    a.seqlens = seqlens->data;
    a.seqlens_i64 = seqlens->dtype == DSV_I64;
  }
  a.causal = causal != 0;
  MergeArgs m{};
  fill_merge(m, a, out, (int)D);
  if (present(lse)) {
    m.lse = static_cast<float*>(lse->data);
    m.l_sb = lse->stride[0];
    m.l_sh = lse->stride[1];
    m.l_sm = lse->stride[2];
  }
  AttnExtents ex = common_extents(q, out, workspace, p);
  ex.pre_k = extent_of("k", k);
  ex.pre_v = extent_of("v", v);
  ex.lse = extent_of("lse", lse);
  return run(a, m, q->dtype, (int)D, false, static_cast<hipStream_t>(stream), ex);
}

}  // namespace

extern "C" {

int dsv_prefix_attention_forward(const dsv_tensor* q, const dsv_tensor* k, const dsv_tensor* v, int64_t n_keys,
                                 dsv_tensor* out, dsv_tensor* lse, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  if (!present(lse)) return fail(DSV_ERR_INVALID, "lse must be float32 [B, H, M]");
  return prefix_attention(q, k, v, nullptr, n_keys, 0, out, lse, workspace, workspace_bytes, stream);
}

int dsv_flash_attn_with_kvcache(const dsv_tensor* q, const dsv_tensor* k_cache, const dsv_tensor* v_cache,
                                const dsv_tensor* cache_seqlens, int64_t n_keys, int causal, dsv_tensor* out,
                                dsv_tensor* softmax_lse, void* workspace, size_t workspace_bytes, void* stream) {
  return prefix_attention(q, k_cache, v_cache, cache_seqlens, n_keys, causal, out, softmax_lse, workspace,
                          workspace_bytes, stream);
}

int dsv_tree_attention_forward(const dsv_tensor* q, const dsv_tensor* k, const dsv_tensor* v,
                               const dsv_tensor* tree_mask, const dsv_tensor* prefix_lse, dsv_tensor* current_out,
                               dsv_tensor* weight, dsv_tensor* tree_lse, void* workspace, size_t workspace_bytes,
                               void* stream) {
  int rc;
  if ((rc = check_q_out(q, current_out)) != DSV_OK) return rc;
  if ((rc = check_kv_dense(k, v, q, "key_states", "value_states")) != DSV_OK) return rc;
  const int64_t B = q->shape[0], M = q->shape[1], H = q->shape[2], D = q->shape[3], Hk = k->shape[2];
  if (k->shape[1] != M) return fail(DSV_ERR_INVALID, "key/value must be the post-cache block of M rows");
  if (M > dsv::kTreeMaxM) return fail(DSV_ERR_UNSUPPORTED, "tree blocks larger than %d nodes are not supported", dsv::kTreeMaxM);
  if (tree_mask == nullptr || (tree_mask->ndim != 3 && tree_mask->ndim != 4))
    return fail(DSV_ERR_INVALID, "tree_mask must be [B, 1, T, T] or [B, T, T]");
  if ((rc = check_nd(tree_mask, "tree_mask", tree_mask->ndim)) != DSV_OK) return rc;
  const int nd = tree_mask->ndim;
  const int64_t T0 = tree_mask->shape[nd - 2], T1 = tree_mask->shape[nd - 1];
  if (T0 < M || T1 < M) return fail(DSV_ERR_INVALID, "tree_mask is smaller than the M x M block");
  if (tree_mask->shape[0] != B && tree_mask->shape[0] != 1) return fail(DSV_ERR_INVALID, "tree_mask batch must be 1 or B");
  if ((rc = check_nd(prefix_lse, "prefix_lse", 3)) != DSV_OK) return rc;
  if (prefix_lse->dtype != DSV_F32 || prefix_lse->shape[0] != B || prefix_lse->shape[1] != H || prefix_lse->shape[2] != M)
    return fail(DSV_ERR_INVALID, "prefix_lse must be float32 viewed as [B, H, M]");
  if ((rc = check_nd(weight, "weight", 4)) != DSV_OK) return rc;
  if (weight->shape[0] != B || weight->shape[1] != M || weight->shape[2] != H || weight->shape[3] != 1)
    return fail(DSV_ERR_INVALID, "weight must be [B, M, H, 1]");
  if (weight->dtype != DSV_BF16 && weight->dtype != DSV_F16 && weight->dtype != DSV_F32)
    return fail(DSV_ERR_INVALID, "weight dtype must be bf16, f16 or f32");
  if (present(tree_lse)) {
    if ((rc = check_nd(tree_lse, "tree_lse", 3)) != DSV_OK) return rc;
    if (tree_lse->dtype != DSV_F32 || tree_lse->shape[0] != B || tree_lse->shape[1] != M || tree_lse->shape[2] != H)
      return fail(DSV_ERR_INVALID, "tree_lse must be float32 [B, M, H]");
  }
  const Plan p = make_plan(B, M, H, Hk, D, 0, 0, true);
  if ((rc = check_ws(p, workspace, workspace_bytes)) != DSV_OK) return rc;

  AttnArgs a{};
  fill_common(a, q, Hk, p, workspace);
  a.n_pre = 0;
  a.has_tree = 1;
  a.tree = dense_src(k, v, 0);
  const int64_t es = elem_size(tree_mask->dtype);
  const int64_t sb = tree_mask->shape[0] > 1 ? tree_mask->stride[0] : 0;
  const int64_t sm = tree_mask->stride[nd - 2], sn = tree_mask->stride[nd - 1];
  a.tmask = static_cast<const char*>(tree_mask->data) + ((T0 - M) * sm + (T1 - M) * sn) * es;
  a.tmask_dtype = tree_mask->dtype;
  a.tm_sb = sb;
  a.tm_sm = sm;
  a.tm_sn = sn;
  MergeArgs m{};
  fill_merge(m, a, current_out, (int)D);
  if (present(tree_lse)) {
    m.lse = static_cast<float*>(tree_lse->data);
    m.l_sb = tree_lse->stride[0];
    m.l_sm = tree_lse->stride[1];
    m.l_sh = tree_lse->stride[2];
  }
  m.plse = static_cast<const float*>(prefix_lse->data);
  m.p_sb = prefix_lse->stride[0];
  m.p_sh = prefix_lse->stride[1];
  m.p_sm = prefix_lse->stride[2];
  m.weight = weight->data;
  m.w_dtype = weight->dtype;
  m.w_sb = weight->stride[0];
  m.w_sm = weight->stride[1];
  m.w_sh = weight->stride[2];
  AttnExtents ex = common_extents(q, current_out, workspace, p);
  ex.tree_k = extent_of("key_states", k);
  ex.tree_v = extent_of("value_states", v);
  ex.tmask = extent_of("tree_mask", tree_mask);
  ex.lse = extent_of("tree_lse", tree_lse);
  ex.plse = extent_of("prefix_lse", prefix_lse);
  ex.weight = extent_of("weight", weight);
  return run(a, m, q->dtype, (int)D, false, static_cast<hipStream_t>(stream), ex);
}

int dsv_verify_bundle(const dsv_tensor* q, const dsv_tensor* k, const dsv_tensor* v, const dsv_tensor* mask,
                      dsv_tensor* out, dsv_tensor* lse, void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if ((rc = check_q_out(q, out)) != DSV_OK) return rc;
  if ((rc = check_kv_dense(k, v, q, "k", "v")) != DSV_OK) return rc;
  const int64_t B = q->shape[0], M = q->shape[1], H = q->shape[2], D = q->shape[3];
  const int64_t N = k->shape[1], Hk = k->shape[2];
  if ((rc = check_byte_mask(mask, B, M, "mask")) != DSV_OK) return rc;
  if ((rc = check_nd(lse, "lse", 3)) != DSV_OK) return rc;
  if (lse->dtype != DSV_F32 || lse->shape[0] != B || lse->shape[1] != M || lse->shape[2] != H)
    return fail(DSV_ERR_INVALID, "lse must be float32 [B, M, H]");
  const Plan p = make_plan(B, M, H, Hk, D, N, 0, false);
  if ((rc = check_ws(p, workspace, workspace_bytes)) != DSV_OK) return rc;

  AttnArgs a{};
  fill_common(a, q, Hk, p, workspace);
  a.pre = dense_src(k, v, 0);
  a.n_pre = N;
  a.dmask = static_cast<const uint8_t*>(mask->data);
  a.dm_sb = mask->shape[0] > 1 ? mask->stride[0] : 0;
  a.dm_sm = mask->stride[1];
  a.dm_sn = mask->stride[2];
  a.dm_n = mask->shape[2];
  MergeArgs m{};
  fill_merge(m, a, out, (int)D);
  m.lse = static_cast<float*>(lse->data);
  m.l_sb = lse->stride[0];
  m.l_sm = lse->stride[1];
  m.l_sh = lse->stride[2];
  AttnExtents ex = common_extents(q, out, workspace, p);
  ex.pre_k = extent_of("k", k);
  ex.pre_v = extent_of("v", v);
  ex.dmask = extent_of("mask", mask);
  ex.lse = extent_of("lse", lse);
  return run(a, m, q->dtype, (int)D, true, static_cast<hipStream_t>(stream), ex);
}

int dsv_verify_bundle_paged(const dsv_tensor* q, const dsv_tensor* kv_pages, const dsv_tensor* page_table,
                            int64_t layer_idx, const dsv_tensor* mask, dsv_tensor* out, dsv_tensor* lse,
                            void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if ((rc = check_q_out(q, out)) != DSV_OK) return rc;
  const int64_t B = q->shape[0], M = q->shape[1], H = q->shape[2], D = q->shape[3];
  KvSrc s{};
  int64_t ps = 0, Hk = 0, Dk = 0, cap = 0;
  if ((rc = paged_src(kv_pages, layer_idx, page_table, B, s, ps, Hk, Dk, cap)) != DSV_OK) return rc;
  if (kv_pages->dtype != q->dtype) return fail(DSV_ERR_INVALID, "q and kv_pages must share a dtype");
  if (Dk != D) return fail(DSV_ERR_INVALID, "kv_pages head_dim differs from q");
  if (H % Hk != 0) return fail(DSV_ERR_INVALID, "query heads must be a multiple of kv_pages heads");
  if ((rc = check_byte_mask(mask, B, M, "mask")) != DSV_OK) return rc;
  const int64_t N = mask->shape[2];
  if (N > cap) return fail(DSV_ERR_INVALID, "mask covers %lld tokens but the page table maps %lld", (long long)N, (long long)cap);
  if ((rc = check_nd(lse, "lse", 3)) != DSV_OK) return rc;
  if (lse->dtype != DSV_F32 || lse->shape[0] != B || lse->shape[1] != M || lse->shape[2] != H)
    return fail(DSV_ERR_INVALID, "lse must be float32 [B, M, H]");
  const Plan p = make_plan(B, M, H, Hk, D, N, ps, false);
  if ((rc = check_ws(p, workspace, workspace_bytes)) != DSV_OK) return rc;

  AttnArgs a{};
  fill_common(a, q, Hk, p, workspace);
  a.pre = s;
  a.n_pre = N;
  a.dmask = static_cast<const uint8_t*>(mask->data);
  a.dm_sb = mask->shape[0] > 1 ? mask->stride[0] : 0;
  a.dm_sm = mask->stride[1];
  a.dm_sn = mask->stride[2];
  a.dm_n = N;
  MergeArgs m{};
  fill_merge(m, a, out, (int)D);
  m.lse = static_cast<float*>(lse->data);
  m.l_sb = lse->stride[0];
  m.l_sm = lse->stride[1];
  m.l_sh = lse->stride[2];
  AttnExtents ex = common_extents(q, out, workspace, p);
  ex.pre_k = extent_raw("kv_pages[layer, 0]", s.k, s.k_bytes);
  ex.pre_v = extent_raw("kv_pages[layer, 1]", s.v, s.v_bytes);
  ex.pre_pt = extent_of("page_table", page_table);
  ex.dmask = extent_of("mask", mask);
  ex.lse = extent_of("lse", lse);
  return run(a, m, q->dtype, (int)D, true, static_cast<hipStream_t>(stream), ex);
}

}  // extern "C"

namespace {

// Scratch of the allocation-free tree verify: a file-scope device array, one
// copy per GPU for the life of the process.  The split plan fills the GPU's
// workgroup slots with (batch, KV head, row block, split) units and needs
// 2 * D + 8 bytes per (split, batch, KV head, query row), about
// slots x 256 rows x (2 * D + 8) bytes (17 MiB at D = 128 on 256 CUs) until
// the 16384-key cap on a split adds splits.  At D = 128, 8 KV heads, 256 CUs
// 32 MiB holds one tree of <= 64 nodes up to 512K prefix tokens, <= 128
// nodes up to 256K, <= 256 nodes up to 128K, and 8 trees of 64 nodes at 64K.
constexpr size_t kNoAllocScratchBytes = DSV_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;

// Per GPU: the scratch array's device address, and the guard that orders
// calls made on different streams: an event recorded after each call's
// kernels and the stream it was recorded on.  A call on another stream first
// makes its stream wait for that event, so two calls never use the array at
// the same time unless a caller hides them from the guard (graph capture,
// see dsv.h).
struct NoAllocDevice {
  void* scratch = nullptr;
  hipEvent_t done = nullptr;
  hipStream_t last = nullptr;
  bool used = false;
};
NoAllocDevice g_noalloc[kMaxDevices];

// Set-up, once per device with that device current: the scratch array's
// address (its name is a host-side stand-in and may not be passed to a
// kernel or a copy) and the guard's event.  Called with g_scratch_mu held.
int noalloc_device(NoAllocDevice** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(DSV_ERR_UNSUPPORTED, "device ordinal %d beyond %d", dev, kMaxDevices);
  NoAllocDevice& d = g_noalloc[dev];
  if (d.scratch == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (p == nullptr || (reinterpret_cast<uintptr_t>(p) & 255) != 0)
      return fail(DSV_ERR_HIP, "scratch array at an unusable address");
    e = hipEventCreateWithFlags(&d.done, hipEventDisableTiming);
    if (e != hipSuccess) return hip_fail(e, "hipEventCreateWithFlags (allocation-free entry point set-up)");
    d.scratch = p;
  }
  *out = &d;
  return DSV_OK;
}

int tree_verify_impl(const dsv_tensor* q, const dsv_tensor* k, const dsv_tensor* v, const dsv_tensor* page_table,
                     int64_t n_prefix, const dsv_tensor* parent, const dsv_tensor* row_perm, dsv_tensor* out,
                     dsv_tensor* lse, void* workspace, size_t workspace_bytes, bool noalloc, void* stream) {
  int rc;
  if ((rc = check_q_out(q, out)) != DSV_OK) return rc;
  const int64_t B = q->shape[0], M = q->shape[1], H = q->shape[2], D = q->shape[3];
  if (M > dsv::kTreeMaxM) return fail(DSV_ERR_UNSUPPORTED, "trees larger than %d nodes are not supported", dsv::kTreeMaxM);
  if (n_prefix < 0) return fail(DSV_ERR_INVALID, "n_prefix must be >= 0");
  KvSrc src{};
  int64_t Hk = 0, ps = 0, cap = 0;
  if (present(page_table)) {
    // k, v: [P, Hk, ps, D] page-pool halves.
    if ((rc = check_nd(k, "k_pages", 4)) != DSV_OK) return rc;
    if ((rc = check_nd(v, "v_pages", 4)) != DSV_OK) return rc;
    if ((rc = check_vec16(k, "k_pages")) != DSV_OK) return rc;
    if ((rc = check_vec16(v, "v_pages")) != DSV_OK) return rc;
    for (int i = 0; i < 4; ++i)
      if (k->shape[i] != v->shape[i]) return fail(DSV_ERR_INVALID, "k_pages and v_pages shapes differ");
    if (k->dtype != q->dtype || v->dtype != q->dtype) return fail(DSV_ERR_INVALID, "q and pages must share a dtype");
    if (k->shape[3] != D) return fail(DSV_ERR_INVALID, "page head_dim differs from q");
    ps = k->shape[2];
    const int sh = log2_exact(ps);
    if (sh < 0) return fail(DSV_ERR_UNSUPPORTED, "page_size %lld must be a power of two", (long long)ps);
    if ((rc = check_nd(page_table, "page_table", page_table->ndim)) != DSV_OK) return rc;
    if (page_table->ndim != 1 && page_table->ndim != 2) return fail(DSV_ERR_INVALID, "page_table must be 1-d or 2-d");
    if (page_table->dtype != DSV_I32 && page_table->dtype != DSV_I64)
      return fail(DSV_ERR_INVALID, "page_table must be int32 or int64");
    if (page_table->ndim == 2 && page_table->shape[0] != B && page_table->shape[0] != 1)
      return fail(DSV_ERR_INVALID, "page_table batch must be 1 or B");
    if (page_table->stride[page_table->ndim - 1] != 1) return fail(DSV_ERR_INVALID, "page_table innermost stride must be 1");
    Hk = k->shape[1];
    src.k = static_cast<const uint16_t*>(k->data);
    src.v = static_cast<const uint16_t*>(v->data);
    src.k_sp = k->stride[0];
    src.k_sh = k->stride[1];
    src.k_st = k->stride[2];
    src.v_sp = v->stride[0];
    src.v_sh = v->stride[1];
    src.v_st = v->stride[2];
    src.pt = page_table->data;
    src.pt_i64 = page_table->dtype == DSV_I64;
    src.ps_shift = sh;
    src.pt_sb = (page_table->ndim == 2 && page_table->shape[0] > 1) ? page_table->stride[0] : 0;
    src.n_phys = k->shape[0];
    src.k_bytes = span_bytes(k);
    src.v_bytes = span_bytes(v);
    cap = page_table->shape[page_table->ndim - 1] * ps;
  } else {
    if ((rc = check_kv_dense(k, v, q, "k_cache", "v_cache")) != DSV_OK) return rc;
    Hk = k->shape[2];
    src = dense_src(k, v, 0);
    cap = k->shape[1];
  }
  if (H % Hk != 0) return fail(DSV_ERR_INVALID, "query heads must be a multiple of key heads");
  if (n_prefix + M > cap)
    return fail(DSV_ERR_INVALID, "cache holds %lld tokens, n_prefix + M = %lld", (long long)cap, (long long)(n_prefix + M));
  if (parent == nullptr || (parent->ndim != 1 && parent->ndim != 2))
    return fail(DSV_ERR_INVALID, "parent must be [M] or [B, M]");
  if ((rc = check_nd(parent, "parent", parent->ndim)) != DSV_OK) return rc;
  if (parent->dtype != DSV_I32 && parent->dtype != DSV_I64) return fail(DSV_ERR_INVALID, "parent must be int32 or int64");
  if (parent->shape[parent->ndim - 1] != M) return fail(DSV_ERR_INVALID, "parent must have M entries per tree");
  if (parent->ndim == 2 && parent->shape[0] != B && parent->shape[0] != 1)
    return fail(DSV_ERR_INVALID, "parent batch must be 1 or B");
  if (present(row_perm)) {
    if ((rc = check_nd(row_perm, "row_perm", 1)) != DSV_OK) return rc;
    if (row_perm->dtype != DSV_I32 || row_perm->shape[0] != M || row_perm->stride[0] != 1)
      return fail(DSV_ERR_INVALID, "row_perm must be a contiguous int32 [M] permutation");
  }
  if (present(lse)) {
    if ((rc = check_nd(lse, "lse", 3)) != DSV_OK) return rc;
    if (lse->dtype != DSV_F32 || lse->shape[0] != B || lse->shape[1] != M || lse->shape[2] != H)
      return fail(DSV_ERR_INVALID, "lse must be float32 [B, M, H]");
  }
  const Plan p = make_plan(B, M, H, Hk, D, n_prefix, ps, true);
  // The allocation-free entry point holds g_scratch_mu from here to the end
  // of its launches, so that the guard's wait, the kernels and the record of
  // the guard's event are one step for other threads.
  std::unique_lock<std::mutex> lock(g_scratch_mu, std::defer_lock);
  NoAllocDevice* nad = nullptr;
  bool guard = false;
  if (noalloc) {
    if (p.total > kNoAllocScratchBytes)
      return fail(DSV_ERR_UNSUPPORTED,
                  "this shape needs %zu bytes of split scratch, above the %zu bytes of the allocation-free entry "
                  "point; use dsv_tree_verify with a workspace",
                  p.total, kNoAllocScratchBytes);
    lock.lock();
    if ((rc = noalloc_device(&nad)) != DSV_OK) return rc;
    workspace = nad->scratch;
    workspace_bytes = kNoAllocScratchBytes;
    // Under stream capture the guard stands aside: the captured kernels run
    // when the graph is replayed, in the order the caller gives the replays.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cs);
    if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
    guard = cs == hipStreamCaptureStatusNone && !g_dry_run;
  }
  if ((rc = check_ws(p, workspace, workspace_bytes)) != DSV_OK) return rc;

  AttnArgs a{};
  fill_common(a, q, Hk, p, workspace);
  a.pre = src;
  a.pre.key0 = 0;
  a.n_pre = n_prefix;
  a.has_tree = 1;
  a.tree = src;
  a.tree.key0 = n_prefix;
  a.tpar = parent->data;
  a.tpar_i64 = parent->dtype == DSV_I64;
  a.tpar_sb = (parent->ndim == 2 && parent->shape[0] > 1) ? parent->stride[0] : 0;
  a.tpar_sm = parent->stride[parent->ndim - 1];
  a.row_perm = present(row_perm) ? static_cast<const int32_t*>(row_perm->data) : nullptr;
  MergeArgs m{};
  fill_merge(m, a, out, (int)D);
  if (present(lse)) {
    m.lse = static_cast<float*>(lse->data);
    m.l_sb = lse->stride[0];
    m.l_sm = lse->stride[1];
    m.l_sh = lse->stride[2];
  }
  AttnExtents ex = common_extents(q, out, workspace, p);
  ex.pre_k = ex.tree_k = extent_raw("k", src.k, src.k_bytes);
  ex.pre_v = ex.tree_v = extent_raw("v", src.v, src.v_bytes);
  ex.pre_pt = ex.tree_pt = extent_of("page_table", page_table);
  ex.tpar = extent_of("parent", parent);
  ex.perm = extent_of("row_perm", row_perm);
  ex.lse = extent_of("lse", lse);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (guard && nad->used && nad->last != st) {
    // The previous call ran on another stream: this one starts after it.
    const hipError_t e = hipStreamWaitEvent(st, nad->done, 0);
    if (e != hipSuccess) return hip_fail(e, "hipStreamWaitEvent (allocation-free entry point guard)");
  }
  rc = run(a, m, q->dtype, (int)D, false, st, ex);
  if (rc == DSV_OK && guard) {
    const hipError_t e = hipEventRecord(nad->done, st);
    if (e != hipSuccess) return hip_fail(e, "hipEventRecord (allocation-free entry point guard)");
    nad->last = st;
    nad->used = true;
  }
  return rc;
}

}  // namespace

extern "C" {

int dsv_tree_verify(const dsv_tensor* q, const dsv_tensor* k, const dsv_tensor* v, const dsv_tensor* page_table,
                    int64_t n_prefix, const dsv_tensor* parent, const dsv_tensor* row_perm, dsv_tensor* out,
                    dsv_tensor* lse, void* workspace, size_t workspace_bytes, void* stream) {
  return tree_verify_impl(q, k, v, page_table, n_prefix, parent, row_perm, out, lse, workspace, workspace_bytes,
                          false, stream);
}

int dsv_tree_verify_noalloc(const dsv_tensor* q, const dsv_tensor* k, const dsv_tensor* v,
                            const dsv_tensor* page_table, int64_t n_prefix, const dsv_tensor* parent,
                            const dsv_tensor* row_perm, dsv_tensor* out, dsv_tensor* lse, void* stream) {
  return tree_verify_impl(q, k, v, page_table, n_prefix, parent, row_perm, out, lse, nullptr, 0, true, stream);
}

// ----------------------------------------------------------------------------
// Acceptance
// ----------------------------------------------------------------------------

size_t dsv_accept_workspace_bytes(int64_t T, int64_t M, int64_t V) {
  if (T <= 0 || M <= 0 || V <= 0) return 0;
  const size_t rows = (size_t)T * M * dsv::accept_max_chunks(V);
  // per (row, range) statistics, the typical sums, and per row the sampling
  // mode's kept-set bounds
  return align_up(rows * 16, 256) + align_up(rows * 4, 256) + align_up((size_t)T * M * 16, 256);
}

int dsv_kv_append(const dsv_tensor* k, const dsv_tensor* v, const dsv_tensor* cos, const dsv_tensor* sin,
                  dsv_tensor* k_dst, dsv_tensor* v_dst, const dsv_tensor* page_table, int64_t start,
                  const dsv_tensor* q, dsv_tensor* q_out, void* stream) {
  int rc;
  // A [lead..., X, Y, D] operand with an optional leading 1: the last three dims.
  auto last3 = [&](const dsv_tensor* t, const char* name, int64_t s[3], int64_t st[3]) -> int {
    int r;
    if (t == nullptr || (t->ndim != 3 && t->ndim != 4)) return fail(DSV_ERR_INVALID, "%s must be 3-d or [1, ...] 4-d", name);
    if ((r = check_nd(t, name, t->ndim)) != DSV_OK) return r;
    if (t->ndim == 4 && t->shape[0] != 1) return fail(DSV_ERR_INVALID, "%s leading dimension must be 1", name);
    const int o = t->ndim - 3;
    for (int x = 0; x < 3; ++x) {
      s[x] = t->shape[o + x];
      st[x] = t->stride[o + x];
    }
    if (st[2] != 1) return fail(DSV_ERR_INVALID, "%s innermost stride must be 1", name);
    if ((reinterpret_cast<uintptr_t>(t->data) & 15) != 0 || (st[0] * 2) % 16 != 0 || (st[1] * 2) % 16 != 0)
      return fail(DSV_ERR_INVALID, "%s rows must be 16-byte aligned", name);
    return DSV_OK;
  };
  int64_t ks[3], kst[3], vs[3], vst[3];
  if ((rc = last3(k, "k", ks, kst)) != DSV_OK) return rc;
  if ((rc = last3(v, "v", vs, vst)) != DSV_OK) return rc;
  if (k->dtype != DSV_BF16 && k->dtype != DSV_F16) return fail(DSV_ERR_INVALID, "k must be bf16 or f16");
  if (v->dtype != k->dtype) return fail(DSV_ERR_INVALID, "k and v must share a dtype");
  const int64_t M = ks[0], Hk = ks[1], D = ks[2];
  if (vs[0] != M || vs[1] != Hk || vs[2] != D) return fail(DSV_ERR_INVALID, "v must match k");
  if (M < 1 || Hk < 1) return fail(DSV_ERR_INVALID, "empty k");
  if (D % 16 != 0) return fail(DSV_ERR_UNSUPPORTED, "head_dim %lld must be a multiple of 16", (long long)D);
  // The kernel's counts are 32-bit and its grid covers one thread per
  // 16-element chunk of every row.
  if (M > (1 << 24) || Hk > (1 << 16) || D > (1 << 12))
    return fail(DSV_ERR_UNSUPPORTED, "k is too large (M <= 2^24, key heads <= 65536, head_dim <= 4096)");
  if (start < 0) return fail(DSV_ERR_INVALID, "start must be >= 0");

  dsv::AppendArgs a{};
  a.f16 = k->dtype == DSV_F16;
  a.M = (int)M;
  a.Hk = (int)Hk;
  a.D = (int)D;
  a.start = start;
  a.k = static_cast<const uint16_t*>(k->data);
  a.k_sm = kst[0];
  a.k_sh = kst[1];
  a.v = static_cast<const uint16_t*>(v->data);
  a.v_sm = vst[0];
  a.v_sh = vst[1];
  if (present(cos) || present(sin)) {
    if (!present(cos) || !present(sin)) return fail(DSV_ERR_INVALID, "cos and sin go together");
    for (const dsv_tensor* t : {cos, sin}) {
      const char* nm = t == cos ? "cos" : "sin";
      if (t->ndim != 2 && t->ndim != 3) return fail(DSV_ERR_INVALID, "%s must be [M, D] or [1, M, D]", nm);
      if ((rc = check_nd(t, nm, t->ndim)) != DSV_OK) return rc;
      const int o = t->ndim - 2;
      if ((t->ndim == 3 && t->shape[0] != 1) || t->shape[o] != M || t->shape[o + 1] != D || t->stride[o + 1] != 1)
        return fail(DSV_ERR_INVALID, "%s must be [M, D] with innermost stride 1", nm);
      if (t->dtype != k->dtype) return fail(DSV_ERR_INVALID, "%s must have the dtype of k", nm);
      if ((reinterpret_cast<uintptr_t>(t->data) & 15) != 0 || (t->stride[o] * 2) % 16 != 0)
        return fail(DSV_ERR_INVALID, "%s rows must be 16-byte aligned", nm);
    }
    a.cos = static_cast<const uint16_t*>(cos->data);
    a.cs_m = cos->stride[cos->ndim - 2];
    a.sin = static_cast<const uint16_t*>(sin->data);
    a.sn_m = sin->stride[sin->ndim - 2];
  }
  if (present(q) || present(q_out)) {
    int64_t qs[3], qst[3], os[3], ost[3];
    if (!present(q) || !present(q_out)) return fail(DSV_ERR_INVALID, "q and q_out go together");
    if ((rc = last3(q, "q", qs, qst)) != DSV_OK) return rc;
    if ((rc = last3(q_out, "q_out", os, ost)) != DSV_OK) return rc;
    if (q->dtype != k->dtype || q_out->dtype != k->dtype) return fail(DSV_ERR_INVALID, "q and q_out must have the dtype of k");
    if (qs[0] != M || qs[2] != D || os[0] != M || os[1] != qs[1] || os[2] != D)
      return fail(DSV_ERR_INVALID, "q and q_out must be [M, H, D]");
    if (qs[1] > (1 << 16)) return fail(DSV_ERR_UNSUPPORTED, "q has more than 65536 heads");
    a.H = (int)qs[1];
    a.q = static_cast<const uint16_t*>(q->data);
    a.q_sm = qst[0];
    a.q_sh = qst[1];
    a.q_out = static_cast<uint16_t*>(q_out->data);
    a.qo_sm = ost[0];
    a.qo_sh = ost[1];
  }
  if ((2 * M * Hk + (int64_t)a.H * M) * (D / 16) > ((int64_t)1 << 31))
    return fail(DSV_ERR_UNSUPPORTED, "k, v and q hold more than 2^31 16-element chunks");
  for (dsv_tensor* t : {k_dst, v_dst}) {
    const char* nm = t == k_dst ? "k_dst" : "v_dst";
    if (t == nullptr || t->data == nullptr) return fail(DSV_ERR_INVALID, "%s missing", nm);
    if (t->dtype != k->dtype) return fail(DSV_ERR_INVALID, "%s must have the dtype of k", nm);
    if ((reinterpret_cast<uintptr_t>(t->data) & 15) != 0) return fail(DSV_ERR_INVALID, "%s must be 16-byte aligned", nm);
  }
  if (present(page_table)) {
    if ((rc = check_nd(page_table, "page_table", 1)) != DSV_OK) return rc;
    if (page_table->dtype != DSV_I32 && page_table->dtype != DSV_I64)
      return fail(DSV_ERR_INVALID, "page_table must be int32 or int64");
    if (page_table->stride[0] != 1) return fail(DSV_ERR_INVALID, "page_table stride must be 1");
    int64_t ps = 0, P = 0;
    for (dsv_tensor* t : {k_dst, v_dst}) {
      const char* nm = t == k_dst ? "k_dst" : "v_dst";
      if ((rc = check_nd(t, nm, 4)) != DSV_OK) return rc;
      if (t->shape[1] != Hk || t->shape[3] != D || t->stride[3] != 1)
        return fail(DSV_ERR_INVALID, "%s must be [P, Hk, page, D] with innermost stride 1", nm);
      for (int x = 0; x < 3; ++x)
        if ((t->stride[x] * 2) % 16 != 0) return fail(DSV_ERR_INVALID, "%s rows must be 16-byte aligned", nm);
      if (t == k_dst) {
        ps = t->shape[2];
        P = t->shape[0];
      } else if (t->shape[2] != ps || t->shape[0] != P) {
        return fail(DSV_ERR_INVALID, "k_dst and v_dst must have the same pages");
      }
    }
    const int sh = log2_exact(ps);
    if (sh < 0) return fail(DSV_ERR_UNSUPPORTED, "page size must be a power of two");
    if (start + M > page_table->shape[0] * ps) return fail(DSV_ERR_INVALID, "tokens [start, start + M) exceed the page table");
    a.pt = page_table->data;
    a.pt_i64 = page_table->dtype == DSV_I64;
    a.ps_shift = sh;
    a.n_phys = P;
    a.k_dst = static_cast<uint16_t*>(k_dst->data);
    a.kd_sp = k_dst->stride[0];
    a.kd_sh = k_dst->stride[1];
    a.kd_st = k_dst->stride[2];
    a.v_dst = static_cast<uint16_t*>(v_dst->data);
    a.vd_sp = v_dst->stride[0];
    a.vd_sh = v_dst->stride[1];
    a.vd_st = v_dst->stride[2];
  } else {
    int64_t S = -1;
    for (dsv_tensor* t : {k_dst, v_dst}) {
      const char* nm = t == k_dst ? "k_dst" : "v_dst";
      int64_t s3[3], st3[3];
      if ((rc = last3(t, nm, s3, st3)) != DSV_OK) return rc;
      if (s3[0] != Hk || s3[2] != D) return fail(DSV_ERR_INVALID, "%s must be [Hk, S, D]", nm);
      if (S >= 0 && s3[1] != S) return fail(DSV_ERR_INVALID, "k_dst and v_dst must hold the same tokens");
      S = s3[1];
      if (t == k_dst) {
        a.k_dst = static_cast<uint16_t*>(t->data);
        a.kd_sh = st3[0];
        a.kd_st = st3[1];
      } else {
        a.v_dst = static_cast<uint16_t*>(t->data);
        a.vd_sh = st3[0];
        a.vd_st = st3[1];
      }
    }
    if (start + M > S) return fail(DSV_ERR_INVALID, "tokens [start, start + M) exceed the cache");
  }
  // Aliasing: a thread reads one row's chunk pair and writes the same pair of
  // the destination row, so a row rotated in place is safe; any other overlap
  // of a read operand with a written one would let one thread overwrite what
  // another still has to read.  Exact in place: q_out == q, or (dense cache)
  // k / v already sitting in the destination's tree slots.
  {
    struct Span {
      const char* name;
      uintptr_t lo, hi;
    };
    auto span = [&](const char* nm, const dsv_tensor* t) {
      const uintptr_t lo = present(t) ? reinterpret_cast<uintptr_t>(t->data) : 0;
      return Span{nm, lo, present(t) ? lo + (uintptr_t)span_bytes(t) : lo};
    };
    auto in_place = [&](const dsv_tensor* src, const dsv_tensor* dst, int64_t dst_st, int64_t dst_sh) {
      if (!present(src) || !present(dst)) return false;
      const int o = src->ndim - 3;
      if (dst == q_out)
        return src->data == dst->data && src->stride[o] == dst->stride[dst->ndim - 3] &&
               src->stride[o + 1] == dst->stride[dst->ndim - 2];
      if (present(page_table)) return false;
      return reinterpret_cast<uintptr_t>(src->data) == reinterpret_cast<uintptr_t>(dst->data) + (uintptr_t)(start * dst_st * 2) &&
             src->stride[o] == dst_st && src->stride[o + 1] == dst_sh;
    };
    const dsv_tensor* srcs[5] = {k, v, q, cos, sin};
    const char* snames[5] = {"k", "v", "q", "cos", "sin"};
    const dsv_tensor* dsts[3] = {k_dst, v_dst, q_out};
    const char* dnames[3] = {"k_dst", "v_dst", "q_out"};
    const int64_t dst_st[3] = {a.kd_st, a.vd_st, 0}, dst_sh[3] = {a.kd_sh, a.vd_sh, 0};
    for (int si = 0; si < 5; ++si) {
      const Span s = span(snames[si], srcs[si]);
      if (s.hi == s.lo) continue;
      for (int di = 0; di < 3; ++di) {
        const Span d = span(dnames[di], dsts[di]);
        if (d.hi == d.lo || s.hi <= d.lo || d.hi <= s.lo) continue;
        if (si == di && in_place(srcs[si], dsts[di], dst_st[di], dst_sh[di])) continue;
        return fail(DSV_ERR_INVALID, "%s overlaps %s: inputs may not alias an output except row for row in place",
                    s.name, d.name);
      }
    }
    for (int i = 0; i < 3; ++i)
      for (int j = i + 1; j < 3; ++j) {
        const Span x = span(dnames[i], dsts[i]), y = span(dnames[j], dsts[j]);
        if (x.hi > x.lo && y.hi > y.lo && x.lo < y.hi && y.lo < x.hi)
          return fail(DSV_ERR_INVALID, "%s overlaps %s: outputs may not alias each other", x.name, y.name);
      }
  }
  if (g_dry_run) return DSV_OK;
  const hipError_t e = dsv::launch_append(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "kv append launch");
  return DSV_OK;
}

int dsv_kv_commit(const dsv_tensor* kv, const dsv_tensor* page_table, int64_t start, const dsv_tensor* path,
                  const dsv_tensor* info, int64_t tree, void* stream) {
  int rc;
  if (kv == nullptr || kv->ndim < 2 || kv->ndim > 6) return fail(DSV_ERR_INVALID, "kv must have 2..6 dimensions");
  if ((rc = check_nd(kv, "kv", kv->ndim)) != DSV_OK) return rc;
  if (kv->dtype != DSV_BF16 && kv->dtype != DSV_F16 && kv->dtype != DSV_F32)
    return fail(DSV_ERR_INVALID, "kv must be bf16, f16 or f32");
  const int nd = kv->ndim;
  const int esize = kv->dtype == DSV_F32 ? 4 : 2;
  if (kv->stride[nd - 1] != 1) return fail(DSV_ERR_INVALID, "kv innermost stride must be 1");
  const int64_t D = kv->shape[nd - 1];
  if ((D * esize) % 16 != 0) return fail(DSV_ERR_UNSUPPORTED, "token rows must be a multiple of 16 bytes");
  if ((reinterpret_cast<uintptr_t>(kv->data) & 15) != 0) return fail(DSV_ERR_INVALID, "kv must be 16-byte aligned");
  for (int d = 0; d < nd - 1; ++d)
    if ((kv->stride[d] * esize) % 16 != 0) return fail(DSV_ERR_INVALID, "kv strides must keep token rows 16-byte aligned");
  if (path == nullptr || (path->ndim != 1 && path->ndim != 2)) return fail(DSV_ERR_INVALID, "path must be [M] or [T, M]");
  if ((rc = check_nd(path, "path", path->ndim)) != DSV_OK) return rc;
  if (info == nullptr || (info->ndim != 1 && info->ndim != 2)) return fail(DSV_ERR_INVALID, "info must be [4] or [T, 4]");
  if ((rc = check_nd(info, "info", info->ndim)) != DSV_OK) return rc;
  if (path->dtype != DSV_I64 || info->dtype != DSV_I64) return fail(DSV_ERR_INVALID, "path and info must be int64");
  if (path->stride[path->ndim - 1] != 1 || info->stride[info->ndim - 1] != 1)
    return fail(DSV_ERR_INVALID, "path and info innermost stride must be 1");
  if (info->shape[info->ndim - 1] < 4) return fail(DSV_ERR_INVALID, "info rows must hold 4 entries");
  const int64_t T = path->ndim == 2 ? path->shape[0] : 1;
  if ((info->ndim == 2 ? info->shape[0] : 1) != T) return fail(DSV_ERR_INVALID, "path and info must hold the same trees");
  if (tree < 0 || tree >= T) return fail(DSV_ERR_INVALID, "tree %lld out of range", (long long)tree);
  const int64_t M = path->shape[path->ndim - 1];
  if (M < 1) return fail(DSV_ERR_INVALID, "path must hold at least one node");
  if (M * (D * esize / 16) > (int64_t)dsv::kCommitThreads * dsv::kCommitChunks)
    return fail(DSV_ERR_UNSUPPORTED, "M * row bytes above %d KiB", dsv::kCommitThreads * dsv::kCommitChunks / 64);
  if (start < 0) return fail(DSV_ERR_INVALID, "start must be >= 0");

  dsv::CommitArgs c{};
  c.data = kv->data;
  c.esize = esize;
  c.D = (int)D;
  c.start = start;
  c.M = (int)M;
  c.path = static_cast<const int64_t*>(path->data) + (path->ndim == 2 ? tree * path->stride[0] : 0);
  c.info = static_cast<const int64_t*>(info->data) + (info->ndim == 2 ? tree * info->stride[0] : 0);
  if (present(page_table)) {
    if (nd != 6) return fail(DSV_ERR_INVALID, "a paged kv must be [L, 2, P, Hk, page, D]");
    if ((rc = check_nd(page_table, "page_table", 1)) != DSV_OK) return rc;
    if (page_table->dtype != DSV_I32 && page_table->dtype != DSV_I64)
      return fail(DSV_ERR_INVALID, "page_table must be int32 or int64");
    if (page_table->stride[0] != 1) return fail(DSV_ERR_INVALID, "page_table stride must be 1");
    const int sh = log2_exact(kv->shape[4]);
    if (sh < 0) return fail(DSV_ERR_UNSUPPORTED, "page size must be a power of two");
    if (start + M > page_table->shape[0] * kv->shape[4])
      return fail(DSV_ERR_INVALID, "tokens [start, start + M) exceed the page table");
    c.nlead = 3;
    const int lead[3] = {0, 1, 3};
    c.rows = 1;
    for (int x = 0; x < 3; ++x) {
      c.lead_shape[x] = kv->shape[lead[x]];
      c.lead_stride[x] = kv->stride[lead[x]];
      c.rows *= kv->shape[lead[x]];
    }
    c.pt = page_table->data;
    c.pt_i64 = page_table->dtype == DSV_I64;
    c.ps_shift = sh;
    c.page_stride = kv->stride[2];
    c.n_phys = kv->shape[2];
    c.tok_stride = kv->stride[4];
  } else {
    if (nd < 3) return fail(DSV_ERR_INVALID, "a dense kv must be [..., S, D] with at least one leading dimension");
    if (start + M > kv->shape[nd - 2]) return fail(DSV_ERR_INVALID, "tokens [start, start + M) exceed the cache");
    c.nlead = nd - 2;
    c.rows = 1;
    for (int x = 0; x < nd - 2; ++x) {
      c.lead_shape[x] = kv->shape[x];
      c.lead_stride[x] = kv->stride[x];
      c.rows *= kv->shape[x];
    }
    c.tok_stride = kv->stride[nd - 2];
  }
  if (g_dry_run) return DSV_OK;
  const hipError_t e = dsv::launch_commit(c, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "kv commit launch");
  return DSV_OK;
}

int dsv_bundle_order(const dsv_tensor* parent, int64_t bundle_size, int64_t num_bundles, int64_t max_bundles,
                     dsv_tensor* perm, dsv_tensor* bundle_of, void* stream) {
  int rc;
  if (parent == nullptr || (parent->ndim != 1 && parent->ndim != 2)) return fail(DSV_ERR_INVALID, "parent must be [M] or [B, M]");
  if ((rc = check_nd(parent, "parent", parent->ndim)) != DSV_OK) return rc;
  if (parent->dtype != DSV_I32 && parent->dtype != DSV_I64) return fail(DSV_ERR_INVALID, "parent must be int32 or int64");
  const int nd = parent->ndim;
  const int64_t B = nd == 2 ? parent->shape[0] : 1, M = parent->shape[nd - 1];
  if (M < 1 || M > dsv::kBundleMaxNodes)
    return fail(DSV_ERR_UNSUPPORTED, "trees of %lld nodes are not supported (1..%d)", (long long)M, dsv::kBundleMaxNodes);
  if (B < 1 || B > 0x7fffffff) return fail(DSV_ERR_INVALID, "batch size out of range");
  if (num_bundles < 0 || num_bundles > 0x7fffffff) return fail(DSV_ERR_INVALID, "num_bundles must be >= 0");
  if (num_bundles == 0 && (bundle_size < 1 || bundle_size > 0x7fffffff))
    return fail(DSV_ERR_INVALID, "bundle_size must be >= 1");
  for (dsv_tensor* t : {perm, bundle_of}) {
    const char* nm = t == perm ? "perm" : "bundle_of";
    if (t == bundle_of && !present(t)) continue;
    if (t == nullptr || t->ndim != nd) return fail(DSV_ERR_INVALID, "%s must have the shape of parent", nm);
    if ((rc = check_nd(t, nm, nd)) != DSV_OK) return rc;
    if (t->dtype != DSV_I32) return fail(DSV_ERR_INVALID, "%s must be int32", nm);
    if (t->shape[nd - 1] != M || (nd == 2 && t->shape[0] != B)) return fail(DSV_ERR_INVALID, "%s must have the shape of parent", nm);
    if (t->stride[nd - 1] != 1 || (nd == 2 && B > 1 && t->stride[0] != M)) return fail(DSV_ERR_INVALID, "%s must be contiguous", nm);
  }
  dsv::BundleArgs a{};
  a.B = (int)B;
  a.M = (int)M;
  a.parent = parent->data;
  a.p_i64 = parent->dtype == DSV_I64;
  a.p_st = nd == 2 ? parent->stride[0] : 0;
  a.p_sm = parent->stride[nd - 1];
  a.bundle_size = num_bundles > 0 ? 1 : (int)bundle_size;
  a.num_bundles = (int)num_bundles;
  // The scheduler stops once it holds max_bundles bundles, checked after each
  // one is added: at least one bundle is always emitted.
  a.max_bundles = (int)std::min<int64_t>(std::max<int64_t>(max_bundles, 1), 0x7fffffff);
  a.perm = static_cast<int32_t*>(perm->data);
  a.bundle_of = present(bundle_of) ? static_cast<int32_t*>(bundle_of->data) : nullptr;
  if (g_dry_run) return DSV_OK;
  const hipError_t e = dsv::launch_bundle_order(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "bundle order launch");
  return DSV_OK;
}

}  // extern "C"

// Validation and arguments shared by both acceptance entry points: tree
// shape (T, M), vocabulary V, the tree tensors and the outputs.
static int accept_common(int mode, int64_t T, int64_t M, int64_t V, const dsv_tensor* draft,
                         const dsv_tensor* parent, const dsv_tensor* pos, int64_t max_hops, float temperature,
                         float posterior_threshold, float posterior_alpha, dsv_tensor* out_path,
                         dsv_tensor* out_tokens, dsv_tensor* out_info, dsv_tensor* out_next, dsv::AcceptArgs& a) {
  int rc;
  if (M < 1 || M > 1024) return fail(DSV_ERR_UNSUPPORTED, "trees of %lld nodes are not supported (1..1024)", (long long)M);
  if (T < 1 || T > (1 << 20)) return fail(DSV_ERR_INVALID, "tree count %lld out of range (1..2^20)", (long long)T);
  if (V < 1 || V > 0x7fffffff) return fail(DSV_ERR_INVALID, "vocab size out of range");
  if ((rc = check_nd(draft, "draft", 2)) != DSV_OK) return rc;
  if (draft->dtype != DSV_I64 || draft->shape[0] != T || draft->shape[1] != M)
    return fail(DSV_ERR_INVALID, "draft must be int64 [T, M]");
  // A root-only tree (M == 1) has an empty parent tensor, possibly without
  // storage; nothing reads it then.
  if (M > 1) {
    if ((rc = check_nd(parent, "parent", 2)) != DSV_OK) return rc;
  } else if (parent == nullptr || parent->ndim != 2) {
    return fail(DSV_ERR_INVALID, "parent must be int64 [T, M-1]");
  }
  if (parent->dtype != DSV_I64 || parent->shape[0] != T || parent->shape[1] != M - 1)
    return fail(DSV_ERR_INVALID, "parent must be int64 [T, M-1]");
  if (pos == nullptr || (pos->ndim != 1 && pos->ndim != 2)) return fail(DSV_ERR_INVALID, "pos must be [M] or [T, M]");
  if ((rc = check_nd(pos, "pos", pos->ndim)) != DSV_OK) return rc;
  if (pos->dtype != DSV_I64 || pos->shape[pos->ndim - 1] != M) return fail(DSV_ERR_INVALID, "pos must be int64 with M entries");
  if (pos->ndim == 2 && pos->shape[0] != T && pos->shape[0] != 1) return fail(DSV_ERR_INVALID, "pos batch must be 1 or T");
  if (max_hops < 0) return fail(DSV_ERR_INVALID, "max_hops must be >= 0");
  if (mode == DSV_ACCEPT_TYPICAL && !(temperature > 0.f)) return fail(DSV_ERR_INVALID, "temperature must be > 0");
  auto chk_out = [&](const dsv_tensor* t, const char* name, int64_t cols) -> int {
    int r;
    if ((r = check_nd(t, name, 2)) != DSV_OK) return r;
    if (t->dtype != DSV_I64 || t->shape[0] != T || t->shape[1] != cols || t->stride[1] != 1)
      return fail(DSV_ERR_INVALID, "%s must be contiguous int64 [T, %lld]", name, (long long)cols);
    return DSV_OK;
  };
  if ((rc = chk_out(out_path, "out_path", M)) != DSV_OK) return rc;
  if ((rc = chk_out(out_tokens, "out_tokens", M)) != DSV_OK) return rc;
  if ((rc = chk_out(out_info, "out_info", 4)) != DSV_OK) return rc;
  if (present(out_next) && (rc = chk_out(out_next, "out_next", M)) != DSV_OK) return rc;

  a.mode = mode;
  a.T = (int)T;
  a.M = (int)M;
  a.V = V;
  a.draft = static_cast<const int64_t*>(draft->data);
  a.d_st = draft->stride[0];
  a.d_sm = draft->stride[1];
  a.parent = static_cast<const int64_t*>(parent->data);
  a.p_st = parent->stride[0];
  a.p_sm = parent->stride[1];
  a.pos = static_cast<const int64_t*>(pos->data);
  a.pos_st = (pos->ndim == 2 && pos->shape[0] > 1) ? pos->stride[0] : 0;
  a.pos_sm = pos->stride[pos->ndim - 1];
  a.max_hops = (int)std::min<int64_t>(max_hops, 1 << 20);
  a.inv_temp = mode == DSV_ACCEPT_TYPICAL ? 1.f / temperature : 1.f;
  a.temperature = mode == DSV_ACCEPT_TYPICAL ? temperature : 1.f;  // the typical re-check's T
  a.eps = posterior_threshold;
  a.alpha = posterior_alpha;
  a.out_path = static_cast<int64_t*>(out_path->data);
  a.op_st = out_path->stride[0];
  a.out_tok = static_cast<int64_t*>(out_tokens->data);
  a.ot_st = out_tokens->stride[0];
  a.out_info = static_cast<int64_t*>(out_info->data);
  a.oi_st = out_info->stride[0];
  if (present(out_next)) {
    a.out_next = static_cast<int64_t*>(out_next->data);
    a.on_st = out_next->stride[0];
  }
  return DSV_OK;
}

extern "C" {

int dsv_tree_accept(int mode, const dsv_tensor* logits, const dsv_tensor* draft, const dsv_tensor* parent,
                    const dsv_tensor* pos, int64_t max_hops, float temperature, float posterior_threshold,
                    float posterior_alpha, dsv_tensor* out_path, dsv_tensor* out_tokens, dsv_tensor* out_info,
                    dsv_tensor* out_next, void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if (mode != DSV_ACCEPT_GREEDY && mode != DSV_ACCEPT_TYPICAL) return fail(DSV_ERR_INVALID, "unknown acceptance mode %d", mode);
  if ((rc = check_nd(logits, "logits", 3)) != DSV_OK) return rc;
  if (logits->dtype != DSV_BF16 && logits->dtype != DSV_F16 && logits->dtype != DSV_F32)
    return fail(DSV_ERR_INVALID, "logits must be bf16, f16 or f32");
  if (logits->stride[2] != 1) return fail(DSV_ERR_INVALID, "logits vocab stride must be 1");
  const int64_t T = logits->shape[0], M = logits->shape[1], V = logits->shape[2];
  AcceptArgs a{};
  if ((rc = accept_common(mode, T, M, V, draft, parent, pos, max_hops, temperature, posterior_threshold,
                          posterior_alpha, out_path, out_tokens, out_info, out_next, a)) != DSV_OK)
    return rc;
  const size_t need = dsv_accept_workspace_bytes(T, M, V);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(DSV_ERR_WORKSPACE, "workspace of %zu bytes required (got %zu)", need, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0) return fail(DSV_ERR_WORKSPACE, "workspace must be 256-byte aligned");

  a.logits = logits->data;
  a.l_dtype = logits->dtype;
  a.l_st = logits->stride[0];
  a.l_sm = logits->stride[1];
  dsv::accept_chunking(a, device_cus());
  const size_t rows = (size_t)T * M * a.nchunk;
  a.rstat = static_cast<float4*>(workspace);
  a.rstat2 = reinterpret_cast<float*>(static_cast<char*>(workspace) + align_up(rows * 16, 256));
  if (g_dry_run) return DSV_OK;
  hipEvent_t ev0, ev1;
  take_events(ev0, ev1);
  hipError_t e = dsv::launch_accept(a, static_cast<hipStream_t>(stream), ev0, ev1);
  if (e != hipSuccess) return hip_fail(e, "acceptance kernel launch");
  return DSV_OK;
}

int dsv_tree_accept_sample(const dsv_tensor* logits, const dsv_tensor* draft, const dsv_tensor* parent,
                           const dsv_tensor* pos, int64_t max_hops, float temperature, float top_p, int64_t top_k,
                           uint64_t seed, dsv_tensor* out_path, dsv_tensor* out_tokens, dsv_tensor* out_info,
                           dsv_tensor* out_next, void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if ((rc = check_nd(logits, "logits", 3)) != DSV_OK) return rc;
  if (logits->dtype != DSV_BF16 && logits->dtype != DSV_F16 && logits->dtype != DSV_F32)
    return fail(DSV_ERR_INVALID, "logits must be bf16, f16 or f32");
  if (logits->stride[2] != 1) return fail(DSV_ERR_INVALID, "logits vocab stride must be 1");
  // The reference builds its warpers only when temperature > 1e-5 (compared in
  // double precision, draft/tree_verification.py:21); at or below it the
  // walk is greedy (dsv_tree_accept).
  if (!((double)temperature > 1e-5) || !(temperature < __builtin_huge_valf()))
    return fail(DSV_ERR_INVALID, "temperature must be > 1e-5 (smaller temperatures are greedy acceptance)");
  if (!(top_p >= 0.f && top_p <= 1.f)) return fail(DSV_ERR_INVALID, "top_p must lie in [0, 1]");
  if (top_k < 0) return fail(DSV_ERR_INVALID, "top_k must be >= 0");
  const int64_t T = logits->shape[0], M = logits->shape[1], V = logits->shape[2];
  AcceptArgs a{};
  if ((rc = accept_common(DSV_ACCEPT_GREEDY, T, M, V, draft, parent, pos, max_hops, 1.f, 0.f, 0.f, out_path,
                          out_tokens, out_info, out_next, a)) != DSV_OK)
    return rc;
  const size_t need = dsv_accept_workspace_bytes(T, M, V);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(DSV_ERR_WORKSPACE, "workspace of %zu bytes required (got %zu)", need, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0) return fail(DSV_ERR_WORKSPACE, "workspace must be 256-byte aligned");

  a.mode = 2;
  a.logits = logits->data;
  a.l_dtype = logits->dtype;
  a.l_st = logits->stride[0];
  a.l_sm = logits->stride[1];
  a.temperature = temperature;
  // The warpers that apply, as prepare_logits_processor builds them
  // (draft/tree_verification.py:15-32): top-p when 1e-8 <= top_p < 1, top-k when > 0.
  a.top_p_q = (top_p >= 1e-8f && top_p < 1.f) ? (uint32_t)std::nearbyint((double)top_p * 4294967296.0) : 0u;
  a.top_k = top_k;
  a.seed = seed;
  dsv::accept_chunking(a, device_cus());
  const size_t rows = (size_t)T * M * a.nchunk;
  char* ws = static_cast<char*>(workspace);
  a.rstat = reinterpret_cast<float4*>(ws);
  const size_t max_rows = (size_t)T * M * dsv::accept_max_chunks(V);
  a.sel = (a.top_p_q != 0 || top_k > 0)
              ? reinterpret_cast<uint4*>(ws + align_up(max_rows * 16, 256) + align_up(max_rows * 4, 256))
              : nullptr;
  (void)rows;
  if (g_dry_run) return DSV_OK;
  hipEvent_t ev0, ev1;
  take_events(ev0, ev1);
  hipError_t e = dsv::launch_sample(a, static_cast<hipStream_t>(stream), ev0, ev1);
  if (e != hipSuccess) return hip_fail(e, "sampling acceptance launch");
  return DSV_OK;
}

size_t dsv_lmhead_accept_workspace_bytes(int64_t T, int64_t M, int64_t V) {
  if (T <= 0 || M <= 0 || V <= 0) return 0;
  const size_t R = (size_t)T * M, parts = R * (size_t)dsv::lmhead_blocks(V);
  return align_up(parts * 16, 256) + align_up(parts * 4, 256) + align_up(R * 16, 256) + 2 * align_up(R * 4, 256);
}

int dsv_lmhead_accept(int mode, const dsv_tensor* hidden, const dsv_tensor* weight, const dsv_tensor* draft,
                      const dsv_tensor* parent, const dsv_tensor* pos, int64_t max_hops, float temperature,
                      float posterior_threshold, float posterior_alpha, dsv_tensor* out_path, dsv_tensor* out_tokens,
                      dsv_tensor* out_info, dsv_tensor* out_next, dsv_tensor* logits_out, void* workspace,
                      size_t workspace_bytes, void* stream) {
  int rc;
  if (mode != DSV_ACCEPT_GREEDY && mode != DSV_ACCEPT_TYPICAL) return fail(DSV_ERR_INVALID, "unknown acceptance mode %d", mode);
  if ((rc = check_nd(hidden, "hidden", 3)) != DSV_OK) return rc;
  if ((rc = check_nd(weight, "weight", 2)) != DSV_OK) return rc;
  if (hidden->dtype != DSV_BF16 || weight->dtype != DSV_BF16) return fail(DSV_ERR_UNSUPPORTED, "hidden and weight must be bf16");
  const int64_t T = hidden->shape[0], M = hidden->shape[1], Dm = hidden->shape[2], V = weight->shape[0];
  if (weight->shape[1] != Dm) return fail(DSV_ERR_INVALID, "weight must be [V, %lld]", (long long)Dm);
  if (Dm < dsv::kLmK || Dm % dsv::kLmK != 0 || Dm > (1 << 20))
    return fail(DSV_ERR_UNSUPPORTED, "hidden size %lld must be a positive multiple of %d", (long long)Dm, dsv::kLmK);
  if (hidden->stride[2] != 1 || weight->stride[1] != 1) return fail(DSV_ERR_INVALID, "hidden and weight rows must be contiguous");
  if (hidden->stride[0] != M * hidden->stride[1] && T > 1)
    return fail(DSV_ERR_INVALID, "hidden rows of all trees must share one stride ([T*M, Dm] view)");
  if ((reinterpret_cast<uintptr_t>(hidden->data) & 15) != 0 || (reinterpret_cast<uintptr_t>(weight->data) & 15) != 0 ||
      hidden->stride[1] % 8 != 0 || weight->stride[0] % 8 != 0)
    return fail(DSV_ERR_INVALID, "hidden and weight rows must be 16-byte aligned");
  AcceptArgs a{};
  if ((rc = accept_common(mode, T, M, V, draft, parent, pos, max_hops, temperature, posterior_threshold,
                          posterior_alpha, out_path, out_tokens, out_info, out_next, a)) != DSV_OK)
    return rc;
  if (present(logits_out)) {
    if ((rc = check_nd(logits_out, "logits_out", 3)) != DSV_OK) return rc;
    if (logits_out->dtype != DSV_BF16 || logits_out->shape[0] != T || logits_out->shape[1] != M ||
        logits_out->shape[2] != V || logits_out->stride[2] != 1 || (T > 1 && logits_out->stride[0] != M * logits_out->stride[1]))
      return fail(DSV_ERR_INVALID, "logits_out must be bf16 [T, M, V] with rows of one stride");
  }
  const size_t need = dsv_lmhead_accept_workspace_bytes(T, M, V);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(DSV_ERR_WORKSPACE, "workspace of %zu bytes required (got %zu)", need, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0) return fail(DSV_ERR_WORKSPACE, "workspace must be 256-byte aligned");

  dsv::LmArgs lm{};
  lm.mode = mode;
  lm.h = static_cast<const uint16_t*>(hidden->data);
  lm.ldh = hidden->stride[1];
  lm.w = static_cast<const uint16_t*>(weight->data);
  lm.ldw = weight->stride[0];
  lm.R = (int)(T * M);
  lm.Dm = (int)Dm;
  lm.V = V;
  lm.T = (int)T;
  lm.M = (int)M;
  lm.draft = a.draft;
  lm.d_st = a.d_st;
  lm.d_sm = a.d_sm;
  lm.parent = a.parent;
  lm.p_st = a.p_st;
  lm.p_sm = a.p_sm;
  lm.inv_temp = a.inv_temp;
  lm.nblk = dsv::lmhead_blocks(V);
  const size_t R = (size_t)T * M, parts = R * (size_t)lm.nblk;
  char* ws = static_cast<char*>(workspace);
  lm.rstat = reinterpret_cast<float4*>(ws);
  ws += align_up(parts * 16, 256);
  lm.rstat2 = reinterpret_cast<float*>(ws);
  ws += align_up(parts * 4, 256);
  a.rstat = reinterpret_cast<float4*>(ws);
  ws += align_up(R * 16, 256);
  a.rstat2 = reinterpret_cast<float*>(ws);
  ws += align_up(R * 4, 256);
  lm.xtok = reinterpret_cast<float*>(ws);
  a.xtok = lm.xtok;
  a.nchunk = 1;
  a.chunk = V;
  if (present(logits_out)) {
    lm.lout = static_cast<uint16_t*>(logits_out->data);
    lm.lo_sr = logits_out->stride[1];
    // The typical test re-decides its near-threshold nodes from the written
    // logits (kernel 5 writes them before the walk runs, on this stream).
    a.logits = logits_out->data;
    a.l_dtype = DSV_BF16;
    a.l_st = logits_out->stride[0];
    a.l_sm = logits_out->stride[1];
  }
  if (g_dry_run) return DSV_OK;
  hipEvent_t ev0, ev1;
  take_events(ev0, ev1);
  hipError_t e;
  if (ev0 != nullptr && (e = hipEventRecord(ev0, static_cast<hipStream_t>(stream))) != hipSuccess)
    return hip_fail(e, "timing event");
  e = dsv::launch_lmhead_accept(a, lm, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "lm_head acceptance launch");
  if (ev1 != nullptr && (e = hipEventRecord(ev1, static_cast<hipStream_t>(stream))) != hipSuccess)
    return hip_fail(e, "timing event");
  return DSV_OK;
}

}  // extern "C"
