// C ABI of libcie_attn.so: argument validation, error reporting and launch.
//
// Validation mirrors the checks the reference performs before it launches
// (engine/attention.py:17-25, kernels/flash_attention.py:147-165) and turns
// them into status codes; the Python layer maps the codes back onto the
// reference's exception types.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdarg>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <utility>

#include "cie_attn.h"
#include "kernels.hpp"

namespace cie {

DeviceShape shape_for_cus(int cus) {
  if (cus < 1) cus = kDefaultCUs;
  const int xcds = std::min(std::max(cus / 32, 1), kMaxXcds);  // 32 active CUs per gfx950 XCD
  int shift = 0;
  while ((2 << shift) <= xcds) ++shift;
  return DeviceShape{cus, shift};
}

DeviceShape device_shape() {
  static std::mutex mu;
  static std::map<int, DeviceShape> known;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();  // no device: leave no error behind for a later launch check
    return shape_for_cus(kDefaultCUs);
  }
  std::lock_guard<std::mutex> lock(mu);
  auto it = known.find(dev);
  if (it == known.end()) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) {
      (void)hipGetLastError();
      cus = kDefaultCUs;
    }
    it = known.emplace(dev, shape_for_cus(cus)).first;
  }
  return it->second;
}

hipError_t set_dynamic_lds(const void* kernel, int bytes) {
  static std::mutex mu;
  static std::set<std::pair<const void*, int>> done;  // (kernel, device) pairs already set
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(mu);
  if (done.count({kernel, dev})) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done.insert({kernel, dev});
  return e;
}

}  // namespace cie

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

bool head_dim_ok(int D) { return D == 16 || D == 32 || D == 64 || D == 128 || D == 256; }

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

// head_dim stride 1, outer strides non-negative and 16-byte multiples (the
// kernels move rows in 16-byte vectors).
int check_strides(const char* name, const int64_t* st) {
  if (!st) return fail(CIE_EINVAL, "%s: stride array is NULL", name);
  if (st[3] != 1) return fail(CIE_EINVAL, "%s: head_dim stride must be 1, got %lld", name, (long long)st[3]);
  for (int i = 0; i < 3; ++i) {
    if (st[i] < 0) return fail(CIE_EINVAL, "%s: negative stride %lld", name, (long long)st[i]);
    if (st[i] % 8) return fail(CIE_EINVAL, "%s: stride %lld is not a multiple of 8 elements", name, (long long)st[i]);
  }
  return CIE_OK;
}

int check_ptr(const char* name, const void* ptr) {
  if (!ptr) return fail(CIE_EINVAL, "%s: NULL pointer", name);
  if (!aligned16(ptr)) return fail(CIE_EINVAL, "%s: pointer is not 16-byte aligned", name);
  return CIE_OK;
}

int common_checks(int Hq, int Hk, int D, int dtype) {
  if (dtype != CIE_DTYPE_F16 && dtype != CIE_DTYPE_BF16)
    return fail(CIE_EDTYPE, "unsupported dtype code %d (f16 = 0, bf16 = 1)", dtype);
  if (!head_dim_ok(D))
    return fail(CIE_EHEADDIM, "head_dim must be a power of 2 in [16, 256], got %d", D);
  if (Hq < 1 || Hk < 1) return fail(CIE_EINVAL, "head counts must be positive (Hq=%d, Hk=%d)", Hq, Hk);
  if (Hq % Hk) return fail(CIE_EINVAL, "num_heads %d must be a multiple of num_kv_heads %d", Hq, Hk);
  return CIE_OK;
}

int launch_status(hipError_t e) {
  if (e != hipSuccess) return fail(CIE_ELAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  g_err.clear();
  return CIE_OK;
}

// Kernels compute exp2(s * c - m) with c = |scale| * log2(e) >= 0; a negative
// scale is folded into an exact sign flip of q (s * scale = (-q).k * |scale|).
// A zero scale becomes a tiny positive one (uniform weights either way).
void set_scale(float scale, float* c, uint32_t* q_sign) {
  *q_sign = scale < 0.f ? 0x80008000u : 0u;
  *c = std::max(std::fabs(scale) * cie::kLog2e, 1e-30f);
}

// cos / sin: (rows, D/2) row-major tables of element type dt (fp16, bf16 or
// fp32), as RotaryEmbedding holds them before or after the engine's cast.
int check_rope(const void* cos, const void* sin, int rows, int dt) {
  if (!cos || !sin) return fail(CIE_EINVAL, "rope tables: NULL pointer");
  if (!aligned16(cos) || !aligned16(sin)) return fail(CIE_EINVAL, "rope tables: pointer is not 16-byte aligned");
  if (rows < 1) return fail(CIE_EINVAL, "rope tables need at least one row, got %d", rows);
  if (dt != CIE_TABLE_F16 && dt != CIE_TABLE_BF16 && dt != CIE_TABLE_F32)
    return fail(CIE_EDTYPE, "unsupported rope table dtype code %d (f16 = 0, bf16 = 1, f32 = 2)", dt);
  return CIE_OK;
}

#define CIE_TRY(x)             \
  do {                         \
    int _rc = (x);             \
    if (_rc != CIE_OK) return _rc; \
  } while (0)

}  // namespace

extern "C" {

int cie_abi_version(void) { return CIE_ABI_VERSION; }

const char* cie_last_error(void) { return g_err.c_str(); }

int cie_device_cus(void) { return cie::device_shape().cus; }

int cie_prefill_kernel(int B, int Hq, int Hk, int Lq, int Lk, int D, int causal, int dtype, int cu_count) {
  CIE_TRY(common_checks(Hq, Hk, D, dtype));
  if (B < 0 || Lq < 0 || Lk < 0) return fail(CIE_EINVAL, "negative size (B=%d, Lq=%d, Lk=%d)", B, Lq, Lk);
  const int64_t n_mt = ((int64_t)Lq + 127) / 128;
  if (n_mt * B * Hq > 0x7fffffff) return fail(CIE_EINVAL, "problem too large for one launch");
  cie::FlashParams p{};
  p.B = B; p.Hq = Hq; p.Hk = Hk; p.Lq = Lq; p.Lk = Lk; p.group = Hq / Hk;
  p.n_mt = (int)n_mt;
  p.n_wg = (int)(n_mt * B * Hq);
  p.causal = causal ? 1 : 0;
  const cie::DeviceShape dev = cu_count > 0 ? cie::shape_for_cus(cu_count) : cie::device_shape();
  p.cus = dev.cus;
  p.xcd_shift = dev.xcd_shift;
  g_err.clear();
  return (int)cie::flash_kernel_choice(p, D);
}

}  // extern "C"

static int flash_impl(const void* q, const void* k, const void* v, void* o,
                      const int64_t* q_stride, const int64_t* k_stride,
                      const int64_t* v_stride, const int64_t* o_stride,
                      int B, int Hq, int Hk, int Lq, int Lk, int D,
                      float scale, int causal, int dtype, void* stream,
                      cie::RopeTables rope, const int32_t* q_pos0) {
  CIE_TRY(common_checks(Hq, Hk, D, dtype));
  if (B < 0 || Lq < 0 || Lk < 0) return fail(CIE_EINVAL, "negative size (B=%d, Lq=%d, Lk=%d)", B, Lq, Lk);
  if (!std::isfinite(scale)) return fail(CIE_EINVAL, "scale must be finite");
  if ((int64_t)B * Hq * Lq == 0) {
    g_err.clear();
    return CIE_OK;  // empty output: nothing to compute
  }
  CIE_TRY(check_ptr("q", q));
  CIE_TRY(check_ptr("o", o));
  CIE_TRY(check_strides("q", q_stride));
  CIE_TRY(check_strides("o", o_stride));
  if (Lk > 0) {
    CIE_TRY(check_ptr("k", k));
    CIE_TRY(check_ptr("v", v));
    CIE_TRY(check_strides("k", k_stride));
    CIE_TRY(check_strides("v", v_stride));
  }
  const int64_t n_mt = ((int64_t)Lq + 127) / 128;
  const int64_t n_wg = n_mt * B * Hq;
  if (n_wg > 0x7fffffff) return fail(CIE_EINVAL, "problem too large for one launch");

  cie::FlashParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.o = static_cast<uint16_t*>(o);
  p.qs0 = q_stride[0]; p.qs1 = q_stride[1]; p.qs2 = q_stride[2];
  p.os0 = o_stride[0]; p.os1 = o_stride[1]; p.os2 = o_stride[2];
  if (Lk > 0) {
    p.ks0 = k_stride[0]; p.ks1 = k_stride[1]; p.ks2 = k_stride[2];
    p.vs0 = v_stride[0]; p.vs1 = v_stride[1]; p.vs2 = v_stride[2];
  }
  p.B = B; p.Hq = Hq; p.Hk = Hk; p.Lq = Lq; p.Lk = Lk; p.group = Hq / Hk;
  p.n_mt = (int)n_mt;
  p.n_wg = (int)n_wg;
  set_scale(scale, &p.scale_log2, &p.q_sign);
  p.causal = causal ? 1 : 0;
  p.rope = rope;
  p.q_pos0 = q_pos0;
  const cie::DeviceShape dev = cie::device_shape();
  p.cus = dev.cus;
  p.xcd_shift = dev.xcd_shift;
  return launch_status(cie::launch_flash(p, dtype, D, static_cast<hipStream_t>(stream)));
}

extern "C" {

int cie_flash_fwd(const void* q, const void* k, const void* v, void* o,
                  const int64_t* q_stride, const int64_t* k_stride,
                  const int64_t* v_stride, const int64_t* o_stride,
                  int B, int Hq, int Hk, int Lq, int Lk, int D,
                  float scale, int causal, int dtype, void* stream) {
  return flash_impl(q, k, v, o, q_stride, k_stride, v_stride, o_stride, B, Hq, Hk, Lq, Lk, D, scale, causal,
                    dtype, stream, cie::RopeTables{nullptr, nullptr, 0, 0}, nullptr);
}

int cie_flash_fwd_rope(const void* q, const void* k, const void* v, void* o,
                       const int64_t* q_stride, const int64_t* k_stride,
                       const int64_t* v_stride, const int64_t* o_stride,
                       int B, int Hq, int Hk, int Lq, int Lk, int D,
                       float scale, int causal, int dtype,
                       const void* rope_cos, const void* rope_sin, int rope_rows, int rope_dtype,
                       const int32_t* q_pos0, void* stream) {
  CIE_TRY(check_rope(rope_cos, rope_sin, rope_rows, rope_dtype));
  return flash_impl(q, k, v, o, q_stride, k_stride, v_stride, o_stride, B, Hq, Hk, Lq, Lk, D, scale, causal,
                    dtype, stream, cie::RopeTables{rope_cos, rope_sin, rope_rows, rope_dtype}, q_pos0);
}

// Largest valid context length: the table bound, tightened by the caller's hint.
static int paged_ctx_limit(int max_context, int block_size, int max_blocks_per_seq) {
  const int64_t bound = (int64_t)max_blocks_per_seq * block_size;
  return (int)(max_context > 0 ? std::min<int64_t>(max_context, bound) : bound);
}

size_t cie_paged_workspace_bytes(int B, int Hq, int Hk, int Lq, int D, int max_context,
                                 int block_size, int max_blocks_per_seq) {
  if (B <= 0 || Hq <= 0 || Hk <= 0 || Lq <= 0 || D <= 0 || block_size <= 0 || max_blocks_per_seq < 0 ||
      Hq % Hk)
    return 0;
  if ((int64_t)max_blocks_per_seq * block_size > 0x7fffffff) return 0;
  const cie::PagedGeom g = cie::paged_geometry(
      B, Hq, Hk, Lq, D, paged_ctx_limit(max_context, block_size, max_blocks_per_seq), block_size, cie::device_shape());
  return g.ok ? g.info_bytes + g.slot_bytes : 0;
}

size_t cie_paged_plan_bytes(int B, int Hq, int Hk, int Lq, int D, int max_context, int block_size,
                            int max_blocks_per_seq) {
  if (B <= 0 || Hq <= 0 || Hk <= 0 || Lq <= 0 || D <= 0 || block_size <= 0 || max_blocks_per_seq < 0 ||
      Hq % Hk)
    return 0;
  if ((int64_t)max_blocks_per_seq * block_size > 0x7fffffff) return 0;
  const cie::PagedGeom g = cie::paged_geometry(
      B, Hq, Hk, Lq, D, paged_ctx_limit(max_context, block_size, max_blocks_per_seq), block_size, cie::device_shape());
  if (!g.ok) return 0;
  const cie::PlanLayout L = cie::paged_plan_layout(g, B, max_blocks_per_seq);
  if (L.ints > 0x7fffffff) return 0;
  return L.ints * sizeof(int32_t);
}

int cie_paged_plan(void* plan, size_t plan_bytes, const int32_t* context_lens, const int32_t* block_tables,
                   int64_t block_table_row_stride, int B, int Hq, int Hk, int Lq, int D, int num_blocks,
                   int block_size, int max_blocks_per_seq, int max_context, int for_append) {
  if (!plan || !context_lens || (!block_tables && B > 0)) return fail(CIE_EINVAL, "plan: NULL pointer");
  if (num_blocks < 0 || block_table_row_stride < max_blocks_per_seq)
    return fail(CIE_EINVAL, "plan: block table row stride %lld is below max_blocks_per_seq %d",
                (long long)block_table_row_stride, max_blocks_per_seq);
  const size_t need = cie_paged_plan_bytes(B, Hq, Hk, Lq, D, max_context, block_size, max_blocks_per_seq);
  if (need == 0) return fail(CIE_EINVAL, "plan: unsupported shape");
  if (plan_bytes < need) return fail(CIE_EWORKSPACE, "plan: %zu bytes required, %zu given", need, plan_bytes);
  const int ctx_limit = paged_ctx_limit(max_context, block_size, max_blocks_per_seq);
  const cie::PagedGeom g = cie::paged_geometry(B, Hq, Hk, Lq, D, ctx_limit, block_size, cie::device_shape());
  const cie::PlanLayout L = cie::paged_plan_layout(g, B, max_blocks_per_seq);
  const int split = cie::build_paged_plan(static_cast<int32_t*>(plan), g, L, context_lens, block_tables,
                                          block_table_row_stride, B, Lq, num_blocks, block_size,
                                          max_blocks_per_seq, ctx_limit, for_append ? 1 : 0);
  if (split < 0) return fail(CIE_EINVAL, "plan: a range exceeds the launch geometry");
  g_err.clear();
  return split;
}

}  // extern "C"

static int paged_impl(const void* q, const void* k_cache, const void* v_cache,
                      const int32_t* block_tables, const int32_t* context_lens,
                      void* o, void* workspace, size_t workspace_bytes,
                      const int64_t* q_stride, const int64_t* kc_stride,
                      const int64_t* vc_stride, const int64_t* o_stride,
                      int B, int Hq, int Hk, int Lq, int D,
                      int num_blocks, int block_size, int max_blocks_per_seq,
                      int max_context, float scale, int causal, int dtype,
                      void* stream, cie::RopeTables rope,
                      const void* k_new = nullptr, const void* v_new = nullptr,
                      const int64_t* kn_stride = nullptr, const int64_t* vn_stride = nullptr,
                      const void* plan = nullptr, size_t plan_bytes = 0, int plan_split = -1) {
  CIE_TRY(common_checks(Hq, Hk, D, dtype));
  if (B < 0 || Lq < 0) return fail(CIE_EINVAL, "negative size (B=%d, Lq=%d)", B, Lq);
  if (block_size < 1) return fail(CIE_EINVAL, "block_size must be positive, got %d", block_size);
  if (num_blocks < 0 || max_blocks_per_seq < 0)
    return fail(CIE_EINVAL, "negative pool geometry (num_blocks=%d, max_blocks_per_seq=%d)", num_blocks,
                max_blocks_per_seq);
  if ((int64_t)max_blocks_per_seq * block_size > 0x7fffffff)
    return fail(CIE_EINVAL, "max_blocks_per_seq * block_size exceeds 2^31");
  if (!std::isfinite(scale)) return fail(CIE_EINVAL, "scale must be finite");
  if ((int64_t)B * Hq * Lq == 0) {
    g_err.clear();
    return CIE_OK;
  }
  CIE_TRY(check_ptr("q", q));
  CIE_TRY(check_ptr("o", o));
  CIE_TRY(check_ptr("k_cache", k_cache));
  CIE_TRY(check_ptr("v_cache", v_cache));
  if (plan) {
    CIE_TRY(check_ptr("plan", plan));
    if (plan_split < 0) return fail(CIE_EINVAL, "plan_split must be the count cie_paged_plan returned");
  } else if (!block_tables || !context_lens) {
    return fail(CIE_EINVAL, "block_tables / context_lens: NULL pointer");
  }
  CIE_TRY(check_strides("q", q_stride));
  CIE_TRY(check_strides("o", o_stride));
  CIE_TRY(check_strides("k_cache", kc_stride));
  CIE_TRY(check_strides("v_cache", vc_stride));
  if ((int64_t)(Hk > 0 ? Hk - 1 : 0) * std::max(kc_stride[2], vc_stride[2]) + D >= ((int64_t)1 << 31))
    return fail(CIE_EINVAL, "k_cache / v_cache: the kv heads of a token span 2^31 elements or more");
  if (k_new || v_new) {
    CIE_TRY(check_ptr("k_new", k_new));
    CIE_TRY(check_ptr("v_new", v_new));
    if (!kn_stride || !vn_stride) return fail(CIE_EINVAL, "k_new / v_new strides: NULL pointer");
    for (int i = 0; i < 2; ++i)
      if (kn_stride[i] < 0 || kn_stride[i] % 8 || vn_stride[i] < 0 || vn_stride[i] % 8)
        return fail(CIE_EINVAL, "k_new / v_new strides must be non-negative multiples of 8 elements");
  }

  const int ctx_limit = paged_ctx_limit(max_context, block_size, max_blocks_per_seq);
  if ((int64_t)B * ((ctx_limit + 31) / 32) > 0x7fffffff) return fail(CIE_EINVAL, "problem too large for one launch");
  const cie::PagedGeom g = cie::paged_geometry(B, Hq, Hk, Lq, D, ctx_limit, block_size, cie::device_shape());
  if (!g.ok) return fail(CIE_EINVAL, "paged attention: %s", g.err);
  // with a plan the piece descriptors live in the plan; the workspace holds
  // only the partial states, and none at all when no sequence is split
  const bool merge = !plan || plan_split > 0;
  const size_t need = plan ? (merge ? g.slot_bytes : 0) : g.info_bytes + g.slot_bytes;
  if (need > 0) {
    if (!workspace || workspace_bytes < need)
      return fail(CIE_EWORKSPACE, "workspace of %zu bytes required, %zu given", need,
                  workspace ? workspace_bytes : (size_t)0);
    if (!aligned16(workspace)) return fail(CIE_EINVAL, "workspace: pointer is not 16-byte aligned");
  }

  cie::PagedParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.kc = static_cast<const uint16_t*>(k_cache);
  p.vc = static_cast<const uint16_t*>(v_cache);
  p.o = static_cast<uint16_t*>(o);
  p.bt = block_tables;
  p.lens = context_lens;
  if (plan) {
    const cie::PlanLayout L = cie::paged_plan_layout(g, B, max_blocks_per_seq);
    // the main pass reads a workgroup's range row in the same round trip as
    // the header, before the header is checked: every offset of this
    // launch's layout must lie in the buffer
    if (plan_bytes < L.ints * sizeof(int32_t))
      return fail(CIE_EINVAL, "plan: %zu bytes given, a plan for these arguments has %zu", plan_bytes,
                  L.ints * sizeof(int32_t));
    p.plan = static_cast<const int32_t*>(plan);
    p.plan_ranges = (int)L.ranges;
    p.plan_entries = (int)L.entries;
    p.plan_ids = (int)L.ids;
    p.plan_empty = (int)L.empty;
    p.info = const_cast<int4*>(reinterpret_cast<const int4*>(p.plan + L.info));  // read only in this mode
    p.slots = static_cast<float*>(workspace);
    // the merge pass reads its sequences from the plan's merge table, sized by
    // the split count the plan was built with (capped at the table's size)
    p.plan_mtab = (int)L.mtab;
    p.plan_split = plan_split;
    p.mtab_cap = plan_split > 0 && cie::paged_xcd_runs(g)
                     ? std::min(cie::merge_cap(plan_split * g.NG, g.dev.xcd_shift),
                                cie::merge_table_cap(B, g.NG, g.dev.xcd_shift))
                     : 0;
  } else {
    p.info = static_cast<int4*>(workspace);
    p.slots = reinterpret_cast<float*>(static_cast<char*>(workspace) + g.info_bytes);
  }
  p.qs0 = q_stride[0]; p.qs1 = q_stride[1]; p.qs2 = q_stride[2];
  p.ks0 = kc_stride[0]; p.ks1 = kc_stride[1]; p.ks2 = kc_stride[2];
  p.vs0 = vc_stride[0]; p.vs1 = vc_stride[1]; p.vs2 = vc_stride[2];
  p.os0 = o_stride[0]; p.os1 = o_stride[1]; p.os2 = o_stride[2];
  p.B = B; p.Hq = Hq; p.Hk = Hk; p.Lq = Lq; p.group = Hq / Hk; p.R = g.R; p.Rt = g.Rt;
  p.num_blocks = num_blocks;
  p.max_blocks = max_blocks_per_seq;
  p.block_size = block_size;
  p.ctx_limit = ctx_limit;
  p.bsdiv = cie::make_fastdiv((uint32_t)block_size);
  p.rtdiv = cie::make_fastdiv((uint32_t)g.Rt);
  p.nwvdiv = cie::make_fastdiv((uint32_t)g.NWV);
  p.ngdiv = cie::make_fastdiv((uint32_t)g.NG);
  {
    // Largest element offset of either pool from its base, and the 24-bit
    // multiplier bounds of the narrow address path.
    const int64_t nb1 = num_blocks > 0 ? num_blocks - 1 : 0;
    const int64_t ext_k = nb1 * kc_stride[0] + (int64_t)(block_size - 1) * kc_stride[1] +
                          (int64_t)(Hk - 1) * kc_stride[2] + (int64_t)D;
    const int64_t ext_v = nb1 * vc_stride[0] + (int64_t)(block_size - 1) * vc_stride[1] +
                          (int64_t)(Hk - 1) * vc_stride[2] + (int64_t)D;
    const int64_t lim24 = (int64_t)1 << 24;
    p.narrow = ext_k < ((int64_t)1 << 31) && ext_v < ((int64_t)1 << 31) && num_blocks < lim24 &&
               block_size < lim24 && kc_stride[0] < lim24 && kc_stride[1] < lim24 && vc_stride[0] < lim24 &&
               vc_stride[1] < lim24;
    p.ks0_24 = (uint32_t)kc_stride[0]; p.ks1_24 = (uint32_t)kc_stride[1];
    p.vs0_24 = (uint32_t)vc_stride[0]; p.vs1_24 = (uint32_t)vc_stride[1];
  }
  p.Hg = g.Hg; p.NG = g.NG; p.n_qt = g.n_qt; p.NWV = g.NWV; p.NCH = g.NCH; p.NST = g.NST; p.Wg = g.Wg;
  // ranges in XCD runs only where the plan's merge table follows them
  p.xcd_runs = plan && cie::paged_xcd_runs(g) ? 1 : 0;
  p.xcd_shift = g.dev.xcd_shift;
  set_scale(scale, &p.scale_log2, &p.q_sign);
  p.causal = causal ? 1 : 0;
  p.rope = rope;
  if (k_new) {
    p.kn = static_cast<const uint16_t*>(k_new);
    p.vn = static_cast<const uint16_t*>(v_new);
    p.kns0 = kn_stride[0]; p.kns1 = kn_stride[1];
    p.vns0 = vn_stride[0]; p.vns1 = vn_stride[1];
  }
  return launch_status(cie::launch_paged(p, dtype, D, g.lds_bytes, merge, static_cast<hipStream_t>(stream)));
}

extern "C" {

int cie_paged_fwd(const void* q, const void* k_cache, const void* v_cache,
                  const int32_t* block_tables, const int32_t* context_lens,
                  void* o, void* workspace, size_t workspace_bytes,
                  const int64_t* q_stride, const int64_t* kc_stride,
                  const int64_t* vc_stride, const int64_t* o_stride,
                  int B, int Hq, int Hk, int Lq, int D,
                  int num_blocks, int block_size, int max_blocks_per_seq,
                  int max_context, float scale, int causal, int dtype,
                  void* stream) {
  return paged_impl(q, k_cache, v_cache, block_tables, context_lens, o, workspace, workspace_bytes, q_stride,
                    kc_stride, vc_stride, o_stride, B, Hq, Hk, Lq, D, num_blocks, block_size, max_blocks_per_seq,
                    max_context, scale, causal, dtype, stream, cie::RopeTables{nullptr, nullptr, 0, 0});
}

int cie_paged_fwd_ex(const void* q, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                     const int32_t* block_tables, const int32_t* context_lens, const void* plan,
                     size_t plan_bytes, int plan_split,
                     void* o, void* workspace, size_t workspace_bytes,
                     const int64_t* q_stride, const int64_t* kn_stride, const int64_t* vn_stride,
                     const int64_t* kc_stride, const int64_t* vc_stride, const int64_t* o_stride,
                     int B, int Hq, int Hk, int Lq, int D,
                     int num_blocks, int block_size, int max_blocks_per_seq,
                     int max_context, float scale, int causal, int dtype,
                     const void* rope_cos, const void* rope_sin, int rope_rows, int rope_dtype,
                     void* stream) {
  if ((k_new == nullptr) != (v_new == nullptr)) return fail(CIE_EINVAL, "k_new / v_new: give both or neither");
  cie::RopeTables rope{nullptr, nullptr, 0, 0};
  if (rope_cos || rope_sin) {
    CIE_TRY(check_rope(rope_cos, rope_sin, rope_rows, rope_dtype));
    rope = cie::RopeTables{rope_cos, rope_sin, rope_rows, rope_dtype};
  }
  return paged_impl(q, k_cache, v_cache, block_tables, context_lens, o, workspace, workspace_bytes, q_stride,
                    kc_stride, vc_stride, o_stride, B, Hq, Hk, Lq, D, num_blocks, block_size, max_blocks_per_seq,
                    max_context, scale, causal, dtype, stream, rope, k_new, v_new, kn_stride, vn_stride, plan,
                    plan_bytes, plan ? plan_split : -1);
}

int cie_paged_fwd_noalloc(const void* q, const void* k_cache, const void* v_cache,
                          const int32_t* block_tables, const int32_t* context_lens, void* o,
                          const int64_t* q_stride, const int64_t* kc_stride,
                          const int64_t* vc_stride, const int64_t* o_stride,
                          int B, int Hq, int Hk, int Lq, int D,
                          int num_blocks, int block_size, int max_blocks_per_seq,
                          int max_context, float scale, int causal, int dtype,
                          void* stream) {
  // the workspace this shape needs must fit the static array; checked
  // before any HIP call
  const size_t need = cie_paged_workspace_bytes(B, Hq, Hk, Lq, D, max_context, block_size, max_blocks_per_seq);
  if (need > cie::kPagedScratchBytes)
    return fail(CIE_EWORKSPACE, "this shape needs %zu bytes of workspace, more than the %zu-byte static workspace "
                "of cie_paged_fwd_noalloc; use cie_paged_fwd with a caller workspace", need,
                cie::kPagedScratchBytes);
  if ((int64_t)B * Hq * Lq <= 0 || need == 0)  // empty, or a shape cie_paged_fwd rejects: same result, no lookup
    return paged_impl(q, k_cache, v_cache, block_tables, context_lens, o, nullptr, 0, q_stride, kc_stride,
                      vc_stride, o_stride, B, Hq, Hk, Lq, D, num_blocks, block_size, max_blocks_per_seq,
                      max_context, scale, causal, dtype, stream, cie::RopeTables{nullptr, nullptr, 0, 0});
  void* ws = nullptr;
  const hipError_t e = cie::paged_scratch_ptr(&ws);
  if (e != hipSuccess) return fail(CIE_ELAUNCH, "static workspace lookup failed: %s", hipGetErrorString(e));
  return paged_impl(q, k_cache, v_cache, block_tables, context_lens, o, ws, cie::kPagedScratchBytes, q_stride,
                    kc_stride, vc_stride, o_stride, B, Hq, Hk, Lq, D, num_blocks, block_size, max_blocks_per_seq,
                    max_context, scale, causal, dtype, stream, cie::RopeTables{nullptr, nullptr, 0, 0});
}

int cie_paged_fwd_rope(const void* q, const void* k_cache, const void* v_cache,
                       const int32_t* block_tables, const int32_t* context_lens,
                       void* o, void* workspace, size_t workspace_bytes,
                       const int64_t* q_stride, const int64_t* kc_stride,
                       const int64_t* vc_stride, const int64_t* o_stride,
                       int B, int Hq, int Hk, int Lq, int D,
                       int num_blocks, int block_size, int max_blocks_per_seq,
                       int max_context, float scale, int causal, int dtype,
                       const void* rope_cos, const void* rope_sin, int rope_rows, int rope_dtype,
                       void* stream) {
  CIE_TRY(check_rope(rope_cos, rope_sin, rope_rows, rope_dtype));
  return paged_impl(q, k_cache, v_cache, block_tables, context_lens, o, workspace, workspace_bytes, q_stride,
                    kc_stride, vc_stride, o_stride, B, Hq, Hk, Lq, D, num_blocks, block_size, max_blocks_per_seq,
                    max_context, scale, causal, dtype, stream,
                    cie::RopeTables{rope_cos, rope_sin, rope_rows, rope_dtype});
}

int cie_paged_fwd_append(const void* q, const void* k_new, const void* v_new,
                         void* k_cache, void* v_cache,
                         const int32_t* block_tables, const int32_t* context_lens,
                         void* o, void* workspace, size_t workspace_bytes,
                         const int64_t* q_stride, const int64_t* kn_stride, const int64_t* vn_stride,
                         const int64_t* kc_stride, const int64_t* vc_stride, const int64_t* o_stride,
                         int B, int Hq, int Hk, int Lq, int D,
                         int num_blocks, int block_size, int max_blocks_per_seq,
                         int max_context, float scale, int causal, int dtype,
                         void* stream) {
  if (!k_new || !v_new) return fail(CIE_EINVAL, "k_new / v_new: NULL pointer");
  return paged_impl(q, k_cache, v_cache, block_tables, context_lens, o, workspace, workspace_bytes, q_stride,
                    kc_stride, vc_stride, o_stride, B, Hq, Hk, Lq, D, num_blocks, block_size, max_blocks_per_seq,
                    max_context, scale, causal, dtype, stream, cie::RopeTables{nullptr, nullptr, 0, 0}, k_new, v_new,
                    kn_stride, vn_stride);
}

int cie_paged_fwd_append_rope(const void* q, const void* k_new, const void* v_new,
                              void* k_cache, void* v_cache,
                              const int32_t* block_tables, const int32_t* context_lens,
                              void* o, void* workspace, size_t workspace_bytes,
                              const int64_t* q_stride, const int64_t* kn_stride, const int64_t* vn_stride,
                              const int64_t* kc_stride, const int64_t* vc_stride, const int64_t* o_stride,
                              int B, int Hq, int Hk, int Lq, int D,
                              int num_blocks, int block_size, int max_blocks_per_seq,
                              int max_context, float scale, int causal, int dtype,
                              const void* rope_cos, const void* rope_sin, int rope_rows, int rope_dtype,
                              void* stream) {
  if (!k_new || !v_new) return fail(CIE_EINVAL, "k_new / v_new: NULL pointer");
  CIE_TRY(check_rope(rope_cos, rope_sin, rope_rows, rope_dtype));
  return paged_impl(q, k_cache, v_cache, block_tables, context_lens, o, workspace, workspace_bytes, q_stride,
                    kc_stride, vc_stride, o_stride, B, Hq, Hk, Lq, D, num_blocks, block_size, max_blocks_per_seq,
                    max_context, scale, causal, dtype, stream,
                    cie::RopeTables{rope_cos, rope_sin, rope_rows, rope_dtype}, k_new, v_new, kn_stride, vn_stride);
}

}  // extern "C"

static int append_impl(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                       const int64_t* new_stride, const int64_t* v_new_stride,
                       const int64_t* kc_stride, const int64_t* vc_stride,
                       const int32_t* block_tables, const int32_t* cu_new, const int32_t* start,
                       uint32_t* status, int B, int T, int max_new, int Hk, int D,
                       int num_blocks, int block_size, int max_blocks_per_seq, int dtype, void* stream,
                       cie::RopeTables rope, void* k_out, const int64_t* k_out_stride) {
  if (dtype != CIE_DTYPE_F16 && dtype != CIE_DTYPE_BF16)
    return fail(CIE_EDTYPE, "unsupported dtype code %d (f16 = 0, bf16 = 1)", dtype);
  if (!head_dim_ok(D)) return fail(CIE_EHEADDIM, "head_dim must be a power of 2 in [16, 256], got %d", D);
  if (B < 0 || T < 0 || max_new < 0 || Hk < 1)
    return fail(CIE_EINVAL, "invalid sizes (B=%d, T=%d, max_new=%d, Hk=%d)", B, T, max_new, Hk);
  if (block_size < 1 || num_blocks < 0 || max_blocks_per_seq < 0)
    return fail(CIE_EINVAL, "invalid pool geometry (num_blocks=%d, block_size=%d, max_blocks_per_seq=%d)",
                num_blocks, block_size, max_blocks_per_seq);
  if ((int64_t)max_blocks_per_seq * block_size > 0x7fffffff)
    return fail(CIE_EINVAL, "max_blocks_per_seq * block_size exceeds 2^31");
  if ((int64_t)max_new * Hk * D / 8 >= ((int64_t)1 << 31)) return fail(CIE_EINVAL, "too many new tokens for one launch");
  if (B == 0 || T == 0 || max_new == 0) {
    g_err.clear();
    return CIE_OK;
  }
  CIE_TRY(check_ptr("k_new", k_new));
  CIE_TRY(check_ptr("v_new", v_new));
  CIE_TRY(check_ptr("k_cache", k_cache));
  CIE_TRY(check_ptr("v_cache", v_cache));
  if (!block_tables || !cu_new || !start) return fail(CIE_EINVAL, "block_tables / cu_new / start: NULL pointer");
  // (T, Hk, D) sources: reuse the 4-d stride check on (1, T, Hk, D)
  const int64_t ns[4] = {0, new_stride ? new_stride[0] : 0, new_stride ? new_stride[1] : 0,
                         new_stride ? new_stride[2] : 0};
  const int64_t ms[4] = {0, v_new_stride ? v_new_stride[0] : 0, v_new_stride ? v_new_stride[1] : 0,
                         v_new_stride ? v_new_stride[2] : 0};
  if (!new_stride || !v_new_stride) return fail(CIE_EINVAL, "k_new / v_new: stride array is NULL");
  CIE_TRY(check_strides("k_new", ns));
  CIE_TRY(check_strides("v_new", ms));
  CIE_TRY(check_strides("k_cache", kc_stride));
  CIE_TRY(check_strides("v_cache", vc_stride));

  cie::AppendParams p{};
  p.k_new = static_cast<const uint16_t*>(k_new);
  p.v_new = static_cast<const uint16_t*>(v_new);
  p.kc = static_cast<uint16_t*>(k_cache);
  p.vc = static_cast<uint16_t*>(v_cache);
  p.bt = block_tables;
  p.cu_new = cu_new;
  p.start = start;
  p.status = status;
  p.ns0 = ns[1]; p.ns1 = ns[2];
  p.ms0 = ms[1]; p.ms1 = ms[2];
  p.ks0 = kc_stride[0]; p.ks1 = kc_stride[1]; p.ks2 = kc_stride[2];
  p.vs0 = vc_stride[0]; p.vs1 = vc_stride[1]; p.vs2 = vc_stride[2];
  p.num_blocks = num_blocks;
  p.max_blocks = max_blocks_per_seq;
  p.block_size = block_size;
  p.cpr = (uint32_t)(Hk * D / 8);
  p.lg_cph = (uint32_t)__builtin_ctz((unsigned)(D / 8));
  p.cprdiv = cie::make_fastdiv(p.cpr);
  p.bsdiv = cie::make_fastdiv((uint32_t)block_size);
  p.rope = rope;
  p.updiv = cie::make_fastdiv(p.cpr / 2);
  if (k_out) {
    if (!rope.cos) return fail(CIE_EINVAL, "k_out is only written by the rotary append");
    CIE_TRY(check_ptr("k_out", k_out));
    if (!k_out_stride) return fail(CIE_EINVAL, "k_out: stride array is NULL");
    const int64_t os[4] = {0, k_out_stride[0], k_out_stride[1], k_out_stride[2]};
    CIE_TRY(check_strides("k_out", os));
    p.k_out = static_cast<uint16_t*>(k_out);
    p.os0 = os[1];
    p.os1 = os[2];
  }
  return launch_status(cie::launch_kv_append(p, B, max_new, dtype, D, static_cast<hipStream_t>(stream)));
}

extern "C" {

int cie_kv_append(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                  const int64_t* new_stride, const int64_t* v_new_stride,
                  const int64_t* kc_stride, const int64_t* vc_stride,
                  const int32_t* block_tables, const int32_t* cu_new, const int32_t* start,
                  uint32_t* status, int B, int T, int max_new, int Hk, int D,
                  int num_blocks, int block_size, int max_blocks_per_seq, int dtype, void* stream) {
  return append_impl(k_new, v_new, k_cache, v_cache, new_stride, v_new_stride, kc_stride, vc_stride, block_tables,
                     cu_new, start, status, B, T, max_new, Hk, D, num_blocks, block_size, max_blocks_per_seq, dtype,
                     stream, cie::RopeTables{nullptr, nullptr, 0, 0}, nullptr, nullptr);
}

int cie_kv_append_rope(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                       const int64_t* new_stride, const int64_t* v_new_stride,
                       const int64_t* kc_stride, const int64_t* vc_stride,
                       const int32_t* block_tables, const int32_t* cu_new, const int32_t* start,
                       uint32_t* status, int B, int T, int max_new, int Hk, int D,
                       int num_blocks, int block_size, int max_blocks_per_seq, int dtype,
                       const void* rope_cos, const void* rope_sin, int rope_rows, int rope_dtype,
                       void* k_out, const int64_t* k_out_stride, void* stream) {
  CIE_TRY(check_rope(rope_cos, rope_sin, rope_rows, rope_dtype));
  return append_impl(k_new, v_new, k_cache, v_cache, new_stride, v_new_stride, kc_stride, vc_stride, block_tables,
                     cu_new, start, status, B, T, max_new, Hk, D, num_blocks, block_size, max_blocks_per_seq, dtype,
                     stream, cie::RopeTables{rope_cos, rope_sin, rope_rows, rope_dtype}, k_out, k_out_stride);
}

size_t cie_int8_matmul_workspace_bytes(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return cie::int8_gemm_geometry(M, N, K, cie::device_shape()).workspace_bytes;
}

int cie_int8_matmul(const void* x, const int8_t* w, const void* scales, const void* bias, void* y,
                    int64_t x_row_stride, int64_t w_row_stride, int64_t y_row_stride,
                    int M, int N, int K, int dtype, int scale_dtype,
                    void* workspace, size_t workspace_bytes, void* stream) {
  if (dtype != CIE_DTYPE_F16 && dtype != CIE_DTYPE_BF16)
    return fail(CIE_EDTYPE, "unsupported activation dtype code %d (f16 = 0, bf16 = 1)", dtype);
  if (scale_dtype < 0 || scale_dtype > 2)
    return fail(CIE_EDTYPE, "unsupported scale dtype code %d (f16 = 0, bf16 = 1, f32 = 2)", scale_dtype);
  if (M < 0 || N < 0 || K < 0) return fail(CIE_EINVAL, "negative size (M=%d, N=%d, K=%d)", M, N, K);
  if ((int64_t)M * N == 0) {
    g_err.clear();
    return CIE_OK;
  }
  if (K == 0) return fail(CIE_EINVAL, "in_features K must be positive");
  CIE_TRY(check_ptr("x", x));
  CIE_TRY(check_ptr("w_int8", w));
  if (!y || reinterpret_cast<uintptr_t>(y) % 8) return fail(CIE_EINVAL, "y: NULL or not 8-byte aligned");
  if (!scales) return fail(CIE_EINVAL, "scales: NULL pointer");
  if (reinterpret_cast<uintptr_t>(scales) % (scale_dtype == 2 ? 4 : 2))
    return fail(CIE_EINVAL, "scales: pointer is not aligned to its element size");
  if (bias && reinterpret_cast<uintptr_t>(bias) % 2) return fail(CIE_EINVAL, "bias: misaligned pointer");
  if (x_row_stride < K || x_row_stride % 8)
    return fail(CIE_EINVAL, "x row stride %lld must be >= K and a multiple of 8 elements", (long long)x_row_stride);
  if (w_row_stride < K || w_row_stride % 16)
    return fail(CIE_EINVAL, "w_int8 row stride %lld must be >= K and a multiple of 16 bytes",
                (long long)w_row_stride);
  if (y_row_stride < N) return fail(CIE_EINVAL, "y row stride %lld must be >= N", (long long)y_row_stride);
  const cie::I8Geom g = cie::int8_gemm_geometry(M, N, K, cie::device_shape());
  if ((int64_t)g.n_tiles * g.m_tiles * g.splits > 0x7fffffff) return fail(CIE_EINVAL, "problem too large");
  if (g.workspace_bytes) {
    if (!workspace || workspace_bytes < g.workspace_bytes)
      return fail(CIE_EWORKSPACE, "workspace of %zu bytes required, %zu given", g.workspace_bytes,
                  workspace ? workspace_bytes : (size_t)0);
    if (!aligned16(workspace)) return fail(CIE_EINVAL, "workspace: pointer is not 16-byte aligned");
  }
  cie::I8GemmParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.w = w;
  p.scales = scales;
  p.bias = static_cast<const uint16_t*>(bias);
  p.y = static_cast<uint16_t*>(y);
  p.partial = static_cast<float*>(workspace);
  p.xs = x_row_stride;
  p.wsr = w_row_stride;
  p.ys = y_row_stride;
  p.M = M; p.N = N; p.K = K; p.scale_dtype = scale_dtype;
  p.n_tiles = g.n_tiles; p.m_tiles = g.m_tiles; p.splits = g.splits; p.ksteps = g.ksteps;
  p.m_pad = g.m_pad; p.n_pad = g.n_pad;
  p.xcd_shift = g.dev.xcd_shift;
  return launch_status(cie::launch_int8_gemm(p, g, dtype, static_cast<hipStream_t>(stream)));
}

int cie_rope_apply(const void* x, void* out, const int64_t* x_stride, const int64_t* out_stride,
                   const int32_t* positions, int64_t pos_batch_stride,
                   const void* rope_cos, const void* rope_sin, int rope_rows, int rope_dtype,
                   uint32_t* status, int B, int H, int L, int D, int dtype, void* stream) {
  if (dtype != CIE_DTYPE_F16 && dtype != CIE_DTYPE_BF16)
    return fail(CIE_EDTYPE, "unsupported dtype code %d (f16 = 0, bf16 = 1)", dtype);
  if (!head_dim_ok(D)) return fail(CIE_EHEADDIM, "head_dim must be a power of 2 in [16, 256], got %d", D);
  if (B < 0 || H < 0 || L < 0 || pos_batch_stride < 0)
    return fail(CIE_EINVAL, "invalid sizes (B=%d, H=%d, L=%d, pos_batch_stride=%lld)", B, H, L,
                (long long)pos_batch_stride);
  CIE_TRY(check_rope(rope_cos, rope_sin, rope_rows, rope_dtype));
  // eight heads per thread where that still gives 512 workgroups (4 x 32 x
  // 2048 x 64: 19.0 -> 16.8 us); one head per thread for smaller launches,
  // where fewer, longer threads were slower (a 32-sequence decode step's q:
  // 4.1 -> 6.8 us)
  const int hg = (int64_t)B * H * L * (D / 16) >= cie::kRopeGroupMin ? cie::kRopeHeads : 1;
  const int nhg = (H + hg - 1) / hg;
  const int64_t total = (int64_t)B * nhg * L * (D / 16);
  if (total >= ((int64_t)1 << 31)) return fail(CIE_EINVAL, "too many rows for one launch");
  if (total == 0) {
    g_err.clear();
    return CIE_OK;
  }
  CIE_TRY(check_ptr("x", x));
  CIE_TRY(check_ptr("out", out));
  CIE_TRY(check_strides("x", x_stride));
  CIE_TRY(check_strides("out", out_stride));
  cie::RopeParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.out = static_cast<uint16_t*>(out);
  p.xs0 = x_stride[0]; p.xs1 = x_stride[1]; p.xs2 = x_stride[2];
  p.os0 = out_stride[0]; p.os1 = out_stride[1]; p.os2 = out_stride[2];
  p.pos = positions;
  p.pos_bs = pos_batch_stride;
  p.tab = cie::RopeTables{rope_cos, rope_sin, rope_rows, rope_dtype};
  p.status = status;
  p.B = B; p.H = H; p.L = L;
  p.HG = hg;
  p.NHG = nhg;
  p.total = (uint32_t)total;
  p.ldiv = cie::make_fastdiv((uint32_t)L);
  p.hgdiv = cie::make_fastdiv((uint32_t)nhg);
  return launch_status(cie::launch_rope(p, dtype, D, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
