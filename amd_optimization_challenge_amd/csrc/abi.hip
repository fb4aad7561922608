// extern "C" entry points of libmla_mi355x.so (declared in include/mla_mi355x.h).
// Host code only: argument validation, workspace carve-up, launches.  Nothing
// here allocates device memory or synchronizes the host.
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <mutex>
#include <string>

#include "../../include/mla_mi355x.h"
#include "mla_internal.hpp"

namespace mla {
namespace {
thread_local std::string g_last_error;
}  // namespace

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

namespace {

int hip_fail(hipError_t e, const char* what) {
  return set_error(MLA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr int kMaxDevices = 64;
int g_cu_count[kMaxDevices] = {0};
std::mutex g_cu_mutex;

int cu_count(int* out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return set_error(MLA_ERR_UNSUPPORTED, "device ordinal %d too large", dev);
  std::lock_guard<std::mutex> lock(g_cu_mutex);
  if (g_cu_count[dev] == 0) {
    int n = 0;
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute(MultiprocessorCount)");
    g_cu_count[dev] = n;
  }
  *out = g_cu_count[dev];
  return MLA_OK;
}

int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

bool aligned(const void* p, int a) { return (reinterpret_cast<uintptr_t>(p) & (uintptr_t)(a - 1)) == 0; }

int check_qlen(int batch, int q_seq_len) {
  if (q_seq_len < 1 || batch % q_seq_len != 0)
    return set_error(MLA_ERR_INVALID_ARGUMENT, "q_seq_len must be >= 1 and divide the %d query rows (got %d)", batch,
                q_seq_len);
  return MLA_OK;
}

int check_shape(int batch, int num_heads, int kv_mode) {
  if (batch < 1) return set_error(MLA_ERR_INVALID_ARGUMENT, "batch must be >= 1 (got %d)", batch);
  if (num_heads != 16 && num_heads != 128)
    return set_error(MLA_ERR_UNSUPPORTED, "num_heads must be 16 or 128 (got %d)", num_heads);
  if (kv_mode < MLA_KV_FP8 || kv_mode > MLA_KV_BF16)
    return set_error(MLA_ERR_INVALID_ARGUMENT, "unknown kv_mode %d", kv_mode);
  if (num_heads == 128 && kv_mode == MLA_KV_MXFP4)
    return set_error(MLA_ERR_UNSUPPORTED, "kv_mode mxfp4 (fp4 V) is implemented for num_heads=16 only");
  if (num_heads == 128 && kv_mode == MLA_KV_BF16)
    return set_error(MLA_ERR_UNSUPPORTED, "kv_mode bf16 (a16w16) is implemented for num_heads=16 only");
  return MLA_OK;
}

}  // namespace

// Resident decode work-groups per CU: two for H = 16 with one cache (fp8 or
// mxfp4 rows serve both K and V; the ring fits in half the LDS), else one (the
// LDS ring fills the CU).  kv_mode < 0 gives the largest over the modes (the
// workspace is sized for it).
static int blocks_per_cu(int num_heads, int kv_mode) {
  if (num_heads != 16) return 1;
  return (kv_mode == MLA_KV_FP8 || kv_mode == MLA_KV_MXFP4 || kv_mode < 0) ? 2 : 1;
}

// Items the planner aims for: one per resident work-group slot while the
// batch is smaller than the slots; once it fills them, 1.5 per slot (or one
// per sequence, if more), so that long sequences are still split and the
// items balance without splitting every sequence (each split costs a second
// prologue and a partial output); capped at four rounds of slots.
int target_items_for(int batch, int num_heads, int kv_mode, int num_cu) {
  const int slots = num_cu * blocks_per_cu(num_heads, kv_mode);
  if (batch < slots) return slots;
  const int t = batch > slots * 3 / 2 ? batch : slots * 3 / 2;
  return t < 4 * slots ? t : 4 * slots;
}

// Contiguous rows (no kv_indices) at 16 heads stream well from one work-group
// per CU, so while the batch is below the CU count the target is one item per
// CU rather than per slot (fewer, longer pieces: fewer prologues and
// partials), and from there up the chunk (longest piece) is at least 1024
// tokens: a two-way split of 1024-token sequences costs more in prologues and
// partial outputs than the idle slots it fills.  No sequence is cut into more
// than 32 pieces: the combine folds a sequence's pieces 8 loads at a time per
// thread, on 4 work-groups per 16 heads, so 64 pieces cost more in that serial
// tail than the shorter items save.  On the task's shapes (mxfp4 cache, whole
// call) this took 256 x 1024 from 71 to 61 us, 32 x 8192 from 67 to 64 and
// 4 x 8192 from 38.5 to 35.9; indexed caches keep target_items_for, their
// scattered rows need both slots of a CU in flight (128 x 4096: 97 us at one
// item per slot, 122 at one per CU).
PlanTarget plan_target_for(int batch, int num_heads, int kv_mode, int num_cu, bool contiguous) {
  PlanTarget t{target_items_for(batch, num_heads, kv_mode, num_cu), kPlanMinChunk, 0};
  if (contiguous && num_heads == 16) {
    if (batch < num_cu) t.items = num_cu < t.items ? num_cu : t.items;
    else t.min_chunk = 1024;
    t.max_splits = 32;
  }
  return t;
}

WsLayout workspace_layout(int batch, int num_heads, int kv_mode, int num_cu) {
  WsLayout L;
  // the planner emits at most target + batch items; the layout is sized for the
  // largest target over the kv modes, so mla_combine can recompute it without one
  (void)kv_mode;
  L.target_items = target_items_for(batch, num_heads, -1, num_cu);
  L.max_items = L.target_items + batch;
  int64_t off = 0;
  L.quant_off = off;
  off = align256(off + kQuantScratchBytes);
  L.qfp8_off = off;
  off = align256(off + (int64_t)batch * num_heads * kQKDim);
  L.plan_off = off;
  off = align256(off + (int64_t)(kPlanHeader + 4 * L.max_items + 2 * batch) * 4);
  L.part_o_off = off;
  off = align256(off + (int64_t)L.max_items * num_heads * kVDim * 2);
  L.part_lse_off = off;
  off = align256(off + (int64_t)L.max_items * num_heads * 4);
  L.total = off;
  return L;
}

namespace {

int decode_params(const void* q_fp8, const float* q_scale, const void* k_cache, int64_t k_row_stride,
                  const void* k_scales, int64_t k_scale_stride, const void* v_cache,
                  int64_t v_row_stride, const float* kv_scale, const int32_t* kv_indptr,
                  const int32_t* kv_indices, int batch, int num_heads, float sm_scale, int kv_mode,
                  void* workspace, int64_t workspace_bytes, void* out, float* lse_out, DecodeParams* p,
                  WsLayout* L) {
  int rc = check_shape(batch, num_heads, kv_mode);
  if (rc) return rc;
  int ncu = 0;
  if ((rc = cu_count(&ncu))) return rc;
  *L = workspace_layout(batch, num_heads, kv_mode, ncu);
  if (workspace == nullptr || workspace_bytes < L->total)
    return set_error(MLA_ERR_WORKSPACE_TOO_SMALL, "workspace needs %lld bytes (got %lld)",
                (long long)L->total, (long long)workspace_bytes);
  if (!aligned(workspace, 256)) return set_error(MLA_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
  if (!q_fp8 || !q_scale || !k_cache || !kv_indptr || !out)
    return set_error(MLA_ERR_INVALID_ARGUMENT, "null q/q_scale/k_cache/kv_indptr/out pointer");
  if (!aligned(q_fp8, 16) || !aligned(k_cache, 16) || !aligned(out, 16))
    return set_error(MLA_ERR_INVALID_ARGUMENT, "q, k_cache and out must be 16-byte aligned");
  if (!(sm_scale > 0.f)) return set_error(MLA_ERR_INVALID_ARGUMENT, "sm_scale must be > 0");
  const bool k_fp4 = kv_mode == MLA_KV_MXFP4 || kv_mode == MLA_KV_MXFP4K_FP8V;
  const int64_t krow = kv_mode == MLA_KV_BF16 ? 2 * kQKDim : (k_fp4 ? kFp4RowBytes : kQKDim);
  if (k_row_stride < krow || (k_row_stride % 16) != 0)
    return set_error(MLA_ERR_INVALID_ARGUMENT, "k_row_stride must be >= %lld and a multiple of 16 (got %lld)",
                (long long)krow, (long long)k_row_stride);
  if (k_fp4) {
    if (!k_scales) return set_error(MLA_ERR_INVALID_ARGUMENT, "mxfp4 K needs k_scales");
    if (k_scale_stride < kMxBlocks)
      return set_error(MLA_ERR_INVALID_ARGUMENT, "k_scale_stride must be >= 18 (got %lld)", (long long)k_scale_stride);
  }
  if (kv_mode == MLA_KV_MXFP4K_FP8V) {
    if (!v_cache || !aligned(v_cache, 16)) return set_error(MLA_ERR_INVALID_ARGUMENT, "fp8 V cache missing or misaligned");
    if (v_row_stride < kVDim || (v_row_stride % 16) != 0)
      return set_error(MLA_ERR_INVALID_ARGUMENT, "v_row_stride must be >= 512 and a multiple of 16");
  }
  if ((kv_mode == MLA_KV_FP8 || kv_mode == MLA_KV_MXFP4K_FP8V) && !kv_scale)
    return set_error(MLA_ERR_INVALID_ARGUMENT, "fp8 cache needs kv_scale");
  // the kernels form row offsets as 32 x 32 -> 64-bit products (slot x stride)
  if (k_row_stride > INT32_MAX || k_scale_stride > INT32_MAX || v_row_stride > INT32_MAX)
    return set_error(MLA_ERR_INVALID_ARGUMENT, "row strides must be below 2^31 bytes");
  char* ws = static_cast<char*>(workspace);
  p->q_fp8 = static_cast<const uint8_t*>(q_fp8);
  p->q_scale = q_scale;
  p->k_cache = static_cast<const uint8_t*>(k_cache);
  p->k_row_stride = k_row_stride;
  p->k_scales = static_cast<const uint8_t*>(k_scales);
  p->k_scale_stride = k_scale_stride;
  p->v_cache = static_cast<const uint8_t*>(v_cache);
  p->v_row_stride = v_row_stride;
  p->kv_scale = kv_scale;
  p->kv_indptr = kv_indptr;
  p->kv_indices = kv_indices;
  p->plan = reinterpret_cast<const int32_t*>(ws + L->plan_off);
  p->part_o = reinterpret_cast<uint16_t*>(ws + L->part_o_off);
  p->part_lse = reinterpret_cast<float*>(ws + L->part_lse_off);
  p->out = static_cast<uint16_t*>(out);
  p->lse_out = lse_out;
  p->q_bf16 = nullptr;
  p->q_partials = nullptr;
  p->q_nparts = 0;
  p->q_per_row = 0;
  p->plan_here = 0;
  p->plan_qlen = 1;
  p->plan_target = 0;
  p->plan_min_chunk = kPlanMinChunk;
  p->plan_max_splits = 0;
  p->sm_scale = sm_scale;
  p->batch = batch;
  p->num_heads = num_heads;
  p->max_items = L->max_items;
  return MLA_OK;
}

}  // namespace
}  // namespace mla

using namespace mla;

extern "C" {

const char* mla_last_error(void) { return g_last_error.c_str(); }

int mla_abi_version(void) { return 2; }

int mla_device_cu_count(int* num_cu) {
  if (!num_cu) return set_error(MLA_ERR_INVALID_ARGUMENT, "num_cu is null");
  return cu_count(num_cu);
}

int mla_workspace_bytes(int batch, int num_heads, int kv_mode, int64_t* bytes) {
  if (!bytes) return set_error(MLA_ERR_INVALID_ARGUMENT, "bytes is null");
  int rc = check_shape(batch, num_heads, kv_mode);
  if (rc) return rc;
  int ncu = 0;
  if ((rc = cu_count(&ncu))) return rc;
  *bytes = workspace_layout(batch, num_heads, kv_mode, ncu).total;
  return MLA_OK;
}

int mla_quant_fp8_per_tensor(const void* x_bf16, int64_t n, void* out_fp8, float* out_scale,
                             void* workspace, int64_t workspace_bytes, void* stream) {
  if (n < 1) return set_error(MLA_ERR_INVALID_ARGUMENT, "n must be >= 1");
  if (!x_bf16 || !out_fp8 || !out_scale || !workspace)
    return set_error(MLA_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (!aligned(x_bf16, 16) || !aligned(out_fp8, 8) || !aligned(workspace, 16))
    return set_error(MLA_ERR_INVALID_ARGUMENT, "x must be 16-byte, out 8-byte, workspace 16-byte aligned");
  if (workspace_bytes < kQuantScratchBytes)
    return set_error(MLA_ERR_WORKSPACE_TOO_SMALL, "workspace needs %lld bytes", (long long)kQuantScratchBytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* partials = static_cast<uint32_t*>(workspace);
  int nb = 0;
  hipError_t e = launch_amax(static_cast<const uint16_t*>(x_bf16), n, partials, &nb, nullptr, nullptr, 0, 1,
                             PlanTarget{0, kPlanMinChunk, 0}, 0, nullptr, s);
  if (e != hipSuccess) return hip_fail(e, "amax launch");
  e = launch_quant_fp8(static_cast<const uint16_t*>(x_bf16), n, partials, nb,
                       static_cast<uint8_t*>(out_fp8), out_scale, s);
  if (e != hipSuccess) return hip_fail(e, "quant launch");
  return MLA_OK;
}

int mla_pack_mxfp4(const void* x_bf16, int64_t rows, int cols, int64_t x_row_stride, void* packed,
                   int64_t packed_row_stride, void* scales, int64_t scale_row_stride, void* stream) {
  if (rows < 0 || cols < 32 || (cols % 32) != 0)
    return set_error(MLA_ERR_INVALID_ARGUMENT, "cols must be a positive multiple of 32 (got %d)", cols);
  if (rows == 0) return MLA_OK;
  if (!x_bf16 || !packed || !scales) return set_error(MLA_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (x_row_stride < 2LL * cols || (x_row_stride % 16) != 0 || !aligned(x_bf16, 16))
    return set_error(MLA_ERR_INVALID_ARGUMENT, "x rows must be 16-byte aligned with stride >= 2*cols");
  if (packed_row_stride < cols / 2 || (packed_row_stride % 16) != 0 || !aligned(packed, 16))
    return set_error(MLA_ERR_INVALID_ARGUMENT, "packed rows must be 16-byte aligned with stride >= cols/2");
  if (scale_row_stride < cols / 32)
    return set_error(MLA_ERR_INVALID_ARGUMENT, "scale_row_stride must be >= cols/32");
  hipError_t e = launch_pack_mxfp4(static_cast<const uint16_t*>(x_bf16), rows, cols, x_row_stride,
                                   static_cast<uint8_t*>(packed), packed_row_stride,
                                   static_cast<uint8_t*>(scales), scale_row_stride,
                                   static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "pack launch");
  return MLA_OK;
}

int mla_append_kv(const void* x_bf16, int64_t n, int64_t x_row_stride, const int32_t* slots,
                  void* fp8_cache, int64_t fp8_row_stride, const float* fp8_scale, void* fp4_cache,
                  int64_t fp4_row_stride, void* fp4_scales, int64_t fp4_scale_stride, uint32_t* amax_out,
                  void* stream) {
  if (n < 0 || n > kAppendMaxTokens)
    return set_error(MLA_ERR_INVALID_ARGUMENT, "n must be in [0, %lld] (got %lld)", (long long)kAppendMaxTokens,
                (long long)n);
  if (!fp8_cache && !fp4_cache) return set_error(MLA_ERR_INVALID_ARGUMENT, "no cache to write (both NULL)");
  if (n == 0) return MLA_OK;
  if (!x_bf16) return set_error(MLA_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (x_row_stride < 2LL * kQKDim || (x_row_stride % 16) != 0 || !aligned(x_bf16, 16))
    return set_error(MLA_ERR_INVALID_ARGUMENT, "x rows must be 16-byte aligned with stride >= 1152 bytes");
  if (fp8_cache) {
    if (!fp8_scale) return set_error(MLA_ERR_INVALID_ARGUMENT, "fp8_cache needs fp8_scale");
    if (fp8_row_stride < kQKDim || (fp8_row_stride % 16) != 0 || !aligned(fp8_cache, 16))
      return set_error(MLA_ERR_INVALID_ARGUMENT, "fp8 cache rows must be 16-byte aligned with stride >= 576");
  }
  if (fp4_cache) {
    if (!fp4_scales) return set_error(MLA_ERR_INVALID_ARGUMENT, "fp4_cache needs fp4_scales");
    if (fp4_row_stride < kFp4RowBytes || (fp4_row_stride % 16) != 0 || !aligned(fp4_cache, 16))
      return set_error(MLA_ERR_INVALID_ARGUMENT, "mxfp4 cache rows must be 16-byte aligned with stride >= 288");
    if (fp4_scale_stride < kMxBlocks)
      return set_error(MLA_ERR_INVALID_ARGUMENT, "fp4_scale_stride must be >= 18");
  }
  hipError_t e = launch_append_kv(static_cast<const uint16_t*>(x_bf16), n, x_row_stride, slots,
                                  static_cast<uint8_t*>(fp8_cache), fp8_row_stride, fp8_scale,
                                  static_cast<uint8_t*>(fp4_cache), fp4_row_stride,
                                  static_cast<uint8_t*>(fp4_scales), fp4_scale_stride, amax_out,
                                  static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "append launch");
  return MLA_OK;
}

int mla_expand_pages(const int32_t* page_indptr, const int32_t* page_ids, const int32_t* last_page_lens,
                     int batch, int page_size, int64_t max_pages, int32_t* kv_indptr_out,
                     int32_t* kv_indices_out, void* stream) {
  if (batch < 1) return set_error(MLA_ERR_INVALID_ARGUMENT, "batch must be >= 1 (got %d)", batch);
  if (page_size < 1 || page_size > 65536)
    return set_error(MLA_ERR_INVALID_ARGUMENT, "page_size must be in [1, 65536] (got %d)", page_size);
  if (max_pages < 0 || max_pages * (int64_t)page_size >= (int64_t(1) << 31))
    return set_error(MLA_ERR_INVALID_ARGUMENT,
                     "max_pages * page_size must stay below 2^31 token rows (got %lld x %d)",
                     (long long)max_pages, page_size);
  if (!page_indptr || !last_page_lens || !kv_indptr_out || (max_pages > 0 && (!page_ids || !kv_indices_out)))
    return set_error(MLA_ERR_INVALID_ARGUMENT, "null pointer argument");
  hipError_t e = launch_expand_pages(page_indptr, page_ids, last_page_lens, batch, page_size, max_pages,
                                     kv_indptr_out, kv_indices_out, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "expand_pages launch");
  return MLA_OK;
}

int mla_plan(const int32_t* kv_indptr, int batch, int q_seq_len, int num_heads, int kv_mode, void* workspace,
             int64_t workspace_bytes, void* stream) {
  int rc = check_shape(batch, num_heads, kv_mode);
  if (rc) return rc;
  if ((rc = check_qlen(batch, q_seq_len))) return rc;
  if (!kv_indptr || !workspace) return set_error(MLA_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (!aligned(workspace, 256)) return set_error(MLA_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
  int ncu = 0;
  if ((rc = cu_count(&ncu))) return rc;
  WsLayout L = workspace_layout(batch, num_heads, kv_mode, ncu);
  if (workspace_bytes < L.total)
    return set_error(MLA_ERR_WORKSPACE_TOO_SMALL, "workspace needs %lld bytes (got %lld)", (long long)L.total,
                (long long)workspace_bytes);
  int32_t* plan = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + L.plan_off);
  hipError_t e = launch_plan(kv_indptr, batch, q_seq_len, plan_target_for(batch, num_heads, kv_mode, ncu, false),
                             L.max_items, plan,
                             static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "plan launch");
  return MLA_OK;
}

int mla_decode(const void* q_fp8, const float* q_scale, const void* k_cache, int64_t k_row_stride,
               const void* k_scales, int64_t k_scale_stride, const void* v_cache, int64_t v_row_stride,
               const float* kv_scale, const int32_t* kv_indptr, const int32_t* kv_indices, int batch,
               int num_heads, float sm_scale, int kv_mode, void* workspace, int64_t workspace_bytes,
               void* out_bf16, float* lse_out, void* stream) {
  if (kv_mode == MLA_KV_BF16)
    return set_error(MLA_ERR_UNSUPPORTED, "the bf16 cache takes bf16 Q: use mla_decode_fwd (kv_mode bf16)");
  DecodeParams p{};
  WsLayout L;
  int rc = decode_params(q_fp8, q_scale, k_cache, k_row_stride, k_scales, k_scale_stride, v_cache,
                         v_row_stride, kv_scale, kv_indptr, kv_indices, batch, num_heads, sm_scale,
                         kv_mode, workspace, workspace_bytes, out_bf16, lse_out, &p, &L);
  if (rc) return rc;
  hipError_t e = launch_decode(p, kv_mode, L.max_items, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "decode launch");
  return MLA_OK;
}

int mla_combine(int batch, int num_heads, void* workspace, int64_t workspace_bytes, void* out_bf16,
                float* lse_out, void* stream) {
  int rc = check_shape(batch, num_heads, MLA_KV_FP8);
  if (rc) return rc;
  if (!workspace || !out_bf16) return set_error(MLA_ERR_INVALID_ARGUMENT, "null pointer argument");
  int ncu = 0;
  if ((rc = cu_count(&ncu))) return rc;
  WsLayout L = workspace_layout(batch, num_heads, MLA_KV_FP8, ncu);
  if (workspace_bytes < L.total)
    return set_error(MLA_ERR_WORKSPACE_TOO_SMALL, "workspace needs %lld bytes (got %lld)", (long long)L.total,
                (long long)workspace_bytes);
  char* ws = static_cast<char*>(workspace);
  DecodeParams p = {};
  p.plan = reinterpret_cast<const int32_t*>(ws + L.plan_off);
  p.part_o = reinterpret_cast<uint16_t*>(ws + L.part_o_off);
  p.part_lse = reinterpret_cast<float*>(ws + L.part_lse_off);
  p.out = static_cast<uint16_t*>(out_bf16);
  p.lse_out = lse_out;
  p.batch = batch;
  p.num_heads = num_heads;
  p.max_items = L.max_items;
  hipError_t e = launch_combine(p, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "combine launch");
  return MLA_OK;
}

int mla_decode_fwd(const void* q_bf16, const void* k_cache, int64_t k_row_stride, const void* k_scales,
                   int64_t k_scale_stride, const void* v_cache, int64_t v_row_stride,
                   const float* kv_scale, const int32_t* kv_indptr, const int32_t* kv_indices, int batch,
                   int q_seq_len, int num_heads, float sm_scale, int kv_mode, void* workspace,
                   int64_t workspace_bytes, void* out_bf16, float* lse_out, void* stream) {
  if (!q_bf16 || !aligned(q_bf16, 16)) return set_error(MLA_ERR_INVALID_ARGUMENT, "q must be non-null and 16-byte aligned");
  if (!workspace) return set_error(MLA_ERR_INVALID_ARGUMENT, "null workspace");
  char* ws = static_cast<char*>(workspace);
  int rc = check_shape(batch, num_heads, kv_mode);
  if (rc) return rc;
  if ((rc = check_qlen(batch, q_seq_len))) return rc;
  int ncu = 0;
  if ((rc = cu_count(&ncu))) return rc;
  WsLayout L0 = workspace_layout(batch, num_heads, kv_mode, ncu);
  if (workspace_bytes < L0.total)
    return set_error(MLA_ERR_WORKSPACE_TOO_SMALL, "workspace needs %lld bytes (got %lld)", (long long)L0.total,
                (long long)workspace_bytes);
  uint8_t* q_fp8 = reinterpret_cast<uint8_t*>(ws + L0.qfp8_off);
  float* q_scale = reinterpret_cast<float*>(ws + L0.quant_off + 4096);
  DecodeParams p{};
  WsLayout L;
  rc = decode_params(q_fp8, q_scale, k_cache, k_row_stride, k_scales, k_scale_stride, v_cache,
                     v_row_stride, kv_scale, kv_indptr, kv_indices, batch, num_heads, sm_scale, kv_mode,
                     workspace, workspace_bytes, out_bf16, lse_out, &p, &L);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n = (int64_t)batch * num_heads * kQKDim;
  uint32_t* partials = reinterpret_cast<uint32_t*>(ws + L.quant_off);
  int nb = 0;
  if (kv_mode == MLA_KV_BF16) {  // a16w16: Q is used as it is, no amax pass
    hipError_t e = launch_plan(kv_indptr, batch, q_seq_len,
                               plan_target_for(batch, num_heads, kv_mode, ncu, kv_indices == nullptr),
                               L.max_items, reinterpret_cast<int32_t*>(ws + L.plan_off), s);
    if (e != hipSuccess) return hip_fail(e, "plan launch");
    p.q_bf16 = static_cast<const uint16_t*>(q_bf16);
    e = launch_decode(p, kv_mode, L.max_items, s);
    if (e != hipSuccess) return hip_fail(e, "decode launch");
    e = launch_combine(p, s);
    if (e != hipSuccess) return hip_fail(e, "combine launch");
    return MLA_OK;
  }
  hipError_t e = launch_amax(static_cast<const uint16_t*>(q_bf16), n, partials, &nb, kv_indptr,
                             static_cast<const int32_t*>(kv_indices), batch, q_seq_len,
                             plan_target_for(batch, num_heads, kv_mode, ncu, kv_indices == nullptr),
                             L.max_items, reinterpret_cast<int32_t*>(ws + L.plan_off), s);
  if (e != hipSuccess) return hip_fail(e, "amax+plan launch");
  if (num_heads == 16) {
    // the H = 16 kernel quantizes its sequence's Q from the amax partials
    p.q_bf16 = static_cast<const uint16_t*>(q_bf16);
    p.q_partials = partials;
    p.q_nparts = nb;
  } else {
    e = launch_quant_fp8(static_cast<const uint16_t*>(q_bf16), n, partials, nb, q_fp8, q_scale, s);
    if (e != hipSuccess) return hip_fail(e, "quant launch");
  }
  e = launch_decode(p, kv_mode, L.max_items, s);
  if (e != hipSuccess) return hip_fail(e, "decode launch");
  e = launch_combine(p, s);
  if (e != hipSuccess) return hip_fail(e, "combine launch");
  return MLA_OK;
}

int mla_decode_fwd_a16w8(const void* q_bf16, const void* k_cache, int64_t k_row_stride, const void* k_scales,
                         int64_t k_scale_stride, const void* v_cache, int64_t v_row_stride,
                         const float* kv_scale, const int32_t* kv_indptr, const int32_t* kv_indices, int batch,
                         int q_seq_len, int num_heads, float sm_scale, int kv_mode, void* workspace,
                         int64_t workspace_bytes, void* out_bf16, float* lse_out, void* stream) {
  if (num_heads != 16 || kv_mode != 0)
    return set_error(MLA_ERR_UNSUPPORTED, "the a16w8 route takes 16 heads and the fp8 cache (got %d, kv_mode %d)",
                     num_heads, kv_mode);
  if (!q_bf16 || !aligned(q_bf16, 16)) return set_error(MLA_ERR_INVALID_ARGUMENT, "q must be non-null and 16-byte aligned");
  if (!workspace) return set_error(MLA_ERR_INVALID_ARGUMENT, "null workspace");
  int rc = check_shape(batch, num_heads, kv_mode);
  if (rc) return rc;
  if ((rc = check_qlen(batch, q_seq_len))) return rc;
  int ncu = 0;
  if ((rc = cu_count(&ncu))) return rc;
  WsLayout L0 = workspace_layout(batch, num_heads, kv_mode, ncu);
  if (workspace_bytes < L0.total)
    return set_error(MLA_ERR_WORKSPACE_TOO_SMALL, "workspace needs %lld bytes (got %lld)", (long long)L0.total,
                     (long long)workspace_bytes);
  char* ws = static_cast<char*>(workspace);
  DecodeParams p{};
  WsLayout L;
  // the fp8 Q slots of the workspace are not read on this route
  rc = decode_params(ws + L0.qfp8_off, reinterpret_cast<const float*>(ws + L0.quant_off + 4096), k_cache,
                     k_row_stride, k_scales, k_scale_stride, v_cache, v_row_stride, kv_scale, kv_indptr,
                     kv_indices, batch, num_heads, sm_scale, kv_mode, workspace, workspace_bytes, out_bf16,
                     lse_out, &p, &L);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = launch_plan(kv_indptr, batch, q_seq_len,
                             plan_target_for(batch, num_heads, kv_mode, ncu, kv_indices == nullptr),
                             L.max_items, reinterpret_cast<int32_t*>(ws + L.plan_off), s);
  if (e != hipSuccess) return hip_fail(e, "plan launch");
  p.q_bf16 = static_cast<const uint16_t*>(q_bf16);  // no partials: each work-group scales its own Q rows
  e = launch_decode(p, kv_mode, L.max_items, s);
  if (e != hipSuccess) return hip_fail(e, "decode launch");
  e = launch_combine(p, s);
  if (e != hipSuccess) return hip_fail(e, "combine launch");
  return MLA_OK;
}

int mla_decode_fwd_rowq(const void* q_bf16, const void* k_cache, int64_t k_row_stride, const void* k_scales,
                        int64_t k_scale_stride, const void* v_cache, int64_t v_row_stride,
                        const float* kv_scale, const int32_t* kv_indptr, const int32_t* kv_indices, int batch,
                        int q_seq_len, int num_heads, float sm_scale, int kv_mode, void* workspace,
                        int64_t workspace_bytes, void* out_bf16, float* lse_out, void* stream) {
  if (num_heads != 16 || (kv_mode != MLA_KV_FP8 && kv_mode != MLA_KV_MXFP4))
    return set_error(MLA_ERR_UNSUPPORTED,
                     "the per-row Q route takes 16 heads and the fp8 or mxfp4 cache (got %d, kv_mode %d)", num_heads,
                     kv_mode);
  if (!q_bf16 || !aligned(q_bf16, 16)) return set_error(MLA_ERR_INVALID_ARGUMENT, "q must be non-null and 16-byte aligned");
  if (!workspace) return set_error(MLA_ERR_INVALID_ARGUMENT, "null workspace");
  int rc = check_shape(batch, num_heads, kv_mode);
  if (rc) return rc;
  if ((rc = check_qlen(batch, q_seq_len))) return rc;
  int ncu = 0;
  if ((rc = cu_count(&ncu))) return rc;
  WsLayout L0 = workspace_layout(batch, num_heads, kv_mode, ncu);
  if (workspace_bytes < L0.total)
    return set_error(MLA_ERR_WORKSPACE_TOO_SMALL, "workspace needs %lld bytes (got %lld)", (long long)L0.total,
                     (long long)workspace_bytes);
  char* ws = static_cast<char*>(workspace);
  DecodeParams p{};
  WsLayout L;
  // the fp8 Q slots of the workspace are not read on this route
  rc = decode_params(ws + L0.qfp8_off, reinterpret_cast<const float*>(ws + L0.quant_off + 4096), k_cache,
                     k_row_stride, k_scales, k_scale_stride, v_cache, v_row_stride, kv_scale, kv_indptr,
                     kv_indices, batch, num_heads, sm_scale, kv_mode, workspace, workspace_bytes, out_bf16,
                     lse_out, &p, &L);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const PlanTarget t = plan_target_for(batch, num_heads, kv_mode, ncu, kv_indices == nullptr);
  p.q_bf16 = static_cast<const uint16_t*>(q_bf16);
  p.q_per_row = 1;
  int grid = L.max_items;
  hipError_t e;
  if (batch <= 256) {
    // the decode plans its own work (one wave up to 64 rows, the block up to
    // 256): one launch fewer; at most max(t.items, batch) items (the chunk
    // search keeps the count within the target, or one piece per row)
    p.plan_here = 1;
    p.plan_qlen = q_seq_len;
    p.plan_target = t.items;
    p.plan_min_chunk = t.min_chunk;
    p.plan_max_splits = t.max_splits;
    grid = t.items + batch < L.max_items ? t.items + batch : L.max_items;
  } else {
    e = launch_plan(kv_indptr, batch, q_seq_len, t, L.max_items, reinterpret_cast<int32_t*>(ws + L.plan_off), s);
    if (e != hipSuccess) return hip_fail(e, "plan launch");
  }
  e = launch_decode(p, kv_mode, grid, s);
  if (e != hipSuccess) return hip_fail(e, "decode launch");
  e = launch_combine(p, s);
  if (e != hipSuccess) return hip_fail(e, "combine launch");
  return MLA_OK;
}

int mla_absorb_q(const void* q_nope, const void* q_rope, const void* w_uk, int batch, int num_heads,
                 void* q_out, void* stream) {
  if (batch < 1 || num_heads < 1 || num_heads > 65535)
    return set_error(MLA_ERR_INVALID_ARGUMENT, "batch must be >= 1 and num_heads in [1, 65535] (got %d, %d)", batch,
                num_heads);
  if (!q_nope || !q_rope || !w_uk || !q_out) return set_error(MLA_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (!aligned(q_nope, 16) || !aligned(q_rope, 16) || !aligned(w_uk, 16) || !aligned(q_out, 16))
    return set_error(MLA_ERR_INVALID_ARGUMENT, "q_nope, q_rope, w_uk and q_out must be 16-byte aligned");
  hipError_t e = launch_absorb_q(static_cast<const uint16_t*>(q_nope), static_cast<const uint16_t*>(q_rope),
                                 static_cast<const uint16_t*>(w_uk), batch, num_heads,
                                 static_cast<uint16_t*>(q_out), static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "absorb launch");
  return MLA_OK;
}

int mla_v_up_proj(const void* o, const void* w_uv, int batch, int num_heads, void* y_bf16, void* out_fp8,
                  float* out_scale, void* workspace, int64_t workspace_bytes, void* stream) {
  if (batch < 1 || num_heads < 1 || num_heads > kUpProjMaxHeads)
    return set_error(MLA_ERR_INVALID_ARGUMENT, "batch must be >= 1 and num_heads in [1, %d] (got %d, %d)",
                kUpProjMaxHeads, batch, num_heads);
  if (!o || !w_uv || !y_bf16) return set_error(MLA_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (!aligned(o, 16) || !aligned(w_uv, 16) || !aligned(y_bf16, 16))
    return set_error(MLA_ERR_INVALID_ARGUMENT, "o, w_uv and y must be 16-byte aligned");
  const bool fp8 = out_fp8 != nullptr;
  if (fp8) {
    if (!out_scale || !workspace) return set_error(MLA_ERR_INVALID_ARGUMENT, "the fp8 output needs out_scale and workspace");
    if (!aligned(out_fp8, 8) || !aligned(workspace, 16))
      return set_error(MLA_ERR_INVALID_ARGUMENT, "out_fp8 must be 8-byte and workspace 16-byte aligned");
    if (workspace_bytes < kQuantScratchBytes)
      return set_error(MLA_ERR_WORKSPACE_TOO_SMALL, "workspace needs %lld bytes", (long long)kQuantScratchBytes);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* partials = fp8 ? static_cast<uint32_t*>(workspace) : nullptr;
  int nparts = 0;
  hipError_t e = launch_v_up_proj(static_cast<const uint16_t*>(o), static_cast<const uint16_t*>(w_uv), batch,
                                  num_heads, static_cast<uint16_t*>(y_bf16), partials, &nparts, s);
  if (e != hipSuccess) return hip_fail(e, "v_up_proj launch");
  if (fp8) {
    e = launch_quant_fp8(static_cast<const uint16_t*>(y_bf16), (int64_t)batch * num_heads * 128, partials,
                         nparts, static_cast<uint8_t*>(out_fp8), out_scale, s);
    if (e != hipSuccess) return hip_fail(e, "quant launch");
  }
  return MLA_OK;
}

int mla_selftest(int which, const void* in, void* out, void* stream) {
  if (!in || !out) return set_error(MLA_ERR_INVALID_ARGUMENT, "null pointer argument");
  hipError_t e = launch_selftest(which, in, out, static_cast<hipStream_t>(stream));
  if (e == hipErrorInvalidValue) return set_error(MLA_ERR_INVALID_ARGUMENT, "unknown selftest %d", which);
  if (e != hipSuccess) return hip_fail(e, "selftest launch");
  return MLA_OK;
}

}  // extern "C"
