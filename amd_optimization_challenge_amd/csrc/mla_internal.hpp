// Host-side declarations shared between the library's translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mla_common.hpp"

namespace mla {

// Blocks used by the amax pass (also the number of partial maxima written).
constexpr int kAmaxMaxBlocks = 1024;
// Largest token count of one mla_append_kv call (72 lanes per token stay below 2^31).
constexpr int64_t kAppendMaxTokens = (1LL << 31) / (kQKDim / 8);
// Byte size of the quantizer scratch area at the front of every workspace.
constexpr int64_t kQuantScratchBytes = 8192;
// Device scratch of mla_decode_fwd_noalloc (per device, held until exit).
constexpr int64_t kNoAllocScratchBytes = 64LL << 20;

// Records the thread's last error message (mla_last_error) and returns code.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Workspace carve-up for one decode call; every offset is 256-byte aligned.
struct WsLayout {
  int64_t quant_off;   // kQuantScratchBytes: amax partials [1024] u32, q_scale f32 at +4096
  int64_t qfp8_off;    // B*H*576 bytes
  int64_t plan_off;    // (kPlanHeader + 4*max_items + 2*B) int32
  int64_t part_o_off;  // max_items*H*512 bf16
  int64_t part_lse_off;// max_items*H f32
  int64_t total;
  int max_items;
  int target_items;
};

// What the split planner aims for: `items` work items, a chunk (longest
// piece) of at least `min_chunk` tokens (a multiple of 64), and, when
// max_splits > 0, no sequence cut into more than max_splits pieces.
struct PlanTarget {
  int items;
  int min_chunk;
  int max_splits;
};
// smallest chunk by default: a piece of two tiles at least, so that short
// batches are not cut into one-tile items whose fixed costs (ring start,
// partial write, combine input) exceed their work
constexpr int kPlanMinChunk = 128;

int target_items_for(int batch, int num_heads, int kv_mode, int num_cu);
PlanTarget plan_target_for(int batch, int num_heads, int kv_mode, int num_cu, bool contiguous);
WsLayout workspace_layout(int batch, int num_heads, int kv_mode, int num_cu);

// quant.hip
hipError_t launch_amax(const uint16_t* x, int64_t n, uint32_t* partials, int* nblocks,
                       const int32_t* kv_indptr, const int32_t* kv_indices, int batch, int qlen,
                       PlanTarget target, int max_items, int32_t* plan, hipStream_t stream);
// partials: 16-byte aligned, nblocks <= kAmaxMaxBlocks maxima (read four at a
// time, so up to three words past nblocks are read and ignored)
hipError_t launch_quant_fp8(const uint16_t* x, int64_t n, const uint32_t* partials, int nblocks,
                            uint8_t* out, float* out_scale, hipStream_t stream);
hipError_t launch_pack_mxfp4(const uint16_t* x, int64_t rows, int cols, int64_t x_stride,
                             uint8_t* packed, int64_t packed_stride, uint8_t* scales,
                             int64_t scale_stride, hipStream_t stream);
hipError_t launch_plan(const int32_t* kv_indptr, int batch, int qlen, PlanTarget target, int max_items,
                       int32_t* plan, hipStream_t stream);
hipError_t launch_expand_pages(const int32_t* page_indptr, const int32_t* page_ids, const int32_t* last_page_lens,
                               int batch, int page_size, int64_t max_pages, int32_t* kv_indptr_out,
                               int32_t* kv_indices_out, hipStream_t stream);
hipError_t launch_append_kv(const uint16_t* x, int64_t n, int64_t x_stride, const int32_t* slots,
                            uint8_t* fp8_cache, int64_t fp8_stride, const float* fp8_scale,
                            uint8_t* fp4_cache, int64_t fp4_stride, uint8_t* fp4_scales,
                            int64_t fp4_scale_stride, uint32_t* amax_out, hipStream_t stream);

// decode.hip
hipError_t launch_decode(const DecodeParams& p, int kv_mode, int grid, hipStream_t stream);
hipError_t launch_combine(const DecodeParams& p, hipStream_t stream);
// decode_h128.hip: H = 128 with the fp8 cache
hipError_t launch_decode_h128f(const DecodeParams& p, int grid, hipStream_t stream);
hipError_t launch_decode_h128m(const DecodeParams& p, int grid, hipStream_t stream);

// neighbours.hip
hipError_t launch_absorb_q(const uint16_t* q_nope, const uint16_t* q_rope, const uint16_t* w_uk, int batch,
                           int heads, uint16_t* q_out, hipStream_t stream);
hipError_t launch_v_up_proj(const uint16_t* o, const uint16_t* w_uv, int batch, int heads, uint16_t* y,
                            uint32_t* amax_partials, int* nparts, hipStream_t stream);
// Largest head count of v_up_proj with the FP8 output (one partial max per
// head and 32-column slice, kAmaxMaxBlocks in all).
constexpr int kUpProjMaxHeads = kAmaxMaxBlocks / 4;

// selftest.hip
hipError_t launch_selftest(int which, const void* in, void* out, hipStream_t stream);

}  // namespace mla
