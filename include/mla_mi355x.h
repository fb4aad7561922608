/*
 * mla_mi355x.h -- C ABI of the MI355X (gfx950) MLA absorbed-decode operator.
 *
 * Every entry point is `extern "C"`, takes plain device pointers, sizes and a
 * HIP stream handle (`void*`, 0 = the null stream), never synchronizes the
 * host, never allocates device memory, and returns an `int` status
 * (MLA_OK = 0).  On failure `mla_last_error()` returns a message for the
 * calling thread.  All device memory is caller-owned; scratch lives in the
 * caller-provided workspace whose size `mla_workspace_bytes` reports.
 *
 * `batch` counts query rows: sequences x q_seq_len, the q_seq_len rows of a
 * sequence consecutive.  Row i of a sequence with L keys attends to its first
 * L - (q_seq_len - 1 - i) keys (the uniform-qo_len causal decode of
 * competitor_submissions/mi355x_reference/reference.py:188-193); q_seq_len = 1
 * is plain decode.
 *
 * Layouts (row-major, byte strides given in bytes), S = batch / q_seq_len:
 *   q            [batch, num_heads, 576]  bf16
 *   q_fp8        [batch, num_heads, 576]  float8 e4m3fn (OCP)
 *   fp8 cache    [slots, 576]             e4m3fn, one per-tensor f32 scale
 *   mxfp4 cache  [slots, 288]             e2m1 pairs, low nibble = even element
 *   mxfp4 scales [slots, scale_stride]    e8m0, first 18 used (stride >= 18)
 *   kv_indptr    [S + 1]                  int32, token offsets into kv_indices
 *   kv_indices   [kv_indptr[S]]           int32 cache slot per token (page size 1);
 *                                         NULL means identity (slot = offset)
 *   out          [batch, num_heads, 512]  bf16
 *   lse_out      [batch, num_heads]       f32 ln sum exp(scores), optional (NULL =
 *                                         not written); -inf for a row with no keys
 *
 * References below are path:line in dorhuri123/AMD_optimization_challenge.
 */
#ifndef MLA_MI355X_H
#define MLA_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define MLA_OK 0
#define MLA_ERR_INVALID_ARGUMENT 1
#define MLA_ERR_UNSUPPORTED 2
#define MLA_ERR_WORKSPACE_TOO_SMALL 3
#define MLA_ERR_HIP 4

/* kv_mode: which cache feeds the scores (K, 576 dims) and the values (V, 512 dims) */
#define MLA_KV_FP8 0          /* K = V = fp8 cache (V = first 512 dims)            */
#define MLA_KV_MXFP4 1        /* K = V = mxfp4 cache (V = first 256 B + 16 scales)   */
#define MLA_KV_MXFP4K_FP8V 2  /* K = mxfp4 cache, V = first 512 dims of fp8 cache    */
#define MLA_KV_BF16 3         /* K = V = bf16 cache (a16w16; V = first 512 dims),     */
                              /* 16 heads, mla_decode_fwd only (Q used as given)      */

/* Message describing the last failure on this thread ("" if none). */
const char* mla_last_error(void);

/* ABI version, bumped on any signature change (2: q_seq_len, lse_out). */
int mla_abi_version(void);

/* Number of compute units on the current device (used by the split planner). */
int mla_device_cu_count(int* num_cu);

/*
 * Workspace size for one decode call of this shape.  Replaces the buffer sizing
 * of AITER's get_mla_metadata_info_v1 (competitor_submissions/mi355x_reference/
 * reference.py:174-179) plus the logits/lse allocations of mla_decode_fwd
 * (mixed-mla/asm_dumps/aiter_mla.py:357-366).
 */
int mla_workspace_bytes(int batch, int num_heads, int kv_mode, int64_t* bytes);

/*
 * Per-tensor FP8 quantization of n bf16 values: amax -> scale = bf16(amax/448)
 * -> e4m3fn(clamp(bf16(x/scale), +-448)), bit-exact to quantize_fp8
 * (competitor_submissions/mi355x_reference/reference.py:65-80).  Writes the f32
 * scale to out_scale[0].  workspace needs >= 8 KiB; it is left reusable.
 */
int mla_quant_fp8_per_tensor(const void* x_bf16, int64_t n, void* out_fp8,
                             float* out_scale, void* workspace,
                             int64_t workspace_bytes, void* stream);

/*
 * MXFP4 pack of `rows` bf16 rows of `cols` elements (cols % 32 == 0): one e8m0
 * per 32 elements plus e2m1 nibbles, bit-exact to quantize_mxfp4 /
 * dynamic_mxfp4_quant (competitor_submissions/mi355x_reference/reference.py:88-113,
 * algorithm restated at mxfp4-mm/submission_v18_custom_fused.py:26-108).
 * Strides in bytes.  Scale columns beyond cols/32 are not written.
 */
int mla_pack_mxfp4(const void* x_bf16, int64_t rows, int cols, int64_t x_row_stride,
                   void* packed, int64_t packed_row_stride, void* scales,
                   int64_t scale_row_stride, void* stream);

/*
 * W_UK absorption, the step before the decode: q_out [batch, H, 576] bf16 =
 * [q_nope[b, h] @ w_uk[h], q_rope[b, h]] for q_nope [batch, H, 128], q_rope
 * [batch, H, 64], w_uk [H, 128, 512] (bf16, contiguous, 16-byte aligned); f32
 * accumulation, one bf16 rounding.  The reference names this step of
 * DeepSeek-style MLA but has no implementation of it (mixed-mla/README.md:213-217).
 */
int mla_absorb_q(const void* q_nope, const void* q_rope, const void* w_uk, int batch, int num_heads,
                 void* q_out, void* stream);

/*
 * v_up_proj, the step after the decode: y_bf16 [batch, H, 128] = o[b, h] @
 * w_uv[h] for o [batch, H, 512] (the decode output), w_uv [H, 512, 128] (bf16,
 * contiguous, 16-byte aligned), 1 <= H <= 256.  out_fp8 (optional): the
 * per-tensor FP8 quantization of y_bf16, as mla_quant_fp8_per_tensor gives it,
 * with its scale in out_scale[0]; it needs a workspace of >= 8 KiB.  No
 * counterpart in the reference, which names the step (mixed-mla/README.md:213-217).
 */
int mla_v_up_proj(const void* o, const void* w_uv, int batch, int num_heads, void* y_bf16, void* out_fp8,
                  float* out_scale, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * KV-cache append: writes n new tokens (bf16 [n, 576], row stride in bytes)
 * into cache rows slots[i] (page size 1; slots == NULL means row i; a negative
 * slot skips its token; slots must be distinct; n <= 29826161 per call).
 * Either cache may be NULL, not both.
 *   fp8 cache   : e4m3fn(clamp(bf16(x / fp8_scale[0]), +-448)) with the
 *                 cache's existing per-tensor scale -- the bytes quantize_fp8
 *                 gives for the whole buffer when its scale is fp8_scale[0]
 *   mxfp4 cache : e2m1 pairs + e8m0 per 32 elements, bit-exact to
 *                 dynamic_mxfp4_quant of the row; scale stride >= 18 (padded
 *                 columns are not written)
 * amax_out (optional, device u32) is max-ed with the bf16 bits of max|x| over
 * the written tokens; tokens above 448 * fp8_scale saturate in the fp8 cache,
 * which the caller detects by comparing it with the scale.  The reference
 * builds its caches whole (competitor_submissions/mi355x_reference/
 * reference.py:318-321, layout competitor_submissions/mi355x_reference/
 * README.md:57-81); this is the incremental writer of the same bytes.
 */
int mla_append_kv(const void* x_bf16, int64_t n, int64_t x_row_stride, const int32_t* slots,
                  void* fp8_cache, int64_t fp8_row_stride, const float* fp8_scale, void* fp4_cache,
                  int64_t fp4_row_stride, void* fp4_scales, int64_t fp4_scale_stride, uint32_t* amax_out,
                  void* stream);

/*
 * Paged caches.  Expands AITER's page table -- page_indptr [batch + 1] over
 * pages, page_ids (page index per page slot), last_page_lens [batch] and
 * page_size, the arguments of mla_decode_fwd at
 * mixed-mla/asm_dumps/aiter_mla.py:149-175 (built as at
 * mixed-mla/submission.py:449-456, :538-544) -- into the token-level
 * kv_indptr_out [batch + 1] and kv_indices_out (at most max_pages * page_size
 * entries) that every decode entry point takes, addressing the cache viewed as
 * [pages * page_size, row].  Sequence b holds (n_b - 1) * page_size + last_b
 * tokens for n_b > 0 pages (last_b clamped to [1, page_size]).  max_pages is
 * the length of page_ids; page_ids * page_size must stay below 2^31.
 */
int mla_expand_pages(const int32_t* page_indptr, const int32_t* page_ids, const int32_t* last_page_lens,
                     int batch, int page_size, int64_t max_pages, int32_t* kv_indptr_out,
                     int32_t* kv_indices_out, void* stream);

/*
 * Split-KV work partition, computed on the device from kv_indptr (no host
 * sync).  Replaces get_mla_metadata_v1
 * (competitor_submissions/mi355x_reference/reference.py:161-209) and the
 * uniform cdiv split of mixed-mla/submission.py:158-160; q_seq_len is the
 * reference's max_seqlen_qo with is_causal (reference.py:188-193).  The plan
 * lives in the workspace and is consumed by mla_decode / mla_combine.
 */
int mla_plan(const int32_t* kv_indptr, int batch, int q_seq_len, int num_heads, int kv_mode,
             void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Split-KV decode over a plan made by mla_plan: per work item, QK^T over the
 * 576-d latent and PV over the 512-d latent with an online softmax; finished
 * sequences are written to `out`, split ones to workspace partials.  Replaces
 * mla_decode_stage1_asm_fwd (mixed-mla/asm_dumps/aiter_mla.py:398-419).
 *   fp8 K   : k_cache = fp8 cache, k_row_stride >= 576, k_scales unused
 *   mxfp4 K : k_cache = packed cache (row stride >= 288), k_scales = e8m0
 *   fp8 V   : v_cache = fp8 cache (row stride >= 512), kv_scale = its scale
 *   mxfp4 V : same rows as K (v_cache ignored)
 * Scores are (q_fp8*q_scale).(k*k_scale) * sm_scale.  lse_out (optional) gets
 * the rows written here, as mla_decode_fwd's return_lse
 * (mixed-mla/asm_dumps/aiter_mla.py:367-371).
 */
int mla_decode(const void* q_fp8, const float* q_scale, const void* k_cache,
               int64_t k_row_stride, const void* k_scales, int64_t k_scale_stride,
               const void* v_cache, int64_t v_row_stride, const float* kv_scale,
               const int32_t* kv_indptr, const int32_t* kv_indices, int batch,
               int num_heads, float sm_scale, int kv_mode, void* workspace,
               int64_t workspace_bytes, void* out_bf16, float* lse_out, void* stream);

/*
 * Log-sum-exp merge of the split partials of every split sequence into `out`
 * (bf16), and their lse into lse_out when it is not NULL.  Replaces
 * mla_reduce_v1 (mixed-mla/asm_dumps/aiter_mla.py:421-430).
 */
int mla_combine(int batch, int num_heads, void* workspace, int64_t workspace_bytes,
                void* out_bf16, float* lse_out, void* stream);

/*
 * The whole operator: quantize q (bf16) to FP8, plan, decode, combine.  This is
 * the C side of custom_kernel(data) (mixed-mla/submission.py:626-644) and of
 * AITER's mla_decode_fwd (mixed-mla/asm_dumps/aiter_mla.py:149-175) with
 * max_seqlen_q = q_seq_len and return_lse = (lse_out != NULL); the per-step
 * entry points above are its stages.
 */
int mla_decode_fwd(const void* q_bf16, const void* k_cache, int64_t k_row_stride,
                   const void* k_scales, int64_t k_scale_stride, const void* v_cache,
                   int64_t v_row_stride, const float* kv_scale,
                   const int32_t* kv_indptr, const int32_t* kv_indices, int batch,
                   int q_seq_len, int num_heads, float sm_scale, int kv_mode, void* workspace,
                   int64_t workspace_bytes, void* out_bf16, float* lse_out, void* stream);

/*
 * The a16w8 route: bf16 Q against the fp8 cache with no tensor-wide Q scale,
 * hence no amax pass -- the reference's bf16-Q paths (AITER's a16w8 decode,
 * mixed-mla/submission.py:86-96 and :414-520 with q left in bf16).  Same
 * arguments as mla_decode_fwd; 16 heads and kv_mode fp8 only
 * (MLA_ERR_UNSUPPORTED otherwise).  Each head row of Q is split into two fp8
 * terms at a power-of-two row scale inside the decode (about the 8
 * significant bits of bf16), so scores are q . (k * kv_scale) * sm_scale with q
 * as given rather than quantized per tensor.
 */
int mla_decode_fwd_a16w8(const void* q_bf16, const void* k_cache, int64_t k_row_stride,
                         const void* k_scales, int64_t k_scale_stride, const void* v_cache,
                         int64_t v_row_stride, const float* kv_scale, const int32_t* kv_indptr,
                         const int32_t* kv_indices, int batch, int q_seq_len, int num_heads,
                         float sm_scale, int kv_mode, void* workspace, int64_t workspace_bytes,
                         void* out_bf16, float* lse_out, void* stream);

/*
 * mla_decode_fwd with Q quantized per head row instead of per tensor: each
 * [576] row of bf16 Q gets the per-tensor rule of quantize_fp8
 * (TASK/reference.py:76-80) with the row as the tensor, inside the decode
 * kernel, so no tensor-wide amax pass runs first; for batch <= 256 query rows
 * the decode kernel also plans its own work, so the call is two launches
 * (decode, combine).  16 heads, the fp8 or the mxfp4 cache.  It replaces the
 * reference's small-shape route, which quantizes Q per 32-element MXFP4 block
 * inside its Triton path for the same reason (mixed-mla/submission.py:321-334);
 * same arguments as mla_decode_fwd.
 */
int mla_decode_fwd_rowq(const void* q_bf16, const void* k_cache, int64_t k_row_stride,
                        const void* k_scales, int64_t k_scale_stride, const void* v_cache,
                        int64_t v_row_stride, const float* kv_scale, const int32_t* kv_indptr,
                        const int32_t* kv_indices, int batch, int q_seq_len, int num_heads,
                        float sm_scale, int kv_mode, void* workspace, int64_t workspace_bytes,
                        void* out_bf16, float* lse_out, void* stream);

/*
 * mla_decode_fwd without a caller workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  Arguments mean what
 * they mean for mla_decode_fwd; the workspace is instead a device array inside
 * the library of mla_noalloc_scratch_bytes() = 64 MiB per device (held from
 * the first call on a device until the process ends).  A shape whose
 * mla_workspace_bytes exceeds it returns MLA_ERR_WORKSPACE_TOO_SMALL.  Calls
 * on one device share that array: calls that overlap on a device (other
 * streams, other threads) race; calls ordered on one stream do not.  It calls
 * no allocator.  The first call on a device resolves the array's address
 * (hipGetSymbolAddress): make it eagerly before capturing a call in a graph.
 */
int mla_decode_fwd_noalloc(const void* q_bf16, const void* k_cache, int64_t k_row_stride,
                           const void* k_scales, int64_t k_scale_stride, const void* v_cache,
                           int64_t v_row_stride, const float* kv_scale,
                           const int32_t* kv_indptr, const int32_t* kv_indices, int batch,
                           int q_seq_len, int num_heads, float sm_scale, int kv_mode,
                           void* out_bf16, float* lse_out, void* stream);

/* Size in bytes of mla_decode_fwd_noalloc's per-device scratch array. */
int64_t mla_noalloc_scratch_bytes(void);

/*
 * Diagnostic (no counterpart in the reference): the decode kernels' KV gather
 * with no compute, to measure the HBM rate a cache layout and issue scheme
 * can reach.  ntokens (a multiple of 64) entries of kv_indices are read in
 * 64-token tiles spread evenly over `groups` work-groups of 64*waves threads.
 *   layout 0: rows = fp8 cache (576 B read per token)
 *   layout 1: rows = mxfp4 cache (288 B) + scales (18 B per token)
 *   layout 2: layout 1 + v_rows = fp8 cache (512 B per token)
 *   method 0: LDS-DMA ring, scales as 6 dword DMAs per tile (the scale buffer
 *             needs 8 readable bytes past its last row's 18)
 *   method 1: LDS-DMA ring, scales as 18 one-byte DMAs per tile
 *   method 2: layout 0 by plain 16-byte loads into registers
 *   method 3: contiguous stream of ntokens * row_stride bytes of rows (no
 *             indices; waves = 4)
 * Supported (layout, method, waves, stages): (0,0,4,2..4), (0,0,8,2|4),
 * (1,0,4,3|4), (1,0,8,4), (1,1,4,3), (2,0,4|8,2), (2,1,4,2), (0,2,4|8,0),
 * (any,3,4,any).  sink: 1 KiB of device memory.
 */
int mla_probe_gather(int layout, int method, int waves, int stages, int groups, const void* rows,
                     int64_t row_stride, const void* scales, int64_t scale_stride, const void* v_rows,
                     int64_t v_row_stride, const int32_t* kv_indices, int64_t ntokens, void* sink,
                     void* stream);

/*
 * LDS read-pattern probe (no counterpart in the reference): `groups`
 * work-groups of 4 waves each repeat 8 LDS reads of one pattern `iters` times;
 * cycles[4 g + w] gets wave w of group g's shader-clock cycles per read
 * instruction.  Patterns (csrc/probe.hip): 0 contiguous ds_read_b128, 1 the
 * 128-head fp8 K fragment reads, 2 contiguous ds_read_b64_tr_b8, 3 the
 * 128-head V^T transpose reads, 4 ds_read_b128 with every lane on the same
 * banks.  For bank-counter passes beside the decode kernels.  cycles: 4 x
 * groups floats; sink: 1 KiB of device memory.
 */
int mla_probe_lds(int pattern, int iters, int groups, float* cycles, void* sink, void* stream);

/*
 * Diagnostics (no counterpart in the reference): runs one wave of a built-in
 * check that pins an MFMA operand/accumulator layout or a conversion the
 * kernels rely on.  `in`/`out` are small device buffers whose layout per
 * `which` is documented in csrc/selftest.hip.
 */
int mla_selftest(int which, const void* in, void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MLA_MI355X_H */
