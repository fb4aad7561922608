// Per-tensor FP8 quantizer, MXFP4 packer and the on-device split planner.
//
// FP8 (competitor_submissions/mi355x_reference/reference.py:65-80): a grid-wide
// |x| max is needed before any element can be quantized, so the work is two
// launches with no atomics and no state that must be pre-zeroed: pass 1 writes
// one partial max per block; pass 2 has every block fold those (<= 1024 words,
// L2-resident) before quantizing its share.  The planner rides along as the
// last block of pass 1 so the decode pipeline pays no extra launch for it.
//
// MXFP4 (reference.py:88-113 -> mxfp4-mm/submission_v18_custom_fused.py:26-108):
// one thread per 32-element block, 64 B in (4 x 16-byte loads), 16 B + 1 B out.
// KV-cache append: one lane per 8 elements into both caches at given rows.
#include "mla_internal.hpp"
#include "mla_plan.hpp"

namespace mla {

// ---------------------------------------------------------------------------
// pass 1: block-partial |x| max over bf16 (bit patterns: |x| ordering equals
// unsigned ordering of (bits & 0x7fff) for non-NaN inputs)
// ---------------------------------------------------------------------------
__device__ __forceinline__ void build_plan(const int32_t* __restrict__ kv_indptr, int batch, int qlen,
                                           int target_items, int min_chunk, int max_splits, int max_items,
                                           int32_t* __restrict__ plan);

__global__ __launch_bounds__(256) void amax_kernel(const uint16_t* __restrict__ x, int64_t n,
                                                   uint32_t* __restrict__ partials, int nblocks,
                                                   const int32_t* __restrict__ kv_indptr,
                                                   const int32_t* __restrict__ kv_indices,
                                                   int batch, int qlen, int target_items, int min_chunk,
                                                   int max_splits, int max_items, int32_t* __restrict__ plan) {
  // trailing block: split planner.  Marked unlikely so that the amax path is
  // the fall-through from the entry and the planner's code sits after it:
  // after a large write (the timing protocols' flush) a launch fetches its
  // code from memory, and amax blocks that jumped over the planner's code paid
  // up to 1.2 us more per call on the 16-head shapes (A/B, one lease)
  if (__builtin_expect((int)blockIdx.x >= nblocks, 0)) {
    build_plan(kv_indptr, batch, qlen, target_items, min_chunk, max_splits, max_items, plan);
    return;
  }
  if (kv_indices != nullptr) {
    // touch one word per 128-B line of this block's share of kv_indices so the
    // decode kernel's first slot fetches hit the caches (the decode reads
    // the indices a few microseconds later); the loaded values only feed a
    // store to a spare scratch word that nothing reads
    const int64_t T = kv_indptr[batch / qlen];
    const int64_t lo = T * blockIdx.x / nblocks, hi = T * (blockIdx.x + 1) / nblocks;
    int acc = 0;
    for (int64_t i = (lo & ~31LL) + 32LL * threadIdx.x; i < hi; i += 32LL * 256) acc ^= kv_indices[i];
    if (acc == 0x5EEDF00D) partials[kAmaxMaxBlocks + 1] = (uint32_t)acc;
  }
  uint32_t m = 0;
  const int64_t nvec = n >> 3;
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nvec; i += (int64_t)nblocks * 256) {
    uint4 v = ldg16_nt(xv + i);
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      m = max(m, w[k] & 0x7FFFu);
      m = max(m, (w[k] >> 16) & 0x7FFFu);
    }
  }
  for (int64_t i = (nvec << 3) + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)nblocks * 256)
    m = max(m, (uint32_t)(x[i] & 0x7FFFu));
  // wave reduce (DPP) then block reduce
  m = (uint32_t)wave_max((int)m);
  __shared__ uint32_t red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) partials[blockIdx.x] = max(max(red[0], red[1]), max(red[2], red[3]));
}

__global__ __launch_bounds__(256) void quant_fp8_kernel(const uint16_t* __restrict__ x, int64_t n,
                                                        const uint32_t* __restrict__ partials,
                                                        int nparts, uint8_t* __restrict__ out,
                                                        float* __restrict__ out_scale) {
  __shared__ float s_scale;
  __shared__ uint32_t red[4];
  const int64_t nvec = n >> 3;
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  // this thread's first 8 inputs are loaded while the partial maxima are folded
  const int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const uint4 first = i0 < nvec ? xv[i0] : make_uint4(0, 0, 0, 0);
  // nparts <= kAmaxMaxBlocks = 4 x 256: one 16-byte load per thread
  uint32_t m = 0;
  if (4 * (int)threadIdx.x < nparts) {
    const uint4 pv = reinterpret_cast<const uint4*>(partials)[threadIdx.x];
    const int k = nparts - 4 * (int)threadIdx.x;
    m = max(pv.x, k > 1 ? pv.y : 0u);
    m = max(m, max(k > 2 ? pv.z : 0u, k > 3 ? pv.w : 0u));
  }
  m = (uint32_t)wave_max((int)m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t a = max(max(red[0], red[1]), max(red[2], red[3]));
    s_scale = fp8_scale_from_amax(a);
    if (blockIdx.x == 0) out_scale[0] = s_scale;
  }
  __syncthreads();
  const Fp8Quant s = make_fp8_quant(s_scale);
  uint2* ov = reinterpret_cast<uint2*>(out);
  if (i0 < nvec) ov[i0] = quant8_fp8(first, s);
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i = i0 + stride;
  for (; i + 3 * stride < nvec; i += 4 * stride) {  // four loads in flight per thread
    uint4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = xv[i + k * stride];
#pragma unroll
    for (int k = 0; k < 4; ++k) ov[i + k * stride] = quant8_fp8(v[k], s);
  }
  for (; i < nvec; i += stride) ov[i] = quant8_fp8(xv[i], s);
  for (int64_t i = (nvec << 3) + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256)
    out[i] = (uint8_t)quant_one(x[i], s);
}

// ---------------------------------------------------------------------------
// MXFP4 pack: e8m0 scale rule of mxfp4-mm/submission_v18_custom_fused.py:50-58
// in integer form; e2m1 rounding (:60-98) by the hardware conversion
// ---------------------------------------------------------------------------
// e8m0 exponent of a 32-element block from the f32 bits of its |x| max: round
// the max up at bit 21, take the f32 exponent, subtract 2 (emax of e2m1),
// clamp to [-127, 127].
__device__ __forceinline__ int mx_exponent(uint32_t amax_f32_bits) {
  const uint32_t rnd = (amax_f32_bits + 0x200000u) & 0xFF800000u;
  const int ef = (int)(rnd >> 23);
  if (ef == 0) return -127;   // log2(0) = -inf, clamped
  if (ef == 255) return 127;  // +inf after round-up, clamped
  return min(max(ef - 127 - 2, -127), 127);
}

// 2^-e as an f32 (2^-127 is the one subnormal case)
__device__ __forceinline__ float mx_qscale(int e) {
  return (e == 127) ? __uint_as_float(0x00400000u) : __uint_as_float((uint32_t)(127 - e) << 23);
}

// Four words of bf16 pairs -> four bytes of e2m1 pairs (low nibble = low
// half) after scaling by qs = 2^-e (exact).  The hardware conversion rounds
// to nearest, ties to the even code, and saturates at 6 -- the rule of
// the reference's bit-trick encoder (mxfp4-mm/submission_v18_custom_fused.py:
// 66-98) -- which a device selftest pins on every value it can receive.
__device__ __forceinline__ uint32_t mx_encode_word4(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, float qs) {
  uint32_t r = 0;
  r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(r, bf16_bits_to_f32(w0 & 0xFFFFu) * qs,
                                               bf16_bits_to_f32(w0 >> 16) * qs, 1.0f, 0);
  r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(r, bf16_bits_to_f32(w1 & 0xFFFFu) * qs,
                                               bf16_bits_to_f32(w1 >> 16) * qs, 1.0f, 1);
  r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(r, bf16_bits_to_f32(w2 & 0xFFFFu) * qs,
                                               bf16_bits_to_f32(w2 >> 16) * qs, 1.0f, 2);
  r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(r, bf16_bits_to_f32(w3 & 0xFFFFu) * qs,
                                               bf16_bits_to_f32(w3 >> 16) * qs, 1.0f, 3);
  return r;
}

// One 32-element block: 16 words of bf16 pairs in, 16 bytes of e2m1 pairs and
// the e8m0 byte out.
__device__ __forceinline__ uint4 mx_block_encode(const uint32_t (&w)[16], uint32_t& e8) {
  uint32_t amax = 0;  // f32 bits of the block |x| max
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    amax = max(amax, (w[k] & 0x7FFFu) << 16);
    amax = max(amax, (w[k] >> 16 & 0x7FFFu) << 16);
  }
  const int e = mx_exponent(amax);
  const float qs = mx_qscale(e);
  e8 = (uint32_t)(e + 127);
  return make_uint4(mx_encode_word4(w[0], w[1], w[2], w[3], qs), mx_encode_word4(w[4], w[5], w[6], w[7], qs),
                    mx_encode_word4(w[8], w[9], w[10], w[11], qs), mx_encode_word4(w[12], w[13], w[14], w[15], qs));
}

__device__ __forceinline__ void load_block64(const uint8_t* p, uint32_t (&w)[16]) {
  const uint4* src = reinterpret_cast<const uint4*>(p);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint4 v = src[k];
    w[4 * k + 0] = v.x;
    w[4 * k + 1] = v.y;
    w[4 * k + 2] = v.z;
    w[4 * k + 3] = v.w;
  }
}

__global__ __launch_bounds__(256) void pack_mxfp4_kernel(const uint8_t* __restrict__ x, int64_t rows,
                                                         int blocks_per_row, int64_t x_stride,
                                                         uint8_t* __restrict__ packed,
                                                         int64_t packed_stride,
                                                         uint8_t* __restrict__ scales,
                                                         int64_t scale_stride) {
  const int64_t total = rows * blocks_per_row;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / blocks_per_row;
    const int j = (int)(i - r * blocks_per_row);
    uint32_t w[16];
    load_block64(x + r * x_stride + (int64_t)j * 64, w);
    uint32_t e8;
    *reinterpret_cast<uint4*>(packed + r * packed_stride + (int64_t)j * 16) = mx_block_encode(w, e8);
    scales[r * scale_stride + j] = (uint8_t)e8;
  }
}

// ---------------------------------------------------------------------------
// KV-cache append: token i (576 bf16) goes to cache row slots[i] of the fp8
// cache (quantized with the cache's existing per-tensor scale, the bytes the
// whole-buffer quantizer gives for that scale) and/or of the mxfp4 cache (its
// per-32 blocks need no global state, so an appended row equals the row of a
// whole-buffer pack).  slot < 0 skips the token.  amax_out (optional) is
// max-ed with the bf16 bits of max|x| over the written tokens.
//
// One lane per 8 elements (72 lanes per token): 16 B loads and 8 B / 4 B
// stores are contiguous across lanes, and a 32-element block is 4 aligned
// lanes that exchange their |x| max by two shuffles.  Lane groups of 4 never
// straddle a token (72 = 4 * 18) or a wave (64 = 4 * 16), and a whole token is
// skipped or written, so the 4 lanes of a block are active together.
// ---------------------------------------------------------------------------
constexpr int kLanesPerToken = kQKDim / 8;  // 72

__global__ __launch_bounds__(256) void append_kv_kernel(
    const uint8_t* __restrict__ x, int n, int64_t x_stride, const int32_t* __restrict__ slots,
    uint8_t* __restrict__ fp8_cache, int64_t fp8_stride, const float* __restrict__ fp8_scale,
    uint8_t* __restrict__ fp4_cache, int64_t fp4_stride, uint8_t* __restrict__ fp4_scales,
    int64_t fp4_scale_stride, uint32_t* __restrict__ amax_out) {
  const uint32_t total = (uint32_t)n * kLanesPerToken;
  const Fp8Quant s = make_fp8_quant(fp8_cache != nullptr ? fp8_scale[0] : 1.0f);
  uint32_t amax = 0;  // bf16 |x| bits over this lane's written chunks
  for (uint32_t u = blockIdx.x * 256u + threadIdx.x; u < total; u += gridDim.x * 256u) {
    const uint32_t t = u / kLanesPerToken;
    const uint32_t p = u - t * kLanesPerToken;
    const int64_t slot = slots != nullptr ? (int64_t)slots[t] : (int64_t)t;
    if (slot < 0) continue;
    const uint4 v = ldg16_nt(x + (int64_t)t * x_stride + p * 16);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t m = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) m = max(m, max(w[k] & 0x7FFFu, (w[k] >> 16) & 0x7FFFu));
    amax = max(amax, m);
    if (fp8_cache != nullptr)
      *reinterpret_cast<uint2*>(fp8_cache + slot * fp8_stride + p * 8) = quant8_fp8(v, s);
    if (fp4_cache != nullptr) {
      m = max(m, (uint32_t)__shfl_xor((int)m, 1, 64));
      m = max(m, (uint32_t)__shfl_xor((int)m, 2, 64));
      const int e = mx_exponent(m << 16);
      const float qs = mx_qscale(e);
      *reinterpret_cast<uint32_t*>(fp4_cache + slot * fp4_stride + p * 4) = mx_encode_word4(w[0], w[1], w[2], w[3], qs);
      if ((p & 3u) == 0) fp4_scales[slot * fp4_scale_stride + (p >> 2)] = (uint8_t)(e + 127);
    }
  }
  if (amax_out != nullptr) {
    // one atomic per block at most, and only when it raises the stored max:
    // atomics on one address serialize, so per-wave atomics would dominate
    __shared__ uint32_t red[4];
    amax = (uint32_t)wave_max((int)amax);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t m = max(max(red[0], red[1]), max(red[2], red[3]));
      if (m > __atomic_load_n(amax_out, __ATOMIC_RELAXED)) atomicMax(amax_out, m);
    }
  }
}

// ---------------------------------------------------------------------------
// split planner (one block of 256 threads)
// Work is planned per query row: `batch` rows, q_seq_len = qlen rows per
// sequence, row r = (sequence r / qlen, query i = r % qlen) attends to the
// causal prefix of length L - (qlen - 1 - i) of its sequence (uniform-qo_len
// causal decode, competitor_submissions/mi355x_reference/reference.py:188-193);
// with qlen = 1 a row is a sequence.  Below, "sequence b" means row b.
// Sequence b is cut into n_b = max(1, ceil(L_b / chunk)) near-equal pieces.
// For batch <= 256, chunk = the smallest multiple of 64 with sum_b n_b <=
// target_items (binary search from c0 = max(min_chunk, 64 ceil(T / (64 target)),
// and, when max_splits > 0, 64 ceil(Lmax / (64 max_splits)) for the longest
// sequence Lmax),
// T = all tokens; the longest sequence if no chunk fits), and the sequences
// are laid out longest piece first so late-starting work-groups get the short
// items.  For larger batches chunk = c0 and the order is the sequence order.
// Either way there are at most target_items + batch items (the workspace
// bound).  Pieces of a sequence are consecutive items; a sequence with
// n_b == 1 writes its output directly (slot -1); otherwise each piece owns
// partial slot = its item index.
// ---------------------------------------------------------------------------
constexpr int kPlanSortMax = 256;

// the nb near-equal pieces of [s0, s0 + L): piece i = [s0 + floor(iL/nb),
// s0 + floor((i+1)L/nb)), computed with one division and a running remainder
__device__ __forceinline__ void emit_pieces(int4* __restrict__ items, int b, int s0, int L, int nb, int first) {
  const int q = L / nb, r = L - q * nb;
  int t = s0, rem = 0;
  for (int i = 0; i < nb; ++i) {
    int t1 = t + q;
    rem += r;
    if (rem >= nb) {
      rem -= nb;
      ++t1;
    }
    items[first + i] = make_int4(b, t, t1, nb > 1 ? first + i : -1);
    t = t1;
  }
}

// Up to 64 rows: one wave plans alone (mla_plan.hpp); lane b writes row b's
// pieces (emit_pieces: the bounds plan_wave_item gives, by a running
// remainder), a few stores per lane instead of a search per item
__device__ __forceinline__ void build_plan_wave(const int32_t* __restrict__ kv_indptr, int batch, int qlen,
                                                int target_items, int min_chunk, int max_splits, int max_items,
                                                int32_t* __restrict__ plan) {
  const WavePlan P = plan_wave(kv_indptr, batch, qlen, target_items, min_chunk, max_splits);
  plan_wave_write_rows(P, batch, max_items, plan);
  int4* items = reinterpret_cast<int4*>(plan + kPlanHeader);
  const int b = (int)(threadIdx.x & 63);
  if (b < batch) emit_pieces(items, b, P.s0_b, P.len_b, P.nb, P.first);
}

__device__ __forceinline__ void build_plan(const int32_t* __restrict__ kv_indptr, int batch, int qlen,
                                           int target_items, int min_chunk, int max_splits, int max_items,
                                           int32_t* __restrict__ plan) {
  if (batch <= 64) {
    if (threadIdx.x < 64)
      build_plan_wave(kv_indptr, batch, qlen, target_items, min_chunk, max_splits, max_items, plan);
    return;
  }
  __shared__ int s_red[kPlanRedInts];
  // ordering key per sequence: piece length, then the lower index first
  __shared__ __attribute__((aligned(16))) uint64_t s_key[kPlanSortMax];
  __shared__ int s_cnt[kPlanSortMax];    // item counts in layout order, then their exclusive scan
  const int tid = threadIdx.x;
  int4* items = reinterpret_cast<int4*>(plan + kPlanHeader);
  int2* binfo = reinterpret_cast<int2*>(plan + kPlanHeader + 4 * max_items);
  if (batch <= kPlanSortMax) {
    const BlockPlan P = plan_block(kv_indptr, batch, qlen, target_items, min_chunk, max_splits, s_key, s_cnt, s_red);
    if (tid < batch) {
      binfo[tid] = make_int2(P.first, P.nb);
      emit_pieces(items, tid, P.s0, P.L, P.nb, P.first);
    }
    if (tid == 0) {
      plan[0] = P.n_items;
      plan[1] = P.chunk;
      plan[2] = (int)(64u * P.hi64 + P.lo64);
      plan[3] = batch;
      plan[4] = max_items;
    }
    return;
  }
  int t_hi = 0, t_lo = 0, t_max = 0;
  for (int b = tid; b < batch; b += 256) {
    const int L = row_len(kv_indptr, b, qlen);
    t_hi += L >> 6;
    t_lo += L & 63;
    t_max = max(t_max, L);
  }
  const unsigned hi64 = (unsigned)block_sum(t_hi, s_red), lo64 = (unsigned)block_sum(t_lo, s_red);
  const int lmax = block_max(t_max, s_red);
  int chunk = 64 * max(min_chunk / 64, (int)tiles_per_item(hi64, lo64, target_items));
  if (max_splits > 0) chunk = max(chunk, 64 * (((lmax + 63) / 64 + max_splits - 1) / max_splits));
  // more sequences than one block sorts: layout order, one 256-row pass at a time
  auto nb_of = [&](int L) { return L > 0 ? (L + chunk - 1) / chunk : 1; };
  int carry = 0;
  for (int base = 0; base < batch; base += 256) {
    const int b = base + tid;
    int L = 0, nb = 0;
    if (b < batch) {
      L = row_len(kv_indptr, b, qlen);
      nb = nb_of(L);
    }
    int tot = 0;
    const int ex = block_exscan(nb, s_red, &tot);
    if (b < batch) {
      binfo[b] = make_int2(carry + ex, nb);
      emit_pieces(items, b, row_start(kv_indptr, b, qlen), L, nb, carry + ex);
    }
    carry += tot;
  }
  if (tid == 0) {
    plan[0] = carry;
    plan[1] = chunk;
    plan[2] = (int)(64u * hi64 + lo64);
    plan[3] = batch;
    plan[4] = max_items;
  }
}

__global__ __launch_bounds__(256) void plan_kernel(const int32_t* __restrict__ kv_indptr, int batch, int qlen,
                                                   int target_items, int min_chunk, int max_splits, int max_items,
                                                   int32_t* __restrict__ plan) {
  build_plan(kv_indptr, batch, qlen, target_items, min_chunk, max_splits, max_items, plan);
}

// ---------------------------------------------------------------------------
// Paged caches: AITER's page table (kv_indptr over pages, page ids,
// kv_last_page_lens, page_size; mixed-mla/asm_dumps/aiter_mla.py:149-175, built
// as at mixed-mla/submission.py:449-456 and :538-544) expanded into the
// token-level kv_indptr / kv_indices every decode kernel reads.  Sequence b
// holds n_b = indptr[b+1] - indptr[b] pages and L_b = (n_b - 1) P + last_b
// tokens (0 when n_b = 0; last_b clamped to [1, P]); its token j is row
// page_ids[indptr[b] + j / P] * P + j % P of the flattened [pages * P, row]
// cache.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int paged_len(const int32_t* __restrict__ page_indptr,
                                         const int32_t* __restrict__ last_page_lens, int b, int P) {
  const int np = page_indptr[b + 1] - page_indptr[b];
  return np > 0 ? (np - 1) * P + min(max(last_page_lens[b], 1), P) : 0;
}

// one block: token counts of every sequence, exclusive scan -> kv_indptr_out
__global__ __launch_bounds__(256) void paged_indptr_kernel(const int32_t* __restrict__ page_indptr,
                                                           const int32_t* __restrict__ last_page_lens,
                                                           int batch, int P, int32_t* __restrict__ kv_indptr_out) {
  __shared__ int red[4];
  int carry = 0;
  for (int base = 0; base < batch; base += 256) {
    const int b = base + (int)threadIdx.x;
    const int L = b < batch ? paged_len(page_indptr, last_page_lens, b, P) : 0;
    int tot = 0;
    const int ex = block_exscan(L, red, &tot);
    if (b < batch) kv_indptr_out[b] = carry + ex;
    carry += tot;
  }
  if (threadIdx.x == 0) kv_indptr_out[batch] = carry;
}

// one thread per page: its sequence by binary search over the page indptr,
// then its up-to-P token rows
__global__ __launch_bounds__(256) void paged_indices_kernel(const int32_t* __restrict__ page_indptr,
                                                            const int32_t* __restrict__ page_ids,
                                                            const int32_t* __restrict__ last_page_lens,
                                                            int batch, int P, int64_t max_pages,
                                                            const int32_t* __restrict__ kv_indptr,
                                                            int32_t* __restrict__ kv_indices_out) {
  const int64_t pg = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (pg >= max_pages || pg >= page_indptr[batch]) return;
  int lo = 0, hi = batch - 1;  // last b with page_indptr[b] <= pg
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (page_indptr[mid] <= pg) lo = mid;
    else hi = mid - 1;
  }
  const int b = lo;
  const int j = (int)(pg - page_indptr[b]);
  const int np = page_indptr[b + 1] - page_indptr[b];
  const int cnt = j == np - 1 ? min(max(last_page_lens[b], 1), P) : P;
  const int32_t row0 = page_ids[pg] * P;
  int32_t* dst = kv_indices_out + kv_indptr[b] + (int64_t)j * P;
  for (int i = 0; i < cnt; ++i) dst[i] = row0 + i;
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
static int amax_blocks_for(int64_t n) {
  int64_t per_block = 256LL * 8 * 4;  // >= 4 vectors per thread
  int64_t b = (n + per_block - 1) / per_block;
  if (b < 1) b = 1;
  if (b > kAmaxMaxBlocks) b = kAmaxMaxBlocks;
  return (int)b;
}

hipError_t launch_amax(const uint16_t* x, int64_t n, uint32_t* partials, int* nblocks,
                       const int32_t* kv_indptr, const int32_t* kv_indices, int batch, int qlen,
                       PlanTarget target, int max_items, int32_t* plan, hipStream_t stream) {
  const int nb = amax_blocks_for(n);
  *nblocks = nb;
  const int grid = nb + (plan != nullptr ? 1 : 0);
  hipLaunchKernelGGL(amax_kernel, dim3(grid), dim3(256), 0, stream, x, n, partials, nb, kv_indptr,
                     plan != nullptr ? kv_indices : nullptr, batch, qlen, target.items, target.min_chunk,
                     target.max_splits, max_items, plan);
  return hipGetLastError();
}

hipError_t launch_quant_fp8(const uint16_t* x, int64_t n, const uint32_t* partials, int nblocks,
                            uint8_t* out, float* out_scale, hipStream_t stream) {
  int64_t g = (n / 8 + 255) / 256;
  if (g < 1) g = 1;
  if (g > 2048) g = 2048;
  hipLaunchKernelGGL(quant_fp8_kernel, dim3((int)g), dim3(256), 0, stream, x, n, partials, nblocks,
                     out, out_scale);
  return hipGetLastError();
}

hipError_t launch_pack_mxfp4(const uint16_t* x, int64_t rows, int cols, int64_t x_stride,
                             uint8_t* packed, int64_t packed_stride, uint8_t* scales,
                             int64_t scale_stride, hipStream_t stream) {
  const int bpr = cols / 32;
  int64_t total = rows * bpr;
  int64_t g = (total + 255) / 256;
  if (g < 1) g = 1;
  if (g > 8192) g = 8192;
  hipLaunchKernelGGL(pack_mxfp4_kernel, dim3((int)g), dim3(256), 0, stream,
                     reinterpret_cast<const uint8_t*>(x), rows, bpr, x_stride, packed,
                     packed_stride, scales, scale_stride);
  return hipGetLastError();
}

hipError_t launch_append_kv(const uint16_t* x, int64_t n, int64_t x_stride, const int32_t* slots,
                            uint8_t* fp8_cache, int64_t fp8_stride, const float* fp8_scale,
                            uint8_t* fp4_cache, int64_t fp4_stride, uint8_t* fp4_scales,
                            int64_t fp4_scale_stride, uint32_t* amax_out, hipStream_t stream) {
  int64_t g = (n * kLanesPerToken + 255) / 256;
  if (g < 1) g = 1;
  if (g > 2048) g = 2048;  // 8 blocks per CU; larger appends loop
  hipLaunchKernelGGL(append_kv_kernel, dim3((int)g), dim3(256), 0, stream,
                     reinterpret_cast<const uint8_t*>(x), (int)n, x_stride, slots, fp8_cache, fp8_stride,
                     fp8_scale, fp4_cache, fp4_stride, fp4_scales, fp4_scale_stride, amax_out);
  return hipGetLastError();
}

hipError_t launch_expand_pages(const int32_t* page_indptr, const int32_t* page_ids, const int32_t* last_page_lens,
                               int batch, int page_size, int64_t max_pages, int32_t* kv_indptr_out,
                               int32_t* kv_indices_out, hipStream_t stream) {
  hipLaunchKernelGGL(paged_indptr_kernel, dim3(1), dim3(256), 0, stream, page_indptr, last_page_lens, batch,
                     page_size, kv_indptr_out);
  if (max_pages > 0) {
    const int64_t g = (max_pages + 255) / 256;
    hipLaunchKernelGGL(paged_indices_kernel, dim3((unsigned)g), dim3(256), 0, stream, page_indptr, page_ids,
                       last_page_lens, batch, page_size, max_pages, kv_indptr_out, kv_indices_out);
  }
  return hipGetLastError();
}

hipError_t launch_plan(const int32_t* kv_indptr, int batch, int qlen, PlanTarget target, int max_items,
                       int32_t* plan, hipStream_t stream) {
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(256), 0, stream, kv_indptr, batch, qlen, target.items,
                     target.min_chunk, target.max_splits, max_items, plan);
  return hipGetLastError();
}

}  // namespace mla
