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
#include "mla_internal.hpp"

namespace mla {

// ---------------------------------------------------------------------------
// pass 1: block-partial |x| max over bf16 (bit patterns: |x| ordering equals
// unsigned ordering of (bits & 0x7fff) for non-NaN inputs)
// ---------------------------------------------------------------------------
__device__ void build_plan(const int32_t* __restrict__ kv_indptr, int batch, int target_items,
                           int max_items, int32_t* __restrict__ plan);

__global__ __launch_bounds__(256) void amax_kernel(const uint16_t* __restrict__ x, int64_t n,
                                                   uint32_t* __restrict__ partials, int nblocks,
                                                   const int32_t* __restrict__ kv_indptr,
                                                   const int32_t* __restrict__ kv_indices,
                                                   int batch, int target_items, int max_items,
                                                   int32_t* __restrict__ plan) {
  if ((int)blockIdx.x >= nblocks) {  // trailing block: split planner
    build_plan(kv_indptr, batch, target_items, max_items, plan);
    return;
  }
  if (kv_indices != nullptr) {
    // touch one word per 128-B line of this block's share of kv_indices so the
    // decode kernel's first slot fetches hit the caches (the decode reads
    // the indices a few microseconds later); the loaded values only feed a
    // store to a spare scratch word that nothing reads
    const int64_t T = kv_indptr[batch];
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
  // wave reduce then block reduce
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off, 64));
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
  uint32_t m = 0;
  for (int i = threadIdx.x; i < nparts; i += 256) m = max(m, partials[i]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t a = max(max(red[0], red[1]), max(red[2], red[3]));
    s_scale = fp8_scale_from_amax(a);
    if (blockIdx.x == 0) out_scale[0] = s_scale;
  }
  __syncthreads();
  const float s = s_scale;
  const int64_t nvec = n >> 3;
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  uint2* ov = reinterpret_cast<uint2*>(out);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nvec; i += (int64_t)gridDim.x * 256) {
    uint4 v = xv[i];
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[2] = {0, 0};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t lo = quant_one(w[k] & 0xFFFFu, s);
      uint32_t hi = quant_one(w[k] >> 16, s);
      o[k >> 1] |= (lo | (hi << 8)) << (16 * (k & 1));
    }
    ov[i] = make_uint2(o[0], o[1]);
  }
  for (int64_t i = (nvec << 3) + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256)
    out[i] = (uint8_t)quant_one(x[i], s);
}

// ---------------------------------------------------------------------------
// MXFP4 pack: e8m0 scale rule and e2m1 rounding of
// mxfp4-mm/submission_v18_custom_fused.py:50-106 in integer form
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t e2m1_encode(float q) {
  uint32_t u = __float_as_uint(q);
  uint32_t s = u & 0x80000000u;
  u ^= s;
  float a = __uint_as_float(u);
  uint32_t code;
  if (a >= 6.0f) {
    code = 7u;
  } else if (a < 1.0f) {
    // add 2^22 so the f32 add rounds |q| to a multiple of 0.5 (ties to even)
    code = __float_as_uint(a + 4194304.0f) - (149u << 23);
  } else {
    uint32_t odd = (u >> 22) & 1u;
    code = ((u + 0xC1200000u - 1u + odd) >> 22) & 0xFFu;  // (1-127)<<23 + 2^21 - 1 (mod 2^32)
  }
  return code | (s >> 28);
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
    const uint4* src = reinterpret_cast<const uint4*>(x + r * x_stride + (int64_t)j * 64);
    uint32_t w[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint4 v = src[k];
      w[4 * k + 0] = v.x;
      w[4 * k + 1] = v.y;
      w[4 * k + 2] = v.z;
      w[4 * k + 3] = v.w;
    }
    uint32_t amax = 0;  // f32 bits of the block |x| max
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      amax = max(amax, (w[k] & 0x7FFFu) << 16);
      amax = max(amax, (w[k] >> 16 & 0x7FFFu) << 16);
    }
    const uint32_t rnd = (amax + 0x200000u) & 0xFF800000u;
    const int ef = (int)(rnd >> 23);
    int e;
    if (ef == 0) e = -127;           // log2(0) = -inf, clamped
    else if (ef == 255) e = 127;     // +inf after round-up, clamped
    else e = min(max(ef - 127 - 2, -127), 127);
    // 2^-e as an f32 (2^-127 is the one subnormal case)
    const float qs = (e == 127) ? __uint_as_float(0x00400000u) : __uint_as_float((uint32_t)(127 - e) << 23);
    uint32_t outw[4] = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      uint32_t c0 = e2m1_encode(bf16_bits_to_f32(w[k] & 0xFFFFu) * qs);
      uint32_t c1 = e2m1_encode(bf16_bits_to_f32(w[k] >> 16) * qs);
      outw[k >> 2] |= (c0 | (c1 << 4)) << (8 * (k & 3));
    }
    *reinterpret_cast<uint4*>(packed + r * packed_stride + (int64_t)j * 16) =
        make_uint4(outw[0], outw[1], outw[2], outw[3]);
    scales[r * scale_stride + j] = (uint8_t)(e + 127);
  }
}

// ---------------------------------------------------------------------------
// split planner (one block of 256 threads)
// chunk = the smallest multiple of 64 tokens for which the item count
// sum_b max(1, ceil(L_b / chunk)) fits target_items (or the longest sequence,
// if even one item per sequence exceeds it).  Sequence b is cut into
// n_b = ceil(L_b / chunk) near-equal pieces (1 piece if empty).  Pieces of a
// sequence are consecutive items; sequences are laid out longest piece first
// (for batch <= 1024) so late-starting work-groups get the short items.  A
// sequence with n_b == 1 writes its output directly (slot -1); otherwise each
// piece owns partial slot = its item index.
// ---------------------------------------------------------------------------
constexpr int kPlanSortMax = 1024;

__device__ long long block_sum_ll(long long v, long long* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

__device__ int block_max_i(int v, int* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = max(v, __shfl_xor(v, off, 64));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return max(max(red[0], red[1]), max(red[2], red[3]));
}

__device__ void build_plan(const int32_t* __restrict__ kv_indptr, int batch, int target_items,
                           int max_items, int32_t* __restrict__ plan) {
  __shared__ long long s_red[4];
  __shared__ int s_redi[4];
  __shared__ int s_n[kPlanSortMax];  // item counts in layout order, then their exclusive scan
  __shared__ int s_piece[kPlanSortMax];
  __shared__ int s_scan[256];
  __shared__ int s_carry;
  __shared__ int s_len[kPlanSortMax];
  __shared__ int s_rank[kPlanSortMax];
  const int tid = threadIdx.x;
  const bool staged = batch <= kPlanSortMax;  // lengths kept in LDS
  long long tsum = 0;
  int lmax = 0;
  for (int b = tid; b < batch; b += 256) {
    const int L = max(kv_indptr[b + 1] - kv_indptr[b], 0);
    if (staged) s_len[b] = L;
    tsum += L;
    lmax = max(lmax, L);
  }
  auto len_of = [&](int b) { return staged ? s_len[b] : max(kv_indptr[b + 1] - kv_indptr[b], 0); };
  const long long total = block_sum_ll(tsum, s_red);
  lmax = block_max_i(lmax, s_redi);
  // binary search on chunk / 64 in [1, ceil(lmax / 64)]
  int lo = 1, hi = max(1, (lmax + kTile - 1) / kTile);
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    const long long c = (long long)mid * kTile;
    long long cnt = 0;
    for (int b = tid; b < batch; b += 256) {
      const long long L = len_of(b);
      cnt += L > 0 ? (L + c - 1) / c : 1;
    }
    cnt = block_sum_ll(cnt, s_red);
    if (cnt <= target_items) hi = mid;
    else lo = mid + 1;
  }
  const long long chunk = (long long)lo * kTile;
  int4* items = reinterpret_cast<int4*>(plan + kPlanHeader);
  int2* binfo = reinterpret_cast<int2*>(plan + kPlanHeader + 4 * max_items);
  if (tid == 0) s_carry = 0;
  __syncthreads();
  if (batch <= kPlanSortMax) {
    // piece length per sequence in LDS, then rank longest first (ties by index)
    for (int b = tid; b < batch; b += 256) {
      const int L = len_of(b);
      const int nb = L > 0 ? (int)((L + chunk - 1) / chunk) : 1;
      s_piece[b] = (L + nb - 1) / nb;
    }
    __syncthreads();
    for (int b = tid; b < batch; b += 256) {
      const int L = len_of(b);
      const int nb = L > 0 ? (int)((L + chunk - 1) / chunk) : 1;
      const int piece = s_piece[b];
      int rank = 0;
      for (int b2 = 0; b2 < batch; ++b2) {
        const int p2 = s_piece[b2];
        rank += (p2 > piece) || (p2 == piece && b2 < b);
      }
      s_n[rank] = nb;
      s_rank[b] = rank;
    }
    __syncthreads();
    // exclusive scan of s_n in place, 256 at a time
    for (int base = 0; base < batch; base += 256) {
      const int i = base + tid;
      const int v = i < batch ? s_n[i] : 0;
      s_scan[tid] = v;
      __syncthreads();
      for (int off = 1; off < 256; off <<= 1) {
        const int a = tid >= off ? s_scan[tid - off] : 0;
        __syncthreads();
        s_scan[tid] += a;
        __syncthreads();
      }
      if (i < batch) s_n[i] = s_carry + s_scan[tid] - v;
      __syncthreads();
      if (tid == 255) s_carry += s_scan[255];
      __syncthreads();
    }
    for (int b = tid; b < batch; b += 256) {
      const int L = len_of(b);
      const int first = s_n[s_rank[b]], nb = L > 0 ? (int)((L + chunk - 1) / chunk) : 1;
      const int s0 = kv_indptr[b];
      binfo[b] = make_int2(first, nb);
      for (int i = 0; i < nb; ++i) {
        const int t0 = s0 + (int)(((long long)i * L) / nb);
        const int t1 = s0 + (int)(((long long)(i + 1) * L) / nb);
        items[first + i] = make_int4(b, t0, t1, nb > 1 ? first + i : -1);
      }
    }
  } else {
    for (int base = 0; base < batch; base += 256) {
      const int b = base + tid;
      int L = 0, nb = 0;
      if (b < batch) {
        L = max(kv_indptr[b + 1] - kv_indptr[b], 0);
        nb = L > 0 ? (int)((L + chunk - 1) / chunk) : 1;
      }
      s_scan[tid] = nb;
      __syncthreads();
      for (int off = 1; off < 256; off <<= 1) {
        const int a = tid >= off ? s_scan[tid - off] : 0;
        __syncthreads();
        s_scan[tid] += a;
        __syncthreads();
      }
      const int first = s_carry + s_scan[tid] - nb;
      if (b < batch) {
        const int s0 = kv_indptr[b];
        binfo[b] = make_int2(first, nb);
        for (int i = 0; i < nb; ++i) {
          const int t0 = s0 + (int)(((long long)i * L) / nb);
          const int t1 = s0 + (int)(((long long)(i + 1) * L) / nb);
          items[first + i] = make_int4(b, t0, t1, nb > 1 ? first + i : -1);
        }
      }
      __syncthreads();
      if (tid == 255) s_carry += s_scan[255];
      __syncthreads();
    }
  }
  __syncthreads();
  if (tid == 0) {
    plan[0] = s_carry;
    plan[1] = (int)chunk;
    plan[2] = (int)total;
    plan[3] = batch;
    plan[4] = max_items;
  }
}

__global__ __launch_bounds__(256) void plan_kernel(const int32_t* __restrict__ kv_indptr, int batch,
                                                   int target_items, int max_items,
                                                   int32_t* __restrict__ plan) {
  build_plan(kv_indptr, batch, target_items, max_items, plan);
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
                       const int32_t* kv_indptr, const int32_t* kv_indices, int batch, int target_items,
                       int max_items, int32_t* plan, hipStream_t stream) {
  const int nb = amax_blocks_for(n);
  *nblocks = nb;
  const int grid = nb + (plan != nullptr ? 1 : 0);
  hipLaunchKernelGGL(amax_kernel, dim3(grid), dim3(256), 0, stream, x, n, partials, nb, kv_indptr,
                     plan != nullptr ? kv_indices : nullptr, batch, target_items, max_items, plan);
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

hipError_t launch_plan(const int32_t* kv_indptr, int batch, int target_items, int max_items,
                       int32_t* plan, hipStream_t stream) {
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(256), 0, stream, kv_indptr, batch, target_items,
                     max_items, plan);
  return hipGetLastError();
}

}  // namespace mla
