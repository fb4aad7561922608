// The split planner's one-wave form (up to 64 query rows) and block form (up
// to 256), shared by the planner kernel (which writes every item) and the
// 16-head decode kernel when it plans its own work (it needs one item; its
// work-group 0 writes the rows' piece counts and the header the combine
// reads).  The plan itself is described in quant.hip.
#pragma once

#include "mla_common.hpp"

namespace mla {

// ceil(total / (64 target)) for total = 64 s1 + s0 (the sums of L >> 6 and of
// L & 63 over the rows), in 32-bit arithmetic: ceil(total / 64) = s1 +
// ceil(s0 / 64), and nested ceilings of integer quotients compose.  Valid while
// the sum of L over all rows stays below 2^37 (s1 < 2^31) and there are fewer
// than 2^25 rows (s0 < 2^31).
__device__ __forceinline__ unsigned tiles_per_item(unsigned s1, unsigned s0, int target) {
  const unsigned t64 = s1 + (s0 + 63u) / 64u;
  return (t64 + (unsigned)target - 1u) / (unsigned)target;
}

// first key token and key count of query row r
__device__ __forceinline__ int row_start(const int32_t* __restrict__ kv_indptr, int r, int qlen) {
  return kv_indptr[r / qlen];
}
__device__ __forceinline__ int row_len(const int32_t* __restrict__ kv_indptr, int r, int qlen) {
  const int b = r / qlen, i = r - b * qlen;
  return max(kv_indptr[b + 1] - kv_indptr[b] - (qlen - 1 - i), 0);
}

// One wave's plan of up to 64 rows, in registers.  Lane b (b < batch) holds
// row b's first item and piece count; in rank order (lane = rank, rows ranked
// by piece length, longest first) x is the inclusive item count, and seq_r,
// s0_r, len_r, nb_r the rank's row, first key, key count and piece count.
struct WavePlan {
  int n_items, chunk;
  int first, nb;
  int s0_b, len_b;  // lane b's own row: first key, key count
  int x, nb_r, seq_r, s0_r, len_r;
  unsigned hi64, lo64;
};

// every reduction, the binary search and the ordering in registers
// (shuffles; ds_permute to scatter each row's item count to its rank
// position and ds_bpermute to gather its first item back): one round trip to
// kv_indptr and no barriers.  The whole wave must be active.
__device__ __forceinline__ WavePlan plan_wave(const int32_t* __restrict__ kv_indptr, int batch, int qlen,
                                              int target_items, int min_chunk, int max_splits) {
  const int lane = threadIdx.x & 63;
  const bool act = lane < batch;
  const int s0 = act ? row_start(kv_indptr, lane, qlen) : 0;
  const int L = act ? row_len(kv_indptr, lane, qlen) : 0;
  WavePlan P;
  P.hi64 = (unsigned)wave_sum(L >> 6);
  P.lo64 = (unsigned)wave_sum(L & 63);
  const int lmax = wave_max(L);
  const int L64 = (L + 63) >> 6;  // ceil(L / (64 m)) = ceil(L64 / m)
  const unsigned s64 = (unsigned)wave_sum(L64);
  int lo = max(min_chunk / 64, (int)tiles_per_item(P.hi64, P.lo64, target_items));
  if (max_splits > 0) lo = max(lo, ((lmax + 63) / 64 + max_splits - 1) / max_splits);
  // m = ceil(s64 / (target - batch)) already fits: the count at m is at most
  // sum(L64 / m + 1) <= s64 / m + batch <= target
  int hi = (lmax + 63) / 64;
  if (target_items > batch) hi = min(hi, (int)((s64 + (unsigned)(target_items - batch) - 1u) / (unsigned)(target_items - batch)));
  hi = max(lo, hi);
  const int l64min = -wave_max(act ? -L64 : -0x7FFFFFFF);
  if (l64min == (lmax + 63) / 64) {
    // every row as long (a common batch): the count at m is batch ceil(L64 / m),
    // so the smallest m in [lo, hi] within the target is ceil(L64 / k), k =
    // target / batch pieces a row, clamped (hi when no m fits)
    const int k = target_items / max(batch, 1);
    lo = hi = k > 0 ? min(hi, max(lo, (l64min + k - 1) / k)) : hi;
  }
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    const int cnt = wave_sum(act ? (L64 > 0 ? (L64 + mid - 1) / mid : 1) : 0);
    if (cnt <= target_items) hi = mid;
    else lo = mid + 1;
  }
  P.chunk = lo * 64;
  P.nb = act ? (L > 0 ? (L64 + lo - 1) / lo : 1) : 0;
  const int piece = act ? (L > 0 ? (L + P.nb - 1) / P.nb : 0) : -1;
  // rank by piece length, longest first (ties by index); inactive lanes (piece
  // -1) never count and rank last.  Equal pieces on every row (a common
  // batch) leave the rows in index order.  Otherwise key = (piece + 1) 64 +
  // 63 - lane orders both at once (unique, the inactive lanes' keys below the
  // rest) while it fits 31 bits, and the rank is the number of larger keys:
  // one readlane, compare and add per lane, all 64 read with constant lane
  // indices, so the loop unrolls into independent readlanes.
  int rank = lane;
  const int pmax = wave_max(piece), pmin = -wave_max(act ? -piece : -0x7FFFFFFF);
  if (pmin != pmax) {
    rank = 0;
    if (pmax < (1 << 24)) {
      const int key = (piece + 1) * 64 + 63 - lane;
#pragma unroll
      for (int b2 = 0; b2 < 64; ++b2) rank += __builtin_amdgcn_readlane(key, b2) > key;
    } else {
#pragma unroll
      for (int b2 = 0; b2 < 64; ++b2) {
        const int p2 = __builtin_amdgcn_readlane(piece, b2);
        rank += (p2 > piece) || (p2 == piece && b2 < lane);
      }
    }
    if (!act) rank = lane;
  }
  // item counts in rank order -> inclusive scan -> each row's first item
  P.nb_r = __builtin_amdgcn_ds_permute(rank << 2, P.nb);
  P.x = wave_incl_sum(P.nb_r);
  P.n_items = __builtin_amdgcn_readlane(P.x, 63);
  P.first = __builtin_amdgcn_ds_bpermute(rank << 2, P.x - P.nb_r);
  P.seq_r = __builtin_amdgcn_ds_permute(rank << 2, lane);
  P.s0_r = __builtin_amdgcn_ds_permute(rank << 2, s0);
  P.len_r = __builtin_amdgcn_ds_permute(rank << 2, L);
  P.s0_b = s0;
  P.len_b = L;
  return P;
}

// Item i of the plan as (row, first key, end key, partial slot or -1), for a
// per-lane i (lanes may ask different items; the whole wave must be active;
// i >= n_items gives row -1).  In rank order x is non-decreasing (ranks past
// the batch add 0), so item i belongs to rank c = #{r : x_r <= i}, found by a
// 6-step binary search over x; piece j of [s0, s0 + L) in n pieces starts at
// s0 + j q + floor(j r / n) (q = L / n, r = L % n), the bounds a running
// remainder over the pieces gives; j r < n^2 stays in 32 bits.
__device__ __forceinline__ int4 plan_wave_item(const WavePlan& P, int i) {
  int c = 0;
#pragma unroll
  for (int step = 32; step >= 1; step >>= 1)
    if (__builtin_amdgcn_ds_bpermute((c + step - 1) << 2, P.x) <= i) c += step;
  const int bi = __builtin_amdgcn_ds_bpermute(c << 2, P.seq_r);
  const int sb = __builtin_amdgcn_ds_bpermute(c << 2, P.s0_r);
  const int lb = __builtin_amdgcn_ds_bpermute(c << 2, P.len_r);
  const int nbb = __builtin_amdgcn_ds_bpermute(c << 2, P.nb_r);
  const int fb = __builtin_amdgcn_ds_bpermute(c << 2, P.x - P.nb_r);
  if (i >= P.n_items || nbb <= 0) return make_int4(-1, 0, 0, -1);
  const unsigned j = (unsigned)(i - fb), n = (unsigned)nbb;
  const unsigned q = (unsigned)lb / n, r = (unsigned)lb - q * n;
  const int t0 = sb + (int)(j * q + (j * r) / n);
  const int t1 = sb + (int)((j + 1) * q + ((j + 1) * r) / n);
  return make_int4(bi, t0, t1, nbb > 1 ? i : -1);
}

// The same for a wave-uniform i (a work-group's own item): x is non-decreasing
// in rank order, so the rank #{r : x_r <= i} is one ballot's population, and
// the rank's fields are read from its lane.
__device__ __forceinline__ int4 plan_wave_item_uniform(const WavePlan& P, int i) {
  if (i >= P.n_items) return make_int4(-1, 0, 0, -1);
  const int c = (int)__builtin_popcountll(__builtin_amdgcn_ballot_w64(P.x <= i));  // < 64: i < x_63
  const int bi = __builtin_amdgcn_readlane(P.seq_r, c);
  const int sb = __builtin_amdgcn_readlane(P.s0_r, c);
  const int lb = __builtin_amdgcn_readlane(P.len_r, c);
  const int nbb = __builtin_amdgcn_readlane(P.nb_r, c);
  const int fb = __builtin_amdgcn_readlane(P.x, c) - nbb;
  if (nbb <= 0) return make_int4(-1, 0, 0, -1);
  const unsigned j = (unsigned)(i - fb), n = (unsigned)nbb;
  const unsigned q = (unsigned)lb / n, r = (unsigned)lb - q * n;
  const int t0 = sb + (int)(j * q + (j * r) / n);
  const int t1 = sb + (int)((j + 1) * q + ((j + 1) * r) / n);
  return make_int4(bi, t0, t1, nbb > 1 ? i : -1);
}

// the rows' (first item, piece count) and the plan header
__device__ __forceinline__ void plan_wave_write_rows(const WavePlan& P, int batch, int max_items,
                                                     int32_t* __restrict__ plan) {
  const int lane = threadIdx.x & 63;
  if (lane < batch) reinterpret_cast<int2*>(plan + kPlanHeader + 4 * max_items)[lane] = make_int2(P.first, P.nb);
  if (lane == 0) {
    plan[0] = P.n_items;
    plan[1] = P.chunk;
    plan[2] = (int)(64u * P.hi64 + P.lo64);
    plan[3] = batch;
    plan[4] = max_items;
  }
}

// sum / max of one non-negative int per thread over the 256-thread block
// (`red` holds 4 ints; every thread gets the result)
__device__ __forceinline__ int block_sum(int v, int* red) {
  const int t = wave_sum(v);
  __syncthreads();  // red free
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = t;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}
__device__ __forceinline__ int block_max(int v, int* red) {
  const int t = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = t;
  __syncthreads();
  return max(max(red[0], red[1]), max(red[2], red[3]));
}

// exclusive scan of one int per thread over the 256-thread block; *total =
// the block sum (same in every thread)
__device__ __forceinline__ int block_exscan(int v, int* red, int* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int x = wave_incl_sum(v);
  __syncthreads();  // red free
  if (lane == 63) red[w] = x;
  __syncthreads();
  int base = 0;
  for (int i = 0; i < w; ++i) base += red[i];
  *total = red[0] + red[1] + red[2] + red[3];
  return base + x - v;
}

// Up to 256 rows, one per thread of a 256-thread block (every thread must
// call it): the block form of the plan, which the planner kernel uses above
// 64 rows and the 16-head decode for up to 256.  Thread b < batch gets row
// b's length, piece count, first key and first item; every thread gets the
// chunk, the item count and the length sums.  Scratch: 256 keys (8 bytes
// each), 256 counts and kPlanRedInts ints of LDS; it ends with a barrier after
// its last scratch read.  The chunk is the one-wave plan's (the same search
// bounds, the same closed form for equal lengths), found three candidates a
// round; each reduction round is one barrier, its partials in one of two
// banks of s_red that alternate, so a bank is rewritten only after every
// thread has passed the barrier that follows its reads.
struct BlockPlan {
  int chunk, n_items;
  unsigned hi64, lo64;
  int L, nb, s0, first;
};
constexpr int kPlanRedInts = 64;
__device__ __forceinline__ BlockPlan plan_block(const int32_t* __restrict__ kv_indptr, int batch, int qlen,
                                                int target_items, int min_chunk, int max_splits,
                                                uint64_t* s_key, int* s_cnt, int* s_red) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const bool act = tid < batch;
  BlockPlan P;
  P.L = act ? row_len(kv_indptr, tid, qlen) : 0;
  P.s0 = act ? row_start(kv_indptr, tid, qlen) : 0;
  const int L64 = (P.L + 63) >> 6;
  // round 1 (bank 0): sums of L >> 6, L & 63 and ceil(L / 64), max of L, min of ceil(L / 64)
  {
    const int a0 = wave_sum(P.L >> 6), a1 = wave_sum(P.L & 63), a2 = wave_max(P.L), a3 = wave_sum(L64);
    const int a4 = wave_max(act ? -L64 : -0x7FFFFFFF);
    if (lane == 0) {
      s_red[w] = a0;
      s_red[4 + w] = a1;
      s_red[8 + w] = a2;
      s_red[12 + w] = a3;
      s_red[16 + w] = a4;
    }
  }
  __syncthreads();
  P.hi64 = (unsigned)(s_red[0] + s_red[1] + s_red[2] + s_red[3]);
  P.lo64 = (unsigned)(s_red[4] + s_red[5] + s_red[6] + s_red[7]);
  const int lmax = max(max(s_red[8], s_red[9]), max(s_red[10], s_red[11]));
  const unsigned s64 = (unsigned)(s_red[12] + s_red[13] + s_red[14] + s_red[15]);
  const int l64min = -max(max(s_red[16], s_red[17]), max(s_red[18], s_red[19]));
  int lo = max(min_chunk / 64, (int)tiles_per_item(P.hi64, P.lo64, target_items));
  if (max_splits > 0) lo = max(lo, ((lmax + 63) / 64 + max_splits - 1) / max_splits);
  // m = ceil(s64 / (target - batch)) already fits (at most s64 / m + batch items)
  int hi = (lmax + 63) / 64;
  if (target_items > batch)
    hi = min(hi, (int)((s64 + (unsigned)(target_items - batch) - 1u) / (unsigned)(target_items - batch)));
  hi = max(lo, hi);
  if (l64min == (lmax + 63) / 64) {  // every row as long: the count at m is batch ceil(L64 / m)
    const int k = target_items / max(batch, 1);
    lo = hi = k > 0 ? min(hi, max(lo, (l64min + k - 1) / k)) : hi;
  }
  // smallest m in [lo, hi) whose item count fits the target (else hi): the
  // count is non-increasing in m; three probes a round keep the answer in [lo, hi]
  int bank = 1;
  while (lo < hi) {
    const int d = hi - lo;
    const int m1 = lo + d / 4, m2 = lo + d / 2, m3 = lo + (3 * d) / 4;
    auto cnt = [&](int m) { return act ? (L64 > 0 ? (L64 + m - 1) / m : 1) : 0; };
    const int c1 = wave_sum(cnt(m1)), c2 = wave_sum(cnt(m2)), c3 = wave_sum(cnt(m3));
    int* rb = s_red + 32 * bank;
    if (lane == 0) {
      rb[w] = c1;
      rb[4 + w] = c2;
      rb[8 + w] = c3;
    }
    __syncthreads();
    const int n1 = rb[0] + rb[1] + rb[2] + rb[3], n2 = rb[4] + rb[5] + rb[6] + rb[7];
    const int n3 = rb[8] + rb[9] + rb[10] + rb[11];
    if (n1 <= target_items) {
      hi = m1;
    } else if (n2 <= target_items) {
      lo = m1 + 1;
      hi = m2;
    } else if (n3 <= target_items) {
      lo = m2 + 1;
      hi = m3;
    } else {
      lo = m3 + 1;
    }
    bank ^= 1;
  }
  P.chunk = lo * 64;
  P.nb = act ? (P.L > 0 ? (P.L + P.chunk - 1) / P.chunk : 1) : 0;
  // rank rows by piece length, longest first (ties by index); equal pieces on
  // every row leave them in index order
  const int piece = act ? (P.L > 0 ? (P.L + P.nb - 1) / P.nb : 0) : -1;
  {
    const int a0 = wave_max(act ? piece : 0), a1 = wave_max(act ? -piece : -0x7FFFFFFF);
    int* rb = s_red + 32 * bank;
    if (lane == 0) {
      rb[w] = a0;
      rb[4 + w] = a1;
    }
  }
  __syncthreads();
  const int* rp = s_red + 32 * bank;
  const int pmax = max(max(rp[0], rp[1]), max(rp[2], rp[3]));
  const int npmin = max(max(rp[4], rp[5]), max(rp[6], rp[7]));
  int rank = tid;
  if (pmax != -npmin) {
    rank = 0;
    if (pmax < (1 << 23)) {
      // key = (piece + 1) 256 + 255 - b: a larger key ranks earlier, "no row"
      // is 0, below every real one; four keys per 16-byte LDS read
      uint32_t* k32 = reinterpret_cast<uint32_t*>(s_key);
      const uint32_t key = act ? ((uint32_t)(piece + 1) << 8) | (uint32_t)(255 - tid) : 0u;
      k32[tid] = key;
      __syncthreads();
      if (act) {
        const uint4* kv = reinterpret_cast<const uint4*>(k32);
#pragma unroll 8
        for (int b2 = 0; b2 < (batch + 3) / 4; ++b2) {
          const uint4 q = kv[b2];
          rank += (q.x > key) + (q.y > key) + (q.z > key) + (q.w > key);
        }
      }
    } else {
      // key = piece << 32 | (2^32 - 1 - b), two per 16-byte LDS read
      const uint64_t key = piece < 0 ? 0ull : ((uint64_t)(uint32_t)piece << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)tid);
      s_key[tid] = key;
      __syncthreads();
      if (act) {
        const ulonglong2* kv = reinterpret_cast<const ulonglong2*>(s_key);
#pragma unroll 8
        for (int b2 = 0; b2 < (batch + 1) / 2; ++b2) {
          const ulonglong2 q = kv[b2];
          rank += (q.x > key) + (q.y > key);
        }
      }
    }
  }
  if (act) s_cnt[rank] = P.nb;
  __syncthreads();
  int total = 0;
  const int ex = block_exscan(tid < batch ? s_cnt[tid] : 0, s_red, &total);
  __syncthreads();
  if (tid < batch) s_cnt[tid] = ex;
  __syncthreads();
  P.first = act ? s_cnt[rank] : 0;
  P.n_items = total;
  __syncthreads();  // every scratch read done
  return P;
}

}  // namespace mla
