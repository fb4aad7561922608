// Gather-ceiling probe: the decode kernels' KV gather with no compute, to
// measure what HBM rate a given cache layout and issue scheme can reach.
//
// The token stream (kv_indices) is cut into 64-token tiles; work-group g takes
// tiles g, g + G, ... (a perfectly balanced persistent split).  Per tile the
// rows named by kv_indices are fetched exactly as the decode kernels fetch
// them: the tile's 64 slot indices arrive in an LDS slot ring by one dword
// LDS-DMA, several tiles ahead; the rows then arrive by 16-byte LDS-DMAs
// (global_load_lds_dwordx4) into an S-stage ring, with a per-wave vmcnt wait
// and a work-group barrier per tile.  Every wave reads one word of each tile it
// waits for, so the data is consumed.  Variants:
//   layout 0  fp8 rows of 576 B (K = V)                           36 DMAs / tile
//   layout 1  fp4 rows of 288 B + their 18 e8m0 bytes (K = V)      18 + scales
//   layout 2  layout 1 for K + fp8 V rows of 512 B from a second cache
//   method 0  scale bytes by 6 dword DMAs per tile (each lane = one token,
//             dword j of the aligned span that holds its 18 bytes)
//   method 1  scale bytes by 18 one-byte DMAs per tile
//   method 2  layout 0 rows by plain 16-byte loads into registers (two tiles
//             in flight per wave), no LDS ring for the rows
//   method 3  contiguous stream of the same bytes (no indices), plain loads
// Not a reference component: it exists to put a measured ceiling beside the
// decode kernels' HBM rates.
#include "../../include/mla_mi355x.h"
#include "mla_internal.hpp"

namespace mla {
namespace {

template <int LAYOUT, int METHOD>
struct ProbeShape {
  static constexpr int ROWS16 = LAYOUT == 0 ? 36 : 18;          // 16-B chunks of the first row segment
  static constexpr int V16 = LAYOUT == 2 ? 32 : 0;              // of the fp8 V segment
  static constexpr int NROW = ROWS16 + V16;                     // row DMAs per tile (64 chunks each)
  static constexpr int NSC = LAYOUT == 0 ? 0 : (METHOD == 1 ? 18 : 6);  // scale DMAs per tile
  static constexpr int NI = NROW + NSC;                         // DMA instructions per tile
  static constexpr int STAGE = NI * 1024;                       // one KiB of LDS per instruction
};

constexpr int kProbeNSL = 8;  // slot ring stages

template <int LAYOUT, int METHOD, int NW, int S>
__global__ __launch_bounds__(64 * NW) void probe_dma_kernel(const uint8_t* __restrict__ rows, int64_t row_stride,
                                                            const uint8_t* __restrict__ scales,
                                                            int64_t scale_stride, const uint8_t* __restrict__ vrows,
                                                            int64_t v_row_stride, const int32_t* __restrict__ idx,
                                                            int ntiles, uint32_t* __restrict__ sink) {
  using P = ProbeShape<LAYOUT, METHOD>;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
  const uint32_t slot0 = lds0 + S * P::STAGE;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int G = gridDim.x;
  const int my_tiles = ntiles > (int)blockIdx.x ? (ntiles - 1 - (int)blockIdx.x) / G + 1 : 0;
  // instruction k of a tile is issued by wave k % NW; D0 = count of wave 0
  constexpr int KW = (P::NI + NW - 1) / NW;
  const int nmine = P::NI / NW + (w < P::NI % NW ? 1 : 0);

  auto tile_of = [&](int j) { return (int)blockIdx.x + G * j; };  // j-th tile of this group
  auto issue_slots = [&](int j) {
    if (w == 0) {
      const int t = min(tile_of(j), ntiles - 1);  // past the end: any valid tile (uniform counts)
      dma4_to_lds(idx + 64 * t + lane, slot0 + (j % kProbeNSL) * 256);
    }
  };
  auto issue_rows = [&](int j) {
    const int* sl = reinterpret_cast<const int*>(smem + S * P::STAGE + (j % kProbeNSL) * 256);
    const uint32_t sb = lds0 + (j % S) * P::STAGE;
    const uint8_t* src[KW];
#pragma unroll
    for (int i = 0; i < KW; ++i) {  // all slot reads before the first DMA (asm is a memory barrier)
      const int k = w + NW * i;
      src[i] = nullptr;
      if (k < P::ROWS16) {
        const int e = 64 * k + lane, tok = e / P::ROWS16, ch = e - tok * P::ROWS16;
        src[i] = rows + (int64_t)sl[tok] * row_stride + 16 * ch;
      } else if (k < P::NROW) {
        const int e = 64 * (k - P::ROWS16) + lane, tok = e / 32, ch = e - tok * 32;
        src[i] = vrows + (int64_t)sl[tok] * v_row_stride + 16 * ch;
      } else if (k < P::NI) {
        const int j8 = k - P::NROW;  // scale instruction: lane = token
        const int64_t b0 = (int64_t)sl[lane] * scale_stride;
        src[i] = METHOD == 1 ? scales + b0 + j8 : scales + ((b0 & ~3LL) + 4 * j8);
      }
    }
#pragma unroll
    for (int i = 0; i < KW; ++i) {
      const int k = w + NW * i;
      if (k < P::NROW) dma16_to_lds(src[i], sb + 1024 * k);
      else if (k < P::NI) {
        if (METHOD == 1) dma1_to_lds(src[i], sb + 1024 * k);
        else dma4_to_lds(src[i], sb + 1024 * k);
      }
    }
  };
  // pass j issues slots(j + S + 1) then rows(j + S - 1); at its top rows(j) and
  // slots(j + S - 1) (issued in pass j - 2) must have landed
  auto wait_top = [&]() {
    const int d = nmine;
    if constexpr (S == 2) {
      wait_vmcnt<0>();
    } else if constexpr (S == 3) {
      if (w == 0) { if (d == KW) wait_vmcnt<KW + 1>(); else wait_vmcnt<KW>(); }
      else { if (d == KW) wait_vmcnt<KW>(); else wait_vmcnt<KW - 1>(); }
    } else {
      if (w == 0) { if (d == KW) wait_vmcnt<2 * KW + 1>(); else wait_vmcnt<2 * KW - 1>(); }
      else { if (d == KW) wait_vmcnt<2 * KW>(); else wait_vmcnt<2 * KW - 2>(); }
    }
  };
  uint32_t acc = 0;
  if (my_tiles > 0) {
    for (int j = 0; j < S + 1; ++j) issue_slots(j);
    wait_vmcnt<0>();
    lds_barrier();
    for (int j = 0; j < S - 1; ++j) {
      issue_slots(j + S + 1);
      issue_rows(j);
    }
    for (int j = 0; j < my_tiles; ++j) {
      wait_top();
      lds_barrier();  // rows(j) visible; stage of j - 1 free
      issue_slots(j + S + 1);
      issue_rows(j + S - 1);  // past the item: fetches a valid tile (counts stay uniform)
      acc ^= reinterpret_cast<const uint32_t*>(smem + (j % S) * P::STAGE)[threadIdx.x];
    }
    wait_vmcnt<0>();
  }
  if (acc == 0x9E3779B9u) sink[threadIdx.x] = acc;  // keeps the reads live
}

// method 2: layout-0 rows by plain 16-byte loads into registers; slots from
// the same LDS ring; two tiles of loads in flight per wave
template <int NW>
__global__ __launch_bounds__(64 * NW) void probe_reg_kernel(const uint8_t* __restrict__ rows, int64_t row_stride,
                                                            const int32_t* __restrict__ idx, int ntiles,
                                                            uint32_t* __restrict__ sink) {
  constexpr int NI = 36, KW = (NI + NW - 1) / NW;
  __shared__ int sl_ring[kProbeNSL][64];
  const uint32_t slot0 = (uint32_t)(uintptr_t)&sl_ring[0][0];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int G = gridDim.x;
  const int my_tiles = ntiles > (int)blockIdx.x ? (ntiles - 1 - (int)blockIdx.x) / G + 1 : 0;
  auto issue_slots = [&](int j) {
    if (w == 0) {
      const int t = min((int)blockIdx.x + G * j, ntiles - 1);
      dma4_to_lds(idx + 64 * t + lane, slot0 + (j % kProbeNSL) * 256);
    }
  };
  auto load = [&](int j, uint4 (&v)[KW]) {
    const int* sl = sl_ring[j % kProbeNSL];
    int s[KW];
#pragma unroll
    for (int i = 0; i < KW; ++i) {
      const int k = min(w + NW * i, NI - 1);
      const int e = 64 * k + lane, tok = e / 36;
      s[i] = sl[tok];
    }
#pragma unroll
    for (int i = 0; i < KW; ++i) {
      const int k = min(w + NW * i, NI - 1);
      const int e = 64 * k + lane, tok = e / 36, ch = e - tok * 36;
      v[i] = ldg16_nt(rows + (int64_t)s[i] * row_stride + 16 * ch);
    }
  };
  uint32_t acc = 0;
  uint4 a[KW], b[KW];
  if (my_tiles > 0) {
    for (int j = 0; j < 4; ++j) issue_slots(j);
    wait_vmcnt<0>();
    lds_barrier();
    load(0, a);
    for (int j = 0; j < my_tiles; j += 2) {
      issue_slots(j + 4);
      load(j + 1, b);  // past the item: a valid tile
      wait_vmcnt<KW + 1>();
#pragma unroll
      for (int i = 0; i < KW; ++i) acc ^= a[i].x ^ a[i].w;
      lds_barrier();  // slot ring stage reuse, and the per-tile sync of a real kernel
      issue_slots(j + 5);
      load(j + 2, a);
      wait_vmcnt<KW + 1>();
#pragma unroll
      for (int i = 0; i < KW; ++i) acc ^= b[i].x ^ b[i].w;
      lds_barrier();
    }
    wait_vmcnt<0>();
  }
  if (acc == 0x9E3779B9u) sink[threadIdx.x] = acc;
}

// method 3: contiguous stream, 4 independent 16-byte loads per thread in flight
__global__ __launch_bounds__(256) void probe_stream_kernel(const uint4* __restrict__ x, int64_t n16,
                                                           uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    uint4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = ldg16_nt(x + i + k * stride);
#pragma unroll
    for (int k = 0; k < 4; ++k) acc ^= v[k].x ^ v[k].w;
  }
  for (; i < n16; i += stride) {
    const uint4 v = ldg16_nt(x + i);
    acc ^= v.x ^ v.w;
  }
  if (acc == 0x9E3779B9u) sink[threadIdx.x] = acc;
}

// ---------------------------------------------------------------------------
// LDS read-pattern probe: each wave repeats 8 LDS reads of one pattern `iters`
// times and records its shader-clock cycles per read instruction, so a bank
// counter pass (SQ_LDS_BANK_CONFLICT, SQ_ACTIVE_INST_LDS) over these kernels
// shows what the counters read for reads that cannot conflict beside the
// decode kernels' own patterns:
//   0  ds_read_b128, lane l at 16 l (+1 KiB per read): contiguous, no conflict
//   1  ds_read_b128, the 128-head fp8 K fragment reads: 608-byte rows, 16-byte
//      chunk c of row r at 16 (c ^ ((r >> 2) & 7)) (c < 32), lane (l32, hh)
//      reads row l32, chunks 4 ks + 2 hh + j (ks < 4, j < 2)
//   2  ds_read_b64_tr_b8, lane l at 8 l (+512 B per read): contiguous
//   3  ds_read_b64_tr_b8, the 128-head V^T reads: lane (G, m, oo) reads row
//      T0 + 16 cc, chunk 2 dt + (G & 1), byte 8 oo, T0 = 8 (m >> 2) + 4 hh + (m & 3)
//   4  ds_read_b128, lane l at 512 l mod 32 KiB: every lane on the same banks
// ---------------------------------------------------------------------------
constexpr int kLdsProbeBytes = 64 * 608;

__device__ __forceinline__ uint32_t k608(int r, int c) {
  const int x = (r >> 2) & 7;
  return (uint32_t)(r * 608 + 16 * (c < 32 ? (c ^ x) : 32 + ((c - 32) ^ (x & 3))));
}

template <int PAT>
__global__ __launch_bounds__(256) void probe_lds_kernel(int iters, float* __restrict__ cycles,
                                                        uint32_t* __restrict__ sink) {
  __shared__ __attribute__((aligned(16))) uint8_t buf[kLdsProbeBytes];
  for (int i = threadIdx.x; i < kLdsProbeBytes / 16; i += 256)
    reinterpret_cast<uint4*>(buf)[i] = make_uint4(i, i * 3u, i * 5u, i * 7u);
  __syncthreads();
  const int lane = threadIdx.x & 63, l32 = lane & 31, hh = lane >> 5;
  const uint32_t base = (uint32_t)(uintptr_t)buf;
  uint32_t off[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if constexpr (PAT == 0) off[i] = 16 * lane + 1024 * i;
    else if constexpr (PAT == 1) off[i] = k608(l32, 4 * (i >> 1) + 2 * hh + (i & 1));
    else if constexpr (PAT == 2) off[i] = 8 * lane + 512 * i;
    else if constexpr (PAT == 3) {
      const int G = lane >> 4, m = (lane & 15) >> 1, oo = lane & 1;
      const int T0 = 8 * (m >> 2) + 4 * hh + (m & 3);
      off[i] = k608(T0 + 16 * (i & 3), 2 * (i >> 2) + (G & 1)) + 8 * oo;
    } else {
      off[i] = (512 * lane + 16 * i) % 32768;
    }
  }
  uint32_t acc = 0;
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i) asm volatile("" : "+v"(off[i]));  // no hoisting out of the loop
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (PAT == 2 || PAT == 3) {
        const v2i v = lds_read_tr8(base + off[i]);
        acc ^= (uint32_t)v[0] ^ (uint32_t)v[1];
      } else {
        const uint4 v = *reinterpret_cast<const uint4*>(buf + off[i]);
        acc ^= v.x ^ v.w;
      }
    }
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  if (lane == 0) cycles[blockIdx.x * 4 + (threadIdx.x >> 6)] = (float)(t1 - t0) / (8.0f * (float)iters);
  if (acc == 0x9E3779B9u) sink[threadIdx.x] = acc;
}

template <int LAYOUT, int METHOD, int NW, int S>
hipError_t launch_dma(int grid, const uint8_t* rows, int64_t rs, const uint8_t* sc, int64_t ss, const uint8_t* v,
                      int64_t vs, const int32_t* idx, int ntiles, uint32_t* sink, hipStream_t st) {
  using P = ProbeShape<LAYOUT, METHOD>;
  const int lds = S * P::STAGE + kProbeNSL * 256;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&probe_dma_kernel<LAYOUT, METHOD, NW, S>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((probe_dma_kernel<LAYOUT, METHOD, NW, S>), dim3(grid), dim3(64 * NW), lds, st, rows, rs, sc,
                     ss, v, vs, idx, ntiles, sink);
  return hipGetLastError();
}

}  // namespace
}  // namespace mla

using namespace mla;

extern "C" {

int mla_probe_lds(int pattern, int iters, int groups, float* cycles, void* sink, void* stream) {
  if (iters < 1 || groups < 1 || groups > 65535) return set_error(MLA_ERR_INVALID_ARGUMENT, "iters, groups >= 1");
  if (!cycles || !sink) return set_error(MLA_ERR_INVALID_ARGUMENT, "null cycles or sink");
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint32_t* sk = static_cast<uint32_t*>(sink);
  switch (pattern) {
    case 0: hipLaunchKernelGGL(probe_lds_kernel<0>, dim3(groups), dim3(256), 0, st, iters, cycles, sk); break;
    case 1: hipLaunchKernelGGL(probe_lds_kernel<1>, dim3(groups), dim3(256), 0, st, iters, cycles, sk); break;
    case 2: hipLaunchKernelGGL(probe_lds_kernel<2>, dim3(groups), dim3(256), 0, st, iters, cycles, sk); break;
    case 3: hipLaunchKernelGGL(probe_lds_kernel<3>, dim3(groups), dim3(256), 0, st, iters, cycles, sk); break;
    case 4: hipLaunchKernelGGL(probe_lds_kernel<4>, dim3(groups), dim3(256), 0, st, iters, cycles, sk); break;
    default: return set_error(MLA_ERR_INVALID_ARGUMENT, "pattern must be 0..4");
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(MLA_ERR_HIP, "probe launch: %s", hipGetErrorString(e));
  return MLA_OK;
}

int mla_probe_gather(int layout, int method, int waves, int stages, int groups, const void* rows,
                     int64_t row_stride, const void* scales, int64_t scale_stride, const void* v_rows,
                     int64_t v_row_stride, const int32_t* kv_indices, int64_t ntokens, void* sink, void* stream) {
  if (ntokens < 64 || (ntokens % 64) != 0 || ntokens / 64 > (1LL << 30))
    return set_error(MLA_ERR_INVALID_ARGUMENT, "ntokens must be a positive multiple of 64");
  if (groups < 1 || groups > 65535) return set_error(MLA_ERR_INVALID_ARGUMENT, "groups must be in [1, 65535]");
  if (!rows || !sink) return set_error(MLA_ERR_INVALID_ARGUMENT, "null rows or sink");
  if (method != 3 && !kv_indices) return set_error(MLA_ERR_INVALID_ARGUMENT, "kv_indices needed");
  if (layout != 0 && method != 3 && (!scales || scale_stride < kMxBlocks))
    return set_error(MLA_ERR_INVALID_ARGUMENT, "fp4 layouts need scales with stride >= 18");
  if (layout == 2 && !v_rows) return set_error(MLA_ERR_INVALID_ARGUMENT, "layout 2 needs v_rows");
  const int nt = (int)(ntokens / 64);
  const uint8_t* r = static_cast<const uint8_t*>(rows);
  const uint8_t* sc = static_cast<const uint8_t*>(scales);
  const uint8_t* v = static_cast<const uint8_t*>(v_rows);
  uint32_t* sk = static_cast<uint32_t*>(sink);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = hipErrorInvalidValue;
  const int key = layout * 1000 + method * 100 + waves * 10 + stages;
  switch (key) {
    case 44: e = launch_dma<0, 0, 4, 4>(groups, r, row_stride, sc, scale_stride, v, v_row_stride, kv_indices, nt, sk, st); break;
    case 43: e = launch_dma<0, 0, 4, 3>(groups, r, row_stride, sc, scale_stride, v, v_row_stride, kv_indices, nt, sk, st); break;
    case 42: e = launch_dma<0, 0, 4, 2>(groups, r, row_stride, sc, scale_stride, v, v_row_stride, kv_indices, nt, sk, st); break;
    case 84: e = launch_dma<0, 0, 8, 4>(groups, r, row_stride, sc, scale_stride, v, v_row_stride, kv_indices, nt, sk, st); break;
    case 82: e = launch_dma<0, 0, 8, 2>(groups, r, row_stride, sc, scale_stride, v, v_row_stride, kv_indices, nt, sk, st); break;
    case 1044: e = launch_dma<1, 0, 4, 4>(groups, r, row_stride, sc, scale_stride, v, v_row_stride, kv_indices, nt, sk, st); break;
    case 1043: e = launch_dma<1, 0, 4, 3>(groups, r, row_stride, sc, scale_stride, v, v_row_stride, kv_indices, nt, sk, st); break;
    case 1084: e = launch_dma<1, 0, 8, 4>(groups, r, row_stride, sc, scale_stride, v, v_row_stride, kv_indices, nt, sk, st); break;
    case 1143: e = launch_dma<1, 1, 4, 3>(groups, r, row_stride, sc, scale_stride, v, v_row_stride, kv_indices, nt, sk, st); break;
    case 2042: e = launch_dma<2, 0, 4, 2>(groups, r, row_stride, sc, scale_stride, v, v_row_stride, kv_indices, nt, sk, st); break;
    case 2082: e = launch_dma<2, 0, 8, 2>(groups, r, row_stride, sc, scale_stride, v, v_row_stride, kv_indices, nt, sk, st); break;
    case 2142: e = launch_dma<2, 1, 4, 2>(groups, r, row_stride, sc, scale_stride, v, v_row_stride, kv_indices, nt, sk, st); break;
    case 240:
      hipLaunchKernelGGL(probe_reg_kernel<4>, dim3(groups), dim3(256), 0, st, r, row_stride, kv_indices, nt, sk);
      e = hipGetLastError();
      break;
    case 280:
      hipLaunchKernelGGL(probe_reg_kernel<8>, dim3(groups), dim3(512), 0, st, r, row_stride, kv_indices, nt, sk);
      e = hipGetLastError();
      break;
    default:
      if (method == 3 && waves == 4) {
        hipLaunchKernelGGL(probe_stream_kernel, dim3(groups), dim3(256), 0, st, reinterpret_cast<const uint4*>(r),
                           (int64_t)ntokens * row_stride / 16, sk);
        e = hipGetLastError();
      } else {
        return set_error(MLA_ERR_UNSUPPORTED, "no probe variant layout %d method %d waves %d stages %d", layout,
                         method, waves, stages);
      }
  }
  if (e != hipSuccess) return set_error(MLA_ERR_HIP, "probe launch: %s", hipGetErrorString(e));
  return MLA_OK;
}

}  // extern "C"
