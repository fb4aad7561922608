// The per-head products either side of the absorbed decode (DeepSeek-style
// MLA): W_UK absorption (q_nope [B,H,128] x W_UK [H,128,512], written into the
// decode's Q [B,H,576] next to the rope columns) and v_up_proj (o [B,H,512] x
// W_UV [H,512,128], optionally followed by the per-tensor FP8 quantizer).  The
// reference names these steps but does not implement them
// (mixed-mla/README.md:213-217).
//
// Both are batched GEMMs with M = batch rows per head and the weights read
// once: a work-group owns one head and a slice of output columns, stages that
// weight slice transposed in LDS (transposed in registers, 8x8 bf16 at a time,
// so a B fragment is one 16-byte LDS read), and then runs every batch row
// against it, 64 rows at a time (16 per wave), on 16x16x32 bf16 MFMAs with f32
// accumulation; the first chunk's rows are loaded while the weights land.  Results are staged per wave and written as
// 16-byte row segments; the maximum |y| of the work-group (bf16 bits) goes to a
// partial-max slot that the FP8 quantizer folds.
#include "mla_internal.hpp"

namespace mla {

template <int K, int N, int NB>
struct Bmm {
  static_assert(NB % 16 == 0 && N % NB == 0 && K % 32 == 0, "tile shape");
  static constexpr int WST = K + 8;    // transposed weight row stride (bf16): NB columns x K
  static constexpr int OST = NB + 8;   // output staging row stride (bf16)
  static constexpr int NT = NB / 16;   // 16-column MFMA tiles per wave
  static constexpr int KS = K / 32;    // 32-deep MFMA steps
  static constexpr int LDS = 2 * (NB * WST + 4 * 16 * OST);
};

// y[b, h, ycol0 + n] = sum_k x[b, h, k] w[h, k, n]; grid (H, N / NB [+ 1 for
// the rope copy]); rows b >= B are skipped.  x rows: stride xs elements per
// (b, h); y rows: stride ys.  rope (optional): [B, H, 64] bf16 copied to
// y[b, h, ycol0 + N ..].  amax (optional): one partial max of |y| per block.
template <int K, int N, int NB>
__global__ __launch_bounds__(256) void bmm_heads_kernel(const uint16_t* __restrict__ x, int xs,
                                                        const uint16_t* __restrict__ w,
                                                        const uint16_t* __restrict__ rope,
                                                        uint16_t* __restrict__ y, int ys, int ycol0, int B,
                                                        int H, uint32_t* __restrict__ amax) {
  using C = Bmm<K, N, NB>;
  __shared__ __attribute__((aligned(16))) uint16_t lds[C::LDS / 2];
  uint16_t* wt = lds;                    // [NB][WST]: wt[n][k] = w[h][k][n0 + n]
  const int h = blockIdx.x, tid = threadIdx.x;
  const int wv = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
  uint16_t* st = lds + NB * C::WST + wv * 16 * C::OST;  // this wave's [16][OST] output tile

  if ((int)blockIdx.y == N / NB) {  // rope columns pass through
    for (int i = tid; i < B * 8; i += 256) {
      const int b = i >> 3, c = i & 7;
      *reinterpret_cast<uint4*>(y + ((int64_t)b * H + h) * ys + ycol0 + N + 8 * c) =
          *reinterpret_cast<const uint4*>(rope + ((int64_t)b * H + h) * 64 + 8 * c);
    }
    if (amax != nullptr && tid == 0) amax[blockIdx.y * H + h] = 0;
    return;
  }
  const int n0 = NB * blockIdx.y;

  // this lane's A fragments of the first 64-row chunk, in flight while the
  // weights are staged
  uint4 av[C::KS];
  auto load_a = [&](int row0) {
    const int ra = row0 + 16 * wv + l16;
    const uint16_t* xr = x + ((int64_t)min(ra, B - 1) * H + h) * xs + 8 * g;
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) av[ks] = *reinterpret_cast<const uint4*>(xr + 32 * ks);
  };
  load_a(0);

  // weight slice, transposed in registers: a task is 8 rows k x 8 columns,
  // eight 16-byte loads in, eight 16-byte LDS rows out (wt[n][k0 .. k0 + 7])
  const uint16_t* wh = w + (int64_t)h * K * N + n0;
  for (int t = tid; t < (K / 8) * (NB / 8); t += 256) {
    const int c = t % (NB / 8), k0 = 8 * (t / (NB / 8));
    uint32_t r[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint4 v = *reinterpret_cast<const uint4*>(wh + (int64_t)(k0 + i) * N + 8 * c);
      r[i][0] = v.x; r[i][1] = v.y; r[i][2] = v.z; r[i][3] = v.w;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t lo = r[2 * i][j >> 1], hi = r[2 * i + 1][j >> 1];
        o[i] = (j & 1) ? ((lo >> 16) | (hi & 0xFFFF0000u)) : ((lo & 0xFFFFu) | (hi << 16));
      }
      *reinterpret_cast<uint4*>(wt + (8 * c + j) * C::WST + k0) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
  __syncthreads();

  uint32_t mx = 0;
  for (int row0 = 0; row0 < B; row0 += 64) {
    if (row0 > 0) load_a(row0);
    const bool live = row0 + 16 * wv + l16 < B;  // rows past B multiply as zeros
    v4f acc[C::NT];
#pragma unroll
    for (int nt = 0; nt < C::NT; ++nt) acc[nt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
      const v8bf a = __builtin_bit_cast(v8bf, live ? av[ks] : make_uint4(0, 0, 0, 0));
#pragma unroll
      for (int nt = 0; nt < C::NT; ++nt) {
        const v8bf bb = *reinterpret_cast<const v8bf*>(wt + (16 * nt + l16) * C::WST + 32 * ks + 8 * g);
        acc[nt] = mfma16x32_bf16(a, bb, acc[nt]);
      }
    }
    // D[row 4g + r][col 16nt + l16] -> staging -> 16-byte row segments
#pragma unroll
    for (int nt = 0; nt < C::NT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t bits = f32_to_bf16_bits(acc[nt][r]);
        st[(4 * g + r) * C::OST + 16 * nt + l16] = (uint16_t)bits;
        if (row0 + 16 * wv + 4 * g + r < B) mx = max(mx, bits & 0x7FFFu);
      }
    __syncthreads();  // staging written (every wave runs the same row loop)
    for (int e = lane; e < 16 * (NB / 8); e += 64) {  // 16 rows x NB / 8 segments
      const int r = e / (NB / 8), c = e % (NB / 8);
      const int b = row0 + 16 * wv + r;
      if (b < B)
        *reinterpret_cast<uint4*>(y + ((int64_t)b * H + h) * ys + ycol0 + n0 + 8 * c) =
            *reinterpret_cast<const uint4*>(st + r * C::OST + 8 * c);
    }
    __syncthreads();  // staging read before the next chunk rewrites it
  }
  if (amax != nullptr) {
    mx = (uint32_t)wave_max((int)mx);
    __shared__ uint32_t red[4];
    if (lane == 0) red[wv] = mx;
    __syncthreads();
    if (tid == 0) amax[blockIdx.y * H + h] = max(max(red[0], red[1]), max(red[2], red[3]));
  }
}

// Columns per work-group: absorb_q's 512 outputs in 64-wide slices (9 x H
// work-groups with the rope copy), v_up_proj's 128 in 32-wide ones (4 x H).
constexpr int kAbsorbCols = 64;
constexpr int kUpCols = 32;

hipError_t launch_absorb_q(const uint16_t* q_nope, const uint16_t* q_rope, const uint16_t* w_uk, int batch,
                           int heads, uint16_t* q_out, hipStream_t stream) {
  hipLaunchKernelGGL((bmm_heads_kernel<128, 512, kAbsorbCols>), dim3(heads, 512 / kAbsorbCols + 1), dim3(256), 0,
                     stream, q_nope, 128,
                     w_uk, q_rope, q_out, kQKDim, 0, batch, heads, nullptr);
  return hipGetLastError();
}

hipError_t launch_v_up_proj(const uint16_t* o, const uint16_t* w_uv, int batch, int heads, uint16_t* y,
                            uint32_t* amax_partials, int* nparts, hipStream_t stream) {
  *nparts = heads * (128 / kUpCols);
  hipLaunchKernelGGL((bmm_heads_kernel<512, 128, kUpCols>), dim3(heads, 128 / kUpCols), dim3(256), 0, stream, o,
                     kVDim, w_uv, nullptr, y, 128, 0, batch, heads, amax_partials);
  return hipGetLastError();
}

}  // namespace mla
