// The per-head products either side of the absorbed decode (DeepSeek-style
// MLA): W_UK absorption (q_nope [B,H,128] x W_UK [H,128,512], written into the
// decode's Q [B,H,576] next to the rope columns) and v_up_proj (o [B,H,512] x
// W_UV [H,512,128], optionally followed by the per-tensor FP8 quantizer).  The
// reference names these steps but does not implement them
// (mixed-mla/README.md:213-217).
//
// Both are batched GEMMs with M = batch rows per head and the weights read
// once: a work-group owns one head and 64 output columns, stages that weight
// slice transposed in LDS (so a B fragment is one 16-byte LDS read), and then
// runs every batch row against it, 64 rows at a time (16 per wave), on 16x16x32
// bf16 MFMAs with f32 accumulation.  Results are staged per wave and written as
// 16-byte row segments; the maximum |y| of the work-group (bf16 bits) goes to a
// partial-max slot that the FP8 quantizer folds.
#include "mla_internal.hpp"

namespace mla {

template <int K, int N>
struct Bmm {
  static constexpr int WST = K + 8;    // transposed weight row stride (bf16): 64 columns x K
  static constexpr int OST = 64 + 8;   // output staging row stride (bf16)
  static constexpr int LDS = 2 * (64 * WST + 4 * 16 * OST);
};

// y[b, h, ycol0 + n] = sum_k x[b, h, k] w[h, k, n]; grid (H, N / 64 [+ 1 for
// the rope copy]); rows b >= B are skipped.  x rows: stride xs elements per
// (b, h); y rows: stride ys.  rope (optional): [B, H, 64] bf16 copied to
// y[b, h, ycol0 + N ..].  amax (optional): one partial max of |y| per block.
template <int K, int N>
__global__ __launch_bounds__(256) void bmm_heads_kernel(const uint16_t* __restrict__ x, int xs,
                                                        const uint16_t* __restrict__ w,
                                                        const uint16_t* __restrict__ rope,
                                                        uint16_t* __restrict__ y, int ys, int ycol0, int B,
                                                        int H, uint32_t* __restrict__ amax) {
  using C = Bmm<K, N>;
  __shared__ __attribute__((aligned(16))) uint16_t lds[C::LDS / 2];
  uint16_t* wt = lds;                    // [64][WST]: wt[n][k] = w[h][k][n0 + n]
  const int h = blockIdx.x, tid = threadIdx.x;
  const int wv = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
  uint16_t* st = lds + 64 * C::WST + wv * 16 * C::OST;  // this wave's [16][OST] output tile

  if ((int)blockIdx.y == N / 64) {  // rope columns pass through
    for (int i = tid; i < B * 8; i += 256) {
      const int b = i >> 3, c = i & 7;
      *reinterpret_cast<uint4*>(y + ((int64_t)b * H + h) * ys + ycol0 + N + 8 * c) =
          *reinterpret_cast<const uint4*>(rope + ((int64_t)b * H + h) * 64 + 8 * c);
    }
    if (amax != nullptr && tid == 0) amax[blockIdx.y * H + h] = 0;
    return;
  }
  const int n0 = 64 * blockIdx.y;

  // weight slice, transposed: 8 columns per 16-byte load
  const uint16_t* wh = w + (int64_t)h * K * N + n0;
  for (int i = tid; i < K * 8; i += 256) {
    const int k = i >> 3, c = i & 7;
    const uint4 v = *reinterpret_cast<const uint4*>(wh + (int64_t)k * N + 8 * c);
    const uint32_t e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      wt[(8 * c + 2 * j) * C::WST + k] = (uint16_t)(e[j] & 0xFFFFu);
      wt[(8 * c + 2 * j + 1) * C::WST + k] = (uint16_t)(e[j] >> 16);
    }
  }
  __syncthreads();

  uint32_t mx = 0;
  for (int row0 = 0; row0 < B; row0 += 64) {
    const int ra = row0 + 16 * wv + l16;  // this lane's A row
    const uint16_t* xr = x + ((int64_t)min(ra, B - 1) * H + h) * xs + 8 * g;
    v4f acc[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[nt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int ks = 0; ks < K / 32; ++ks) {
      uint4 av = *reinterpret_cast<const uint4*>(xr + 32 * ks);
      if (ra >= B) av = make_uint4(0, 0, 0, 0);
      const v8bf a = __builtin_bit_cast(v8bf, av);
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const v8bf bb = *reinterpret_cast<const v8bf*>(wt + (16 * nt + l16) * C::WST + 32 * ks + 8 * g);
        acc[nt] = mfma16x32_bf16(a, bb, acc[nt]);
      }
    }
    // D[row 4g + r][col 16nt + l16] -> staging -> 16-byte row segments
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t bits = f32_to_bf16_bits(acc[nt][r]);
        st[(4 * g + r) * C::OST + 16 * nt + l16] = (uint16_t)bits;
        if (row0 + 16 * wv + 4 * g + r < B) mx = max(mx, bits & 0x7FFFu);
      }
    __syncthreads();  // staging written (every wave runs the same row loop)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int e = lane + 64 * j, r = e >> 3, c = e & 7;  // 16 rows x 8 segments
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

hipError_t launch_absorb_q(const uint16_t* q_nope, const uint16_t* q_rope, const uint16_t* w_uk, int batch,
                           int heads, uint16_t* q_out, hipStream_t stream) {
  hipLaunchKernelGGL((bmm_heads_kernel<128, 512>), dim3(heads, 512 / 64 + 1), dim3(256), 0, stream, q_nope, 128,
                     w_uk, q_rope, q_out, kQKDim, 0, batch, heads, nullptr);
  return hipGetLastError();
}

hipError_t launch_v_up_proj(const uint16_t* o, const uint16_t* w_uv, int batch, int heads, uint16_t* y,
                            uint32_t* amax_partials, hipStream_t stream) {
  hipLaunchKernelGGL((bmm_heads_kernel<512, 128>), dim3(heads, 128 / 64), dim3(256), 0, stream, o, kVDim, w_uv,
                     nullptr, y, 128, 0, batch, heads, amax_partials);
  return hipGetLastError();
}

}  // namespace mla
