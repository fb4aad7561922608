// Diagnostic kernels that pin the lane layouts and conversion semantics the
// decode kernels rely on (MFMA operand/accumulator layouts, fp8/fp4 converts,
// the LDS byte transpose).  One wave each; inputs are small row-major
// matrices, outputs are row-major f32 (or raw words) for a host-side check.
#include "mla_internal.hpp"

namespace mla {

__device__ __forceinline__ uint32_t gather4(const uint8_t* base, int stride, int k0, int col) {
  return (uint32_t)base[(k0 + 0) * stride + col] | ((uint32_t)base[(k0 + 1) * stride + col] << 8) |
         ((uint32_t)base[(k0 + 2) * stride + col] << 16) | ((uint32_t)base[(k0 + 3) * stride + col] << 24);
}

__global__ void selftest_kernel(int which, const uint8_t* __restrict__ in, uint8_t* __restrict__ out) {
  const int l = threadIdx.x;
  float* D = reinterpret_cast<float*>(out);
  if (which == 0 || which == 2) {  // 16x16x128: A fp8 [16][128] or fp4 [16][64B] + scales [16][4]
    v8i a, b;
    int sc = 127;
    const uint8_t* B;
    if (which == 0) {
      const uint8_t* A = in;
      B = in + 2048;
      for (int i = 0; i < 8; ++i) a[i] = *reinterpret_cast<const int*>(A + (l % 16) * 128 + 32 * (l / 16) + 4 * i);
    } else {
      const uint8_t* A = in;
      const uint8_t* As = in + 1024;
      B = in + 1024 + 64;
      for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const int*>(A + (l % 16) * 64 + 16 * (l / 16) + 4 * i);
      for (int i = 4; i < 8; ++i) a[i] = 0;
      sc = As[(l % 16) * 4 + (l / 16)];
    }
    if (which == 0) {
      for (int i = 0; i < 8; ++i) b[i] = (int)gather4(B, 16, 32 * (l / 16) + 4 * i, l % 16);
    } else {  // fp8 partner order of the fp4 operand: byte j of group g <-> K = 16g + (j&15) + 64(j>>4)
      for (int i = 0; i < 8; ++i) {
        uint32_t wd = 0;
        for (int bb = 0; bb < 4; ++bb) {
          const int j = 4 * i + bb, k = 16 * (l / 16) + (j & 15) + 64 * (j >> 4);
          wd |= (uint32_t)B[k * 16 + (l % 16)] << (8 * bb);
        }
        b[i] = (int)wd;
      }
    }
    v4f c = v4f{0.f, 0.f, 0.f, 0.f};
    c = which == 0 ? mfma16_f8(a, b, c) : mfma16_f4f8(a, sc, b, c);
    for (int r = 0; r < 4; ++r) D[(4 * (l / 16) + r) * 16 + (l % 16)] = c[r];
  } else if (which == 1 || which == 3) {  // 32x32x64: A fp8 [32][64] or fp4 [32][32B] + scales [32][2]
    v8i a, b;
    int sc = 127;
    const uint8_t* B;
    if (which == 1) {
      const uint8_t* A = in;
      B = in + 2048;
      for (int i = 0; i < 8; ++i) a[i] = *reinterpret_cast<const int*>(A + (l % 32) * 64 + 32 * (l / 32) + 4 * i);
    } else {
      const uint8_t* A = in;
      const uint8_t* As = in + 1024;
      B = in + 1024 + 64;
      for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const int*>(A + (l % 32) * 32 + 16 * (l / 32) + 4 * i);
      for (int i = 4; i < 8; ++i) a[i] = 0;
      sc = As[(l % 32) * 2 + (l / 32)];
    }
    if (which == 1) {
      for (int i = 0; i < 8; ++i) b[i] = (int)gather4(B, 32, 32 * (l / 32) + 4 * i, l % 32);
    } else {  // fp8 partner order of the fp4 operand: byte j of group g <-> K = 16g + (j&15) + 32(j>>4)
      for (int i = 0; i < 8; ++i) {
        uint32_t wd = 0;
        for (int bb = 0; bb < 4; ++bb) {
          const int j = 4 * i + bb, k = 16 * (l / 32) + (j & 15) + 32 * (j >> 4);
          wd |= (uint32_t)B[k * 32 + (l % 32)] << (8 * bb);
        }
        b[i] = (int)wd;
      }
    }
    v16f c = v16f{};
    c = which == 1 ? mfma32_f8(a, b, c) : mfma32_f4f8(a, sc, b, c);
    for (int r = 0; r < 16; ++r) D[(8 * (r / 4) + 4 * (l / 32) + (r % 4)) * 32 + (l % 32)] = c[r];
  } else if (which == 15 || which == 16) {  // 16x16x128 fp8 with e8m0 scales on B (15) or A (16)
    const uint8_t* A = in;
    const uint8_t* B = in + 2048;
    const uint8_t* Sc = in + 4096;  // [4 K blocks][16 cols (15) / rows (16)]
    v8i a, b;
    for (int i = 0; i < 8; ++i) a[i] = *reinterpret_cast<const int*>(A + (l % 16) * 128 + 32 * (l / 16) + 4 * i);
    for (int i = 0; i < 8; ++i) b[i] = (int)gather4(B, 16, 32 * (l / 16) + 4 * i, l % 16);
    const int sc = Sc[(l / 16) * 16 + (l % 16)];
    v4f c = v4f{0.f, 0.f, 0.f, 0.f};
    if (which == 15) c = mfma16_f8_bscale(a, b, sc, c);
    else c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, sc, 0, 127);
    for (int r = 0; r < 4; ++r) D[(4 * (l / 16) + r) * 16 + (l % 16)] = c[r];
  } else if (which == 19) {  // 32x32x64 fp8 with e8m0 scales on B: A [32][64], B [64][32], Sc [2][32]
    const uint8_t* A = in;
    const uint8_t* B = in + 2048;
    const uint8_t* Sc = in + 4096;
    v8i a, b;
    for (int i = 0; i < 8; ++i) a[i] = *reinterpret_cast<const int*>(A + (l % 32) * 64 + 32 * (l / 32) + 4 * i);
    for (int i = 0; i < 8; ++i) b[i] = (int)gather4(B, 32, 32 * (l / 32) + 4 * i, l % 32);
    v16f c = mfma32_f8_bscale(a, b, Sc[(l / 32) * 32 + (l % 32)], v16f{});
    for (int r = 0; r < 16; ++r) D[(8 * (r / 4) + 4 * (l / 32) + (r % 4)) * 32 + (l % 32)] = c[r];
  } else if (which == 4) {  // 16x16x32 fp8: A [16][32], B [32][16]
    const uint8_t* A = in;
    const uint8_t* B = in + 512;
    long a = *reinterpret_cast<const long*>(A + (l % 16) * 32 + 8 * (l / 16));
    long b = (long)gather4(B, 16, 8 * (l / 16), l % 16) | ((long)gather4(B, 16, 8 * (l / 16) + 4, l % 16) << 32);
    v4f c = mfma16x32_f8(a, b, v4f{0.f, 0.f, 0.f, 0.f});
    for (int r = 0; r < 4; ++r) D[(4 * (l / 16) + r) * 16 + (l % 16)] = c[r];
  } else if (which == 5) {  // 16x16x32 bf16: A [16][32] bf16, B [32][16] bf16
    const uint16_t* A = reinterpret_cast<const uint16_t*>(in);
    const uint16_t* B = reinterpret_cast<const uint16_t*>(in + 1024);
    v8bf a, b;
    for (int i = 0; i < 8; ++i) {
      a[i] = __builtin_bit_cast(__bf16, A[(l % 16) * 32 + 8 * (l / 16) + i]);
      b[i] = __builtin_bit_cast(__bf16, B[(8 * (l / 16) + i) * 16 + (l % 16)]);
    }
    v4f c = mfma16x32_bf16(a, b, v4f{0.f, 0.f, 0.f, 0.f});
    for (int r = 0; r < 4; ++r) D[(4 * (l / 16) + r) * 16 + (l % 16)] = c[r];
  } else if (which == 6) {  // pack4_fp8: 256 floats -> 256 bytes
    const float* x = reinterpret_cast<const float*>(in);
    reinterpret_cast<uint32_t*>(out)[l] = pack4_fp8(x[4 * l], x[4 * l + 1], x[4 * l + 2], x[4 * l + 3]);
  } else if (which == 7) {  // fp4 byte -> bf16 pair with scale: 64 words + 64 f32 scales -> 256 words
    const uint32_t word = reinterpret_cast<const uint32_t*>(in)[l];
    const float sc = reinterpret_cast<const float*>(in + 256)[l];
    uint32_t* o = reinterpret_cast<uint32_t*>(out);
    o[4 * l + 0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, sc, 0));
    o[4 * l + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, sc, 1));
    o[4 * l + 2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, sc, 2));
    o[4 * l + 3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, sc, 3));
  } else if (which == 8) {  // 4x4 byte transpose: 64 x 4 words
    const uint32_t* x = reinterpret_cast<const uint32_t*>(in) + 4 * l;
    uint32_t y[4];
    transpose4x4_bytes(x[0], x[1], x[2], x[3], y);
    for (int e = 0; e < 4; ++e) reinterpret_cast<uint32_t*>(out)[4 * l + e] = y[e];
  } else if (which == 9) {  // software f32 -> e4m3fn: 256 floats -> 256 bytes
    const float* x = reinterpret_cast<const float*>(in);
    for (int i = 0; i < 4; ++i) out[4 * l + i] = (uint8_t)f32_to_e4m3fn(x[4 * l + i]);
  } else if (which == 20) {  // hardware f32 pair -> e2m1 byte: 4096 floats + f32 scale -> 4096 bytes
    // pair i goes to byte i % 4 of a word that starts as 0xA5A5A5A5; out[i] =
    // that byte, out[2048 + i] = 1 if the other three bytes were kept
    const float* x = reinterpret_cast<const float*>(in);
    const float sc = x[4096];
    for (int i = l; i < 2048; i += 64) {
      const uint32_t old = 0xA5A5A5A5u;
      uint32_t r;
      switch (i & 3) {
        case 0: r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(old, x[2 * i], x[2 * i + 1], sc, 0); break;
        case 1: r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(old, x[2 * i], x[2 * i + 1], sc, 1); break;
        case 2: r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(old, x[2 * i], x[2 * i + 1], sc, 2); break;
        default: r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(old, x[2 * i], x[2 * i + 1], sc, 3); break;
      }
      const int sh = 8 * (i & 3);
      out[i] = (uint8_t)((r >> sh) & 0xFFu);
      out[2048 + i] = (uint8_t)(((r | (0xFFu << sh)) == (old | (0xFFu << sh))) ? 1 : 0);
    }
  } else if (which == 10) {  // hardware e4m3fn -> f32: 64 words -> 256 floats
    const int word = reinterpret_cast<const int*>(in)[l];
    const v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8(word, false);
    const v2f hi = __builtin_amdgcn_cvt_pk_f32_fp8(word, true);
    float* o = reinterpret_cast<float*>(out);
    o[4 * l + 0] = lo[0];
    o[4 * l + 1] = lo[1];
    o[4 * l + 2] = hi[0];
    o[4 * l + 3] = hi[1];
  }
}

// One-hot probe of the fp4 operand: for each of the 128 (16x16x128) or 64
// (32x32x64) fp4 element positions p of row 0 (lane group g = p / 32, element
// e = p % 32 at byte e/2, low nibble for even e) set that element to 1.0 and
// multiply by an fp8 B whose column n holds bit n of the logical K index
// (B lanes built with the fp8 layout).  out[p*8 + n] = D[0][n].
__global__ void fp4_probe_kernel(int big, float* __restrict__ out) {
  const int l = threadIdx.x;
  const int M = big ? 32 : 16;
  const int npos = big ? 64 : 128;
  for (int pidx = 0; pidx < npos; ++pidx) {
    const int g = pidx / 32, e = pidx % 32;
    v8i a = v8i{0, 0, 0, 0, 0, 0, 0, 0};
    if (l % M == 0 && l / M == g) {
      const uint32_t code = 2u;  // e2m1 1.0
      a[(e / 2) / 4] = (int)(code << (8 * ((e / 2) % 4) + 4 * (e % 2)));
    }
    v8i bv;
    for (int i = 0; i < 8; ++i) {
      uint32_t w = 0;
      for (int bb = 0; bb < 4; ++bb) {
        const int k = 32 * (l / M) + 4 * i + bb;  // logical K under the fp8 layout
        const int n = l % M;
        const uint32_t one = 0x38u;  // e4m3 1.0
        w |= (((k >> n) & 1) && n < 8 ? one : 0u) << (8 * bb);
      }
      bv[i] = (int)w;
    }
    if (!big) {
      v4f c = mfma16_f4f8(a, 127, bv, v4f{0.f, 0.f, 0.f, 0.f});
      if (l < 8) out[pidx * 8 + l] = c[0];
    } else {
      v16f c = mfma32_f4f8(a, 127, bv, v16f{});
      if (l < 8) out[pidx * 8 + l] = c[0];
    }
  }
}

// LDS-DMA placement (13) and ds_read_b64_tr_b8 (14).  in: 1024 source bytes.
// 13: lane l DMAs src[16*((7l) % 64) ..+16] to LDS offsets 0, 65536+1024 and
//     131072+4096; out = the three 1 KiB LDS windows.
// 14: LDS[i] = in[i % 1024] for i < 4096; lane l tr-reads at 8l (pattern A) and
//     at 64(l % 8) + 8(l / 8) (pattern B); out = 64 x 8 bytes per pattern.
// 21: as 14 with ds_read_b64_tr_b4.
__global__ void lds_probe_kernel(int which, const uint8_t* __restrict__ src, uint8_t* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[136192];
  const int l = threadIdx.x;
  const uint32_t base = (uint32_t)(uintptr_t)lds;
  if (which == 13) {
    const uint32_t offs[3] = {0u, 65536u + 1024u, 131072u + 4096u};
    for (int k = 0; k < 3; ++k) dma16_to_lds(src + ((l * 7) % 64) * 16, base + offs[k]);
    wait_vmcnt<0>();
    __syncthreads();
    for (int k = 0; k < 3; ++k)
      for (int i = 0; i < 16; ++i) out[k * 1024 + l * 16 + i] = lds[offs[k] + l * 16 + i];
  } else if (which == 17 || which == 18) {
    // 17: lane l DMAs the 2 bytes at src + 2l, 18: the byte at src + l, to M0 = 0;
    // out = LDS bytes 0 .. 511 (pre-filled with 0xEE)
    for (int i = l; i < 512; i += 64) lds[i] = 0xEE;
    __syncthreads();
    if (which == 17) dma2_to_lds(src + 2 * l, base);
    else dma1_to_lds(src + l, base);
    wait_vmcnt<0>();
    __syncthreads();
    for (int i = l; i < 512; i += 64) out[i] = lds[i];
  } else {
    for (int i = l; i < 4096; i += 64) lds[i] = src[i % 1024];
    __syncthreads();
    const v2i a = which == 21 ? lds_read_tr4(base + 8 * l) : lds_read_tr8(base + 8 * l);
    const v2i b = which == 21 ? lds_read_tr4(base + 64 * (l % 8) + 8 * (l / 8))
                              : lds_read_tr8(base + 64 * (l % 8) + 8 * (l / 8));
    reinterpret_cast<v2i*>(out)[l] = a;
    reinterpret_cast<v2i*>(out)[64 + l] = b;
  }
}

hipError_t launch_selftest(int which, const void* in, void* out, hipStream_t stream) {
  if (which == 13 || which == 14 || which == 17 || which == 18 || which == 21) {
    hipLaunchKernelGGL(lds_probe_kernel, dim3(1), dim3(64), 0, stream, which,
                       static_cast<const uint8_t*>(in), static_cast<uint8_t*>(out));
    return hipGetLastError();
  }
  if (which == 11 || which == 12) {
    hipLaunchKernelGGL(fp4_probe_kernel, dim3(1), dim3(64), 0, stream, which == 12 ? 1 : 0,
                       static_cast<float*>(out));
    return hipGetLastError();
  }
  if (which < 0 || (which > 10 && which != 15 && which != 16 && which != 19 && which != 20))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(selftest_kernel, dim3(1), dim3(64), 0, stream, which,
                     static_cast<const uint8_t*>(in), static_cast<uint8_t*>(out));
  return hipGetLastError();
}

}  // namespace mla
