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
    for (int i = 0; i < 8; ++i) b[i] = (int)gather4(B, 16, 32 * (l / 16) + 4 * i, l % 16);
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
    for (int i = 0; i < 8; ++i) b[i] = (int)gather4(B, 32, 32 * (l / 32) + 4 * i, l % 32);
    v16f c = v16f{};
    c = which == 1 ? mfma32_f8(a, b, c) : mfma32_f4f8(a, sc, b, c);
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
  }
}

hipError_t launch_selftest(int which, const void* in, void* out, hipStream_t stream) {
  if (which < 0 || which > 9) return hipErrorInvalidValue;
  hipLaunchKernelGGL(selftest_kernel, dim3(1), dim3(64), 0, stream, which,
                     static_cast<const uint8_t*>(in), static_cast<uint8_t*>(out));
  return hipGetLastError();
}

}  // namespace mla
