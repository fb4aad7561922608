// Shared device helpers and host-visible layout constants for the gfx950 MLA
// decode library.  Everything here is CDNA4-specific: 64-lane waves, the
// gfx950 f8f6f4 MFMA family and the OCP fp8/fp4 formats gfx950 uses natively.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mla {

constexpr int kQKDim = 576;       // 512 latent + 64 rope
constexpr int kVDim = 512;        // latent part, used as V
constexpr int kFp4RowBytes = 288; // 576 e2m1 values, two per byte
constexpr int kMxBlocks = 18;     // 576 / 32 e8m0 scales per row
constexpr int kScWin = 5;         // dwords that hold a row's 18 e8m0 bytes (LDS-DMA)
constexpr int kTile = 64;         // tokens staged per LDS tile

// ---- plan layout (int32 words inside the workspace) -------------------------
// header[0] = number of work items, [1] = chunk, [2] = total tokens, [3] = batch
// items: int4 {batch, token_begin, token_end, partial_slot (-1 = final)}
// batch_info: int2 {first item, item count}
constexpr int kPlanHeader = 16;

// ---- kernel parameter block --------------------------------------------------
struct DecodeParams {
  const uint8_t* q_fp8;      // [B, H, 576]
  const float* q_scale;      // [1]
  const uint8_t* k_cache;    // fp8 rows or packed fp4 rows
  int64_t k_row_stride;      // bytes
  const uint8_t* k_scales;   // e8m0 rows (fp4 K)
  int64_t k_scale_stride;    // bytes
  const uint8_t* v_cache;    // fp8 rows (fp8 V from a separate cache)
  int64_t v_row_stride;      // bytes
  const float* kv_scale;     // [1] fp8 per-tensor scale (fp8 K and/or V)
  const int32_t* kv_indptr;  // [B+1]
  const int32_t* kv_indices; // [T] or nullptr (identity)
  const int32_t* plan;       // plan block (see above)
  uint16_t* part_o;          // [max_items, H, 512] bf16 (normalized split outputs)
  float* part_lse;           // [max_items, H]  (log2 domain)
  uint16_t* out;             // [B, H, 512] bf16
  float* lse_out;            // [B, H] natural-log lse, or nullptr
  // Q as bf16 with the per-tensor amax partials (the H = 16 kernel quantizes
  // its sequence's Q itself); q_fp8 / q_scale are used when q_bf16 is null
  const uint16_t* q_bf16;    // [B, H, 576] or nullptr
  const uint32_t* q_partials;
  int q_nparts;
  float sm_scale;
  int batch;
  int num_heads;
  int max_items;
  // 16 heads: q_per_row = bf16 Q quantized per head row in the kernel (no
  // tensor-wide scale); plan_here = the kernel plans its own work (batch <= 256
  // query rows, plan_qlen per sequence) with the planner's target, chunk floor
  // and split cap, and its work-group 0 writes the rows' piece counts and the
  // header the combine reads (plan then points at writable workspace)
  int q_per_row;
  int plan_here;
  int plan_qlen;
  int plan_target;
  int plan_min_chunk;
  int plan_max_splits;
};

// ---- vector types ------------------------------------------------------------
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef short s16x2 __attribute__((ext_vector_type(2)));

// 16-byte streaming load (read once; do not keep in cache)
__device__ __forceinline__ uint4 ldg16_nt(const void* p) {
  u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// ---- bf16 / fp8 scalar conversions (bit exact, no fast math) ----------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// Round-to-nearest-even f32 -> bf16 bits for finite inputs.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

// two floats -> bf16 pair (RNE, v_cvt_pk_bf16_f32), a in the low half
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 v2bf_t __attribute__((ext_vector_type(2)));
  const v2bf_t r = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, r);
}

// Round-to-nearest-even f32 -> OCP e4m3fn code for |f| <= 448.
__device__ __forceinline__ uint32_t f32_to_e4m3fn(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t sign = (u >> 24) & 0x80u;
  u &= 0x7FFFFFFFu;
  float a = __uint_as_float(u);
  uint32_t code;
  if (a < 0.015625f) {  // below 2^-6: subnormal grid of 2^-9, k = 8 is 2^-6
    code = (uint32_t)__builtin_rintf(a * 512.0f);
  } else {
    uint32_t odd = (u >> 20) & 1u;
    u += 0x7FFFFu + odd;
    code = (u >> 20) - (120u << 3);
  }
  return sign | code;
}

// bf16 |x|max bits -> f32 scale exactly as torch evaluates
// competitor_submissions/mi355x_reference/reference.py:77-78
__device__ __forceinline__ float fp8_scale_from_amax(uint32_t amax_bits) {
  amax_bits = amax_bits > 0x2B8Du ? amax_bits : 0x2B8Du;  // clamp(min=1e-12) in bf16
  const float a = bf16_bits_to_f32(amax_bits);
  return bf16_bits_to_f32(f32_to_bf16_bits(a / 448.0f));
}

// Per-tensor fp8 quantizer state: the scale and, when it is safe, its
// reciprocal (r = 0 selects the plain division for every element).
struct Fp8Quant {
  float s;
  float r;
};
__device__ __forceinline__ Fp8Quant make_fp8_quant(float s) {
  const float a = fabsf(s);
  const bool ok = a >= 0x1p-125f && a <= 0x1p125f;  // 1/s stays a normal f32
  return Fp8Quant{s, ok ? 1.0f / s : 0.0f};
}

// clamp(bf16(x / s), -448, 448) of reference.py:79-80, exact.  x * r (r the
// correctly rounded 1/s) is within 3 f32 ulps of x / s's correctly rounded
// quotient (two roundings of at most half an ulp each on top of the
// reciprocal's), so both round to the same bf16 unless x * r lies within 3
// ulps of a bf16 tie (low half 0x8000); only there is the division computed.
__device__ __forceinline__ float quant_y(uint32_t h, Fp8Quant q) {
  const float x = bf16_bits_to_f32(h);
  float d = x * q.r;
  if (q.r == 0.0f || (__float_as_uint(d) & 0xFFFFu) - 0x7FFDu <= 6u) d = x / q.s;
  const float y = bf16_bits_to_f32(f32_to_bf16_bits(d));
  return fminf(fmaxf(y, -448.0f), 448.0f);
}
// y = e4m3fn(clamp(bf16(x / s), -448, 448)), reference.py:79-80
__device__ __forceinline__ uint32_t quant_one(uint32_t h, Fp8Quant q) { return f32_to_e4m3fn(quant_y(h, q)); }

// ---- wave helpers ------------------------------------------------------------
__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

// ---- MFMA wrappers (gfx950) --------------------------------------------------
// D = A * B + C, A: 16 x 128 fp8, B: 128 x 16 fp8 (lane l: row/col l%16,
// K elements 32*(l/16) .. +31), D: lane l holds column l%16, rows 4*(l/16)+r.
__device__ __forceinline__ v4f mfma16_f8(v8i a, v8i b, v4f c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}
// fp8 x fp8 with an e8m0 scale on B (one per lane: its column, 32 K values)
__device__ __forceinline__ v4f mfma16_f8_bscale(v8i a, v8i b, int b_scale, v4f c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, b_scale);
}
// Same shape, A = e2m1 (first four dwords) with an e8m0 scale per lane
// (one per 32 K values), B = fp8 with unit scale.
__device__ __forceinline__ v4f mfma16_f4f8(v8i a, int a_scale, v8i b, v4f c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 4, 0, 0, a_scale, 0, 127);
}
// D = A * B + C, A: 32 x 64 fp8, B: 64 x 32 fp8 (lane l: row/col l%32, K
// elements 32*(l/32) .. +31); D: lane l holds column l%32, rows
// 8*(r/4) + 4*(l/32) + r%4 for r = 0..15.
__device__ __forceinline__ v16f mfma32_f8(v8i a, v8i b, v16f c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}
// fp8 x fp8 with an e8m0 scale on B (one per lane: its column, 32 K values)
__device__ __forceinline__ v16f mfma32_f8_bscale(v8i a, v8i b, int b_scale, v16f c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, b_scale);
}
__device__ __forceinline__ v16f mfma32_f4f8(v8i a, int a_scale, v8i b, v16f c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 4, 0, 0, a_scale, 0, 127);
}
// 16x16x32 fp8 (K = 32): lane l: row/col l%16, K elements 8*(l/16) .. +7.
__device__ __forceinline__ v4f mfma16x32_f8(long a, long b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(a, b, c, 0, 0, 0);
}
// 16x16x32 bf16 (K = 32): lane l: row/col l%16, K elements 8*(l/16) .. +7.
__device__ __forceinline__ v4f mfma16x32_bf16(v8bf a, v8bf b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Pack four floats (each in [0, 448]) into four e4m3fn bytes, element i in byte i.
__device__ __forceinline__ uint32_t pack4_fp8(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}
// the same written over `old` (whose bytes all end replaced): the converts
// can then reuse old's register instead of a zeroed copy
__device__ __forceinline__ uint32_t pack4_fp8_over(uint32_t old, float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, (int)old, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}
// eight bf16 (one uint4) -> eight e4m3fn codes of the per-tensor quantizer; the
// hardware convert rounds to nearest even like the reference cast, and after
// the clamp to +-448 no input can overflow it
// Here x * r needs no near-tie test: x and s are both bf16, so x / s is a
// ratio of 8-bit significands times a power of two, never a bf16 tie (a tie
// would make an odd number equal to an even one) and at least 2^-17 of itself
// away from one (|A - ms T| >= 1 for the integers A = mx 2^p, ms < 2^8 and the
// tie's odd numerator T < 2^9), while x * r is within 2^-23 of x / s; and
// results beyond 448 clamp to 448 either way.  The division remains for r = 0
// (s infinite or NaN).
__device__ __forceinline__ uint2 quant8_fp8(uint4 v, Fp8Quant q) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  auto x = [&](int e) { return bf16_bits_to_f32(e & 1 ? w[e >> 1] >> 16 : w[e >> 1] & 0xFFFFu); };
  float y[8];
  if (q.r != 0.0f) {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      y[e] = fminf(fmaxf(bf16_bits_to_f32(f32_to_bf16_bits(x(e) * q.r)), -448.0f), 448.0f);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      y[e] = fminf(fmaxf(bf16_bits_to_f32(f32_to_bf16_bits(x(e) / q.s)), -448.0f), 448.0f);
  }
  return make_uint2(pack4_fp8(y[0], y[1], y[2], y[3]), pack4_fp8(y[4], y[5], y[6], y[7]));
}

// ---- LDS DMA (global_load_lds) and explicit waits --------------------------
// The gfx950 LDS-DMA writes lane l's 16 (4) bytes to LDS at M0 + 16 l (4 l).
// It is issued through inline asm so the compiler does not add conservative
// vmcnt(0) waits before LDS reads and barriers: completion is tracked with
// explicit wait_vmcnt<N>() calls, N = vector-memory ops issued after the one
// that must have landed (vmcnt retires in order).
// M0 is a reserved register the compiler assumes unchanged across inline asm,
// so each DMA saves it and puts it back; an SALU write of M0 needs one wait
// state before an LDS-DMA reads it, given here by an SALU no-op (SALU issue
// costs the wave next to nothing, an s_nop a full issue slot).
// The LDS offset is wave-uniform at every call site; readfirstlane states that
// for the compiler, whose divergence analysis can otherwise leave it in a VGPR,
// which the "s" constraint cannot take.
#define MLA_LDS_DMA(INSN)                                                                          \
  uint32_t saved;                                                                                  \
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_mov_b32 %0, %0\n\t" INSN "\n\t"        \
               "s_mov_b32 m0, %0"                                                                  \
               : "=&s"(saved)                                                                      \
               : "s"(__builtin_amdgcn_readfirstlane(lds_off)), "v"(g)                             \
               : "memory")
__device__ __forceinline__ void dma16_to_lds(const void* g, uint32_t lds_off) {
  MLA_LDS_DMA("global_load_lds_dwordx4 %2, off");
}
// The same with the non-temporal hint (nt), for the cache rows, which are read
// once.  Measured: with the default policy a decode that follows a large write
// (the timing protocols' cache flush, or any producer of that size) runs 15-35 %
// longer than after another decode, as if its reads paid for writing back what
// the write left in the caches; with nt it runs as fast as after a decode.
// Scale rows (7 tokens per 128-B line) and slot indices keep the default
// policy and the line reuse it gives.
__device__ __forceinline__ void dma16_to_lds_nt(const void* g, uint32_t lds_off) {
  MLA_LDS_DMA("global_load_lds_dwordx4 %2, off nt");
}
__device__ __forceinline__ void dma4_to_lds(const void* g, uint32_t lds_off) { MLA_LDS_DMA("global_load_lds_dword %2, off"); }
// two bytes per lane (2-byte aligned source): lane l's bytes land,
// zero-extended, in the dword at M0 + 4 l
__device__ __forceinline__ void dma2_to_lds(const void* g, uint32_t lds_off) { MLA_LDS_DMA("global_load_lds_ushort %2, off"); }
// one byte per lane: lane l's byte lands, zero-extended, in the dword at M0 + 4 l
__device__ __forceinline__ void dma1_to_lds(const void* g, uint32_t lds_off) { MLA_LDS_DMA("global_load_lds_ubyte %2, off"); }
#undef MLA_LDS_DMA
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Work-group barrier for LDS only (no global-memory fence, so outstanding
// DMA/prefetch loads are not drained).
// Wave-wide inclusive prefix sum in lane order: a Hillis-Steele scan inside
// each 16-lane row by DPP row shifts (lanes shifted in from outside the row read
// 0), then the row totals carried forward by the gfx9 row broadcasts (lane 15
// of rows 0 and 2 into rows 1 and 3, lane 31 into rows 2 and 3).  Six VALU ops,
// no LDS round trips.
__device__ __forceinline__ int wave_incl_sum(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);   // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);   // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);   // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);   // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return x;
}
// the same pattern with max, for non-negative values; lane 63 holds the wave max
__device__ __forceinline__ int wave_incl_max(int x) {
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false));
  return x;
}
__device__ __forceinline__ int wave_sum(int x) { return __builtin_amdgcn_readlane(wave_incl_sum(x), 63); }
__device__ __forceinline__ int wave_max(int x) { return __builtin_amdgcn_readlane(wave_incl_max(x), 63); }

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Work-group g of a launch runs on XCD g % 8: the dispatcher deals
// work-groups out round-robin over the 8 XCDs, each with its own L2.  Plan
// items of one query row are consecutive and read the same Q, so items go to
// XCDs M at a time: in each block of 8M work-groups, those of XCD x (g = x,
// x + 8, ..) take items xM .. xM + M - 1.  A partial last block keeps the
// identity, so this is a bijection on [0, G); a block of 8M work-groups that
// divides the CU count keeps every item in the dispatch round it had.
template <int M>
__device__ __forceinline__ int xcd_item(int g, int G) {
  static_assert(M > 0 && (M & (M - 1)) == 0, "M is a power of two");
  const int base = g & ~(8 * M - 1);
  if (base + 8 * M > G) return g;
  const int r = g - base;
  return base + (r & 7) * M + (r >> 3);
}

// ds_read_b64_tr_b8: within each 16-lane group, result lane j gets byte (j & 7)
// of the 8-byte reads of lanes 2m + (j >> 3), m = 0..7, in that order.
typedef int v2i __attribute__((ext_vector_type(2)));
__device__ __forceinline__ v2i lds_read_tr8(uint32_t lds_off) {
  typedef __attribute__((address_space(3))) v2i lds_v2i;
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(uintptr_t)lds_off);
}
// ds_read_b64_tr_b16: within each 16-lane group, result lane j gets element
// (j & 3) of the four 16-bit elements read by lane 4i + (j >> 2) as its element
// i, i = 0..3 (a 16 x 4 -> 4 x 16 element transpose).
typedef short v4s16 __attribute__((ext_vector_type(4)));
typedef short v8s16 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ v4s16 lds_read_tr16(uint32_t lds_off) {
  typedef __attribute__((address_space(3))) v4s16 lds_v4s16;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s16*)(uintptr_t)lds_off);
}
// ds_read_b64_tr_b4: within each 16-lane group, result lane j gets nibble j of
// the 8-byte read of lane m as its nibble m, m = 0..15 (a 16 x 16 nibble
// transpose)
__device__ __forceinline__ v2i lds_read_tr4(uint32_t lds_off) {
  typedef __attribute__((address_space(3))) v2i lds_v2i;
  return __builtin_amdgcn_ds_read_tr4_b64_v2i32((lds_v2i*)(uintptr_t)lds_off);
}

// Byte-transpose of a 4x4 byte block: y[e] byte r = x[r] byte e.
__device__ __forceinline__ void transpose4x4_bytes(uint32_t x0, uint32_t x1, uint32_t x2,
                                                   uint32_t x3, uint32_t y[4]) {
  // pair rows (0,1) and (2,3) byte-interleaved, then merge halves
  uint32_t t01lo = __builtin_amdgcn_perm(x1, x0, 0x05010400u);  // x0b0 x1b0 x0b1 x1b1
  uint32_t t01hi = __builtin_amdgcn_perm(x1, x0, 0x07030602u);  // x0b2 x1b2 x0b3 x1b3
  uint32_t t23lo = __builtin_amdgcn_perm(x3, x2, 0x05010400u);
  uint32_t t23hi = __builtin_amdgcn_perm(x3, x2, 0x07030602u);
  y[0] = __builtin_amdgcn_perm(t23lo, t01lo, 0x05040100u);  // t01lo b0 b1, t23lo b0 b1
  y[1] = __builtin_amdgcn_perm(t23lo, t01lo, 0x07060302u);
  y[2] = __builtin_amdgcn_perm(t23hi, t01hi, 0x05040100u);
  y[3] = __builtin_amdgcn_perm(t23hi, t01hi, 0x07060302u);
}

}  // namespace mla
