// Split-KV MLA absorbed decode for gfx950 and the log-sum-exp split combine.
//
// One work-group (4 waves) runs one work item {batch, token range, slot} from
// the on-device plan.  Per 64-token tile the group gathers the cache rows named
// by kv_indices (page size 1) from HBM with 16-byte loads into registers one
// tile ahead, then writes them to LDS twice: row-major (the QK operand, one
// token per MFMA row) and transposed (the PV operand, one latent dim per MFMA
// row).  Both products run on MFMA:
//   scores  S^T = K . Q^T   K = A operand from LDS, Q = B operand in registers
//   output  O^T = V^T . P^T V^T = A operand from LDS, P = B operand
// so every lane's accumulators belong to a single head and the online-softmax
// rescale is a per-lane scalar.  Heads: H = 16 runs the four waves on four
// 16-token slices of the tile and splits the 512 output dims four ways (the
// tile max and P go through LDS); H = 128 gives each wave 32 heads of its own
// (32x32x64 MFMAs, softmax wave-local, P stays in registers).
//
// Numerics: scores are accumulated in f32 from the fp8/fp4 operands and scaled
// by q_scale * k_scale * sm_scale * log2(e); the softmax uses exp2.  P enters
// the PV product as fp8 e4m3 (x256 to stay clear of the subnormal range) or as
// bf16 when V comes from the MXFP4 cache.  The row sum uses the f32 P.
//
// Behavioural reference: mixed-mla/asm_dumps/aiter_mla.py:149-470 (interface),
// mixed-mla/submission.py:122-250 (split-K online softmax), V5
// mixed-mla/versions/hip_mxfp4_v5/submission.py:214-714 (split + reduce).
#include <type_traits>

#include "mla_internal.hpp"

namespace mla {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kPScale = 256.0f;  // fp8 P = p * 256
constexpr float kRebase = 96.0f;   // H128: max log2 distance of a tile max above the fixed reference

__device__ __forceinline__ int kv_slot(const int32_t* __restrict__ idx, int pos) {
  return idx != nullptr ? idx[pos] : pos;
}

__device__ __forceinline__ v8i ld_v8(const uint8_t* p) {
  uint4 a = *reinterpret_cast<const uint4*>(p);
  uint4 b = *reinterpret_cast<const uint4*>(p + 16);
  v8i r;
  r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w;
  r[4] = b.x; r[5] = b.y; r[6] = b.z; r[7] = b.w;
  return r;
}
__device__ __forceinline__ v8i ld_v4_as_v8(const uint8_t* p) {
  uint4 a = *reinterpret_cast<const uint4*>(p);
  v8i r;
  r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w;
  r[4] = 0; r[5] = 0; r[6] = 0; r[7] = 0;
  return r;
}
__device__ __forceinline__ uint4 ldg16(const uint8_t* p) {
  return ldg16_nt(p);
}
__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }

// byte SEL of `word` holds two e2m1 values (low nibble first); returns them as a
// bf16 pair (low half = low nibble) multiplied by `scale`
template <int SEL>
__device__ __forceinline__ uint32_t cvt_fp4_byte(uint32_t word, float scale) {
  v2bf r = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, SEL);
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ float e8m0_to_f32(uint32_t e) {
  return e == 0 ? __uint_as_float(0x00400000u) : __uint_as_float(e << 23);
}

// ============================================================================
// Tile loader: one 64-token tile of cache rows gathered through kv_indices.
// Thread t serves token quad tq = t / QPT (tokens 4tq .. 4tq+3) and the 16-byte
// chunks ch = t % QPT + QPT*j of those four rows, so it needs four slot indices
// per tile; they are fetched one tile ahead of the rows.  Row loads never wait
// on each other: a token past the end of the item reads slot 0 and is zeroed
// when the registers are written to LDS (after the loads have landed).
// ============================================================================
template <int NT, int KF, int VF, bool IDX>
struct TileLoader {
  static constexpr int QPT = NT / 16;
  static constexpr int KCH = KF == 0 ? 36 : 18;
  static constexpr int KJ = (KCH + QPT - 1) / QPT;
  static constexpr int VJ = VF == 1 ? (32 + QPT - 1) / QPT : 1;
  static constexpr int SJ = KF == 1 ? (kMxBlocks + QPT - 1) / QPT : 1;

  int tq, lq;
  int sl_nxt[4];       // cache slots of the quad's tokens for the next tile to load
  int vmask;           // bit r set: token 4tq+r of the loaded tile is valid
  uint4 kr[KJ][4];
  uint4 vr[VJ][4];
  uint32_t sr[SJ][4];  // e8m0 of block lq + QPT*j for the quad's 4 tokens

  __device__ __forceinline__ void init(int tid) {
    tq = tid / QPT;
    lq = tid - tq * QPT;
  }
  // Slots of tokens pos0 + 4tq + r, r < 4.  Positions are clamped to last
  // (a valid position), so the loads are unconditional and their results are
  // only consumed when the rows are gathered, a tile later.
  __device__ __forceinline__ void load_idx(const DecodeParams& p, int pos0, int last, int (&sl)[4]) const {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int pos = min(pos0 + 4 * tq + r, last);
      if constexpr (IDX) sl[r] = p.kv_indices[pos];
      else sl[r] = pos;
    }
  }
  __device__ __forceinline__ void load_rows(const DecodeParams& p, const int (&sl)[4], int nval) {
    vmask = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) vmask |= (4 * tq + r < nval ? 1 : 0) << r;
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      const int ch = min(lq + QPT * j, KCH - 1);
#pragma unroll
      for (int r = 0; r < 4; ++r) kr[j][r] = ldg16(p.k_cache + (int64_t)sl[r] * p.k_row_stride + 16 * ch);
    }
    if constexpr (VF == 1) {
#pragma unroll
      for (int j = 0; j < VJ; ++j) {
        const int ch = min(lq + QPT * j, 31);
#pragma unroll
        for (int r = 0; r < 4; ++r) vr[j][r] = ldg16(p.v_cache + (int64_t)sl[r] * p.v_row_stride + 16 * ch);
      }
    }
    if constexpr (KF == 1) {
#pragma unroll
      for (int j = 0; j < SJ; ++j) {
        const int blk = min(lq + QPT * j, kMxBlocks - 1);
#pragma unroll
        for (int r = 0; r < 4; ++r) sr[j][r] = p.k_scales[(int64_t)sl[r] * p.k_scale_stride + blk];
      }
    }
  }
  __device__ __forceinline__ bool valid(int r) const { return (vmask >> r) & 1; }
  __device__ __forceinline__ uint4 kget(int j, int r) const { return valid(r) ? kr[j][r] : make_uint4(0, 0, 0, 0); }
  __device__ __forceinline__ uint4 vget(int j, int r) const { return valid(r) ? vr[j][r] : make_uint4(0, 0, 0, 0); }

  // row-major K tile (+ e8m0 scales for fp4 K)
  __device__ __forceinline__ void store_k(uint8_t* Klds, int kst, uint8_t* Slds) const {
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      const int ch = lq + QPT * j;
      if (ch < KCH) {
#pragma unroll
        for (int r = 0; r < 4; ++r) *reinterpret_cast<uint4*>(Klds + (4 * tq + r) * kst + 16 * ch) = kget(j, r);
      }
    }
    if constexpr (KF == 1) {
#pragma unroll
      for (int j = 0; j < SJ; ++j) {
        const int blk = lq + QPT * j;
        if (blk < kMxBlocks) {
#pragma unroll
          for (int r = 0; r < 4; ++r) Slds[(4 * tq + r) * 20 + blk] = valid(r) ? (uint8_t)sr[j][r] : (uint8_t)127;
        }
      }
    }
  }
  // fp8 V^T: for each latent dim of chunk ch, the quad's four bytes as one word
  template <class Off>
  __device__ __forceinline__ void store_vt_fp8(uint8_t* Vt, const uint4 (&x)[4], int ch, Off off) const {
    const uint32_t* x0 = reinterpret_cast<const uint32_t*>(&x[0]);
    const uint32_t* x1 = reinterpret_cast<const uint32_t*>(&x[1]);
    const uint32_t* x2 = reinterpret_cast<const uint32_t*>(&x[2]);
    const uint32_t* x3 = reinterpret_cast<const uint32_t*>(&x[3]);
#pragma unroll
    for (int wd = 0; wd < 4; ++wd) {
      uint32_t y[4];
      transpose4x4_bytes(x0[wd], x1[wd], x2[wd], x3[wd], y);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = 16 * ch + 4 * wd + e;
        *reinterpret_cast<uint32_t*>(Vt + off(d, tq)) = y[e];
      }
    }
  }
  template <class Off>
  __device__ __forceinline__ void store_v_fp8(uint8_t* Vt, Off off) const {
    if constexpr (VF == 0) {
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
        const int ch = lq + QPT * j;
        if (ch < 32) {
          uint4 x[4] = {kget(j, 0), kget(j, 1), kget(j, 2), kget(j, 3)};
          store_vt_fp8(Vt, x, ch, off);
        }
      }
    } else if constexpr (VF == 1) {
#pragma unroll
      for (int j = 0; j < VJ; ++j) {
        const int ch = lq + QPT * j;
        if (ch < 32) {
          uint4 x[4] = {vget(j, 0), vget(j, 1), vget(j, 2), vget(j, 3)};
          store_vt_fp8(Vt, x, ch, off);
        }
      }
    }
  }
};

// Two-term fp8 encoding of four non-negative values (< 448): hi = e4m3(x),
// lo = e4m3(x - hi).  hi + lo carries ~7 significant bits; both terms enter
// the same MFMA accumulator.
__device__ __forceinline__ void pack4_fp8_split(float a, float b, float c, float d, uint32_t& hi,
                                                uint32_t& lo) {
  hi = pack4_fp8(a, b, c, d);
  const v2f h01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, false);
  const v2f h23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, true);
  lo = pack4_fp8(a - h01[0], b - h01[1], c - h23[0], d - h23[1]);
}

// ============================================================================
// H = 16
//   KF: 0 = fp8 K rows (576 B), 1 = packed fp4 K rows (288 B) + e8m0 scales
//   VF: 0 = fp8 V = K rows, 1 = fp8 V from its own cache, 2 = fp4 V = K rows
// ============================================================================
template <int KF, int VF>
struct H16 {
  static constexpr int KROW = KF == 0 ? 576 : 288;
  static constexpr int KST = KROW + 16;               // LDS row stride (bank spread)
  static constexpr bool VB16 = VF == 2;               // V^T / P held as bf16
  static constexpr int VTST = VB16 ? 144 : 72;        // LDS bytes per latent-dim row of V^T
  static constexpr int PST = VB16 ? 144 : 72;
  static constexpr int NPLANE = VB16 ? 1 : 2;         // fp8 P: hi and lo planes
  static constexpr int OFF_K = 0;
  static constexpr int OFF_S = OFF_K + kTile * KST;
  static constexpr int OFF_VT = OFF_S + (KF == 1 ? kTile * 20 : 0);
  static constexpr int OFF_P = OFF_VT + kVDim * VTST;
  static constexpr int OFF_MAX = OFF_P + NPLANE * 16 * PST;
  static constexpr int OFF_L = OFF_MAX + 4 * 16 * 4;
  static constexpr int LDS = OFF_L + 4 * 16 * 4;
};

// fp8 V^T row of latent dim d holds 64 tokens in natural order as eight 8-byte
// chunks; chunk c is stored at c ^ ((d >> 4) & 7) to spread the transposed
// writes of 16 consecutive chunks over the banks.
__device__ __forceinline__ int vt16_quad_off(int d, int tq) {
  return d * 72 + 8 * ((tq >> 1) ^ ((d >> 4) & 7)) + 4 * (tq & 1);
}
__device__ __forceinline__ int vt16_read_off(int d, int chunk8) { return d * 72 + 8 * (chunk8 ^ ((d >> 4) & 7)); }

template <int KF, int VF, bool IDX>
__global__ __launch_bounds__(256, 1) void decode_h16_kernel(const DecodeParams p) {
  using C = H16<KF, VF>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[C::LDS];
  uint8_t* Klds = smem + C::OFF_K;
  uint8_t* Slds = smem + C::OFF_S;
  uint8_t* Vt = smem + C::OFF_VT;
  uint8_t* Pl = smem + C::OFF_P;
  float* wmax = reinterpret_cast<float*>(smem + C::OFF_MAX);
  float* lsum = reinterpret_cast<float*>(smem + C::OFF_L);

  const int32_t* plan = p.plan;
  if ((int)blockIdx.x >= plan[0]) return;
  const int4 it = reinterpret_cast<const int4*>(plan + kPlanHeader)[blockIdx.x];
  const int b = it.x, t_beg = it.y, t_end = it.z, slot = it.w;

  const int tid = threadIdx.x;
  const int w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;

  // ---- Q^T (B operand): head l16, dims 128ks + 32g .. +31 -------------------
  // With fp4 K, the f8f6f4 MFMA pairs fp4 element e of lane group g (K =
  // 32g + e within the 128-step, one MX block) with fp8 byte i of lane group
  // g' where 32g + e = 16g' + (i & 15) + 64 (i >> 4); the fp8 Q operand is
  // gathered in that order.  With fp8 K both operands share one order.
  v8i qv[5];
  {
    const uint8_t* qrow = p.q_fp8 + ((int64_t)b * 16 + l16) * kQKDim;
    if constexpr (KF == 0) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) qv[ks] = ld_v8(qrow + 128 * ks + 32 * g);
      qv[4] = g < 2 ? ld_v8(qrow + 512 + 32 * g) : v8i{0, 0, 0, 0, 0, 0, 0, 0};
    } else {
#pragma unroll
      for (int ks = 0; ks < 5; ++ks) {
        const uint4 lo = *reinterpret_cast<const uint4*>(qrow + 128 * ks + 16 * g);
        const uint4 hi = ks < 4 ? *reinterpret_cast<const uint4*>(qrow + 128 * ks + 64 + 16 * g)
                                : make_uint4(0, 0, 0, 0);
        qv[ks] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
      }
    }
#pragma unroll
    for (int ks = 0; ks < 5; ++ks) asm volatile("" : "+v"(qv[ks]));  // keep resident, no reload
  }
  const float qs = p.q_scale[0];
  const float kvs = (KF == 0 || VF == 1) ? p.kv_scale[0] : 1.0f;
  const float c = qs * (KF == 0 ? kvs : 1.0f) * p.sm_scale * kLog2e;
  const float vscale = (VF == 2 ? 1.0f : kvs / kPScale);

  v4f o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = v4f{0.f, 0.f, 0.f, 0.f};
  float m_run = neg_inf(), l_run = 0.f;

  TileLoader<256, KF, VF, IDX> L;
  L.init(tid);
  auto vt_off = [](int d, int tq) { return vt16_quad_off(d, tq); };

  const int ntok = t_end - t_beg;
  const int ntiles = (ntok + kTile - 1) / kTile;
  const int last = t_end - 1;
  if (ntiles > 0) {
    int sl[4];
    L.load_idx(p, t_beg, last, sl);
    L.load_rows(p, sl, min(kTile, ntok));
    L.load_idx(p, t_beg + kTile, last, L.sl_nxt);
  }

  // one 64-token tile; PF: prefetch the next tile's rows and the slots of the one after
  auto tile = [&](auto pf, int ti) {
    constexpr bool PF = decltype(pf)::value;
    const int t0 = ti * kTile;
    const int nval = min(kTile, ntok - t0);
    // ---- registers -> LDS ------------------------------------------------------
    L.store_k(Klds, C::KST, Slds);
    if constexpr (VF == 2) {
      // fp4 V: chunk lq (latent dims 32lq .. +31, scale block lq) -> bf16 V^T
      const int ch = L.lq;
      float sc[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[r] = e8m0_to_f32(L.valid(r) ? L.sr[0][r] : 127u);
#pragma unroll
      for (int wd = 0; wd < 4; ++wd) {
        uint32_t xw[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) xw[r] = reinterpret_cast<const uint32_t*>(&L.kr[0][r])[wd] & (L.valid(r) ? 0xFFFFFFFFu : 0u);
        uint32_t bf[4][4];  // [token][byte] -> bf16 pair (dims 2k, 2k+1)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          bf[r][0] = cvt_fp4_byte<0>(xw[r], sc[r]);
          bf[r][1] = cvt_fp4_byte<1>(xw[r], sc[r]);
          bf[r][2] = cvt_fp4_byte<2>(xw[r], sc[r]);
          bf[r][3] = cvt_fp4_byte<3>(xw[r], sc[r]);
        }
#pragma unroll
        for (int bt = 0; bt < 4; ++bt) {
          const int d0 = 32 * ch + 8 * wd + 2 * bt;
          const uint2 ev = make_uint2(__builtin_amdgcn_perm(bf[1][bt], bf[0][bt], 0x05040100u),
                                      __builtin_amdgcn_perm(bf[3][bt], bf[2][bt], 0x05040100u));
          const uint2 od = make_uint2(__builtin_amdgcn_perm(bf[1][bt], bf[0][bt], 0x07060302u),
                                      __builtin_amdgcn_perm(bf[3][bt], bf[2][bt], 0x07060302u));
          *reinterpret_cast<uint2*>(Vt + d0 * C::VTST + 8 * L.tq) = ev;
          *reinterpret_cast<uint2*>(Vt + (d0 + 1) * C::VTST + 8 * L.tq) = od;
        }
      }
    } else {
      L.store_v_fp8(Vt, vt_off);
    }
    __syncthreads();  // (A) tile visible
    if constexpr (PF) {
      L.load_rows(p, L.sl_nxt, min(kTile, ntok - t0 - kTile));
      L.load_idx(p, t_beg + t0 + 2 * kTile, last, L.sl_nxt);
    }

    // ---- scores for this wave's 16 tokens ------------------------------------
    v4f s = v4f{0.f, 0.f, 0.f, 0.f};
    const int trow = 16 * w + l16;
    if constexpr (KF == 0) {
      const uint8_t* kp = Klds + trow * C::KST;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) s = mfma16_f8(ld_v8(kp + 128 * ks + 32 * g), qv[ks], s);
      v8i a4 = g < 2 ? ld_v8(kp + 512 + 32 * g) : v8i{0, 0, 0, 0, 0, 0, 0, 0};
      s = mfma16_f8(a4, qv[4], s);
    } else {
      const uint8_t* kp = Klds + trow * C::KST;
      const uint8_t* sp = Slds + trow * 20;
#pragma unroll
      for (int ks = 0; ks < 5; ++ks) {
        const int blk = 4 * ks + g;
        v8i a = (blk < kMxBlocks) ? ld_v4_as_v8(kp + 16 * blk) : v8i{0, 0, 0, 0, 0, 0, 0, 0};
        const int sc = (blk < kMxBlocks) ? (int)sp[blk] : 127;
        s = mfma16_f4f8(a, sc, qv[ks], s);
      }
    }
    // s[r] = score(token 16w + 4g + r, head l16)
    float sv[4];
    float mx = neg_inf();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tok = 16 * w + 4 * g + r;
      sv[r] = tok < nval ? s[r] * c : neg_inf();
      mx = fmaxf(mx, sv[r]);
    }
    mx = fmaxf(mx, shfl_xor_f(mx, 16));
    mx = fmaxf(mx, shfl_xor_f(mx, 32));
    if (g == 0) wmax[w * 16 + l16] = mx;
    __syncthreads();  // (B)
    const float tmax = fmaxf(fmaxf(wmax[l16], wmax[16 + l16]), fmaxf(wmax[32 + l16], wmax[48 + l16]));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = exp2f(m_run - m_new);
    m_run = m_new;
    float pv[4];
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pv[r] = exp2f(sv[r] - m_new);
      psum += pv[r];
    }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] *= alpha;
    if constexpr (!C::VB16) {
      uint32_t hi, lo;
      pack4_fp8_split(pv[0] * kPScale, pv[1] * kPScale, pv[2] * kPScale, pv[3] * kPScale, hi, lo);
      *reinterpret_cast<uint32_t*>(Pl + l16 * C::PST + 16 * w + 4 * g) = hi;
      *reinterpret_cast<uint32_t*>(Pl + 16 * C::PST + l16 * C::PST + 16 * w + 4 * g) = lo;
    } else {
      const uint32_t lo = f32_to_bf16_bits(pv[0]) | (f32_to_bf16_bits(pv[1]) << 16);
      const uint32_t hi = f32_to_bf16_bits(pv[2]) | (f32_to_bf16_bits(pv[3]) << 16);
      *reinterpret_cast<uint2*>(Pl + l16 * C::PST + 2 * (16 * w + 4 * g)) = make_uint2(lo, hi);
    }
    __syncthreads();  // (C) P visible

    // ---- O^T[dims of this wave] += V^T . P^T --------------------------------
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if constexpr (!C::VB16) {
        const long bh = *reinterpret_cast<const long*>(Pl + l16 * C::PST + 32 * j + 8 * g);
        const long bl = *reinterpret_cast<const long*>(Pl + 16 * C::PST + l16 * C::PST + 32 * j + 8 * g);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const int d = 128 * w + 16 * dt + l16;
          const long av = *reinterpret_cast<const long*>(Vt + vt16_read_off(d, 4 * j + g));
          o[dt] = mfma16x32_f8(av, bh, o[dt]);
          o[dt] = mfma16x32_f8(av, bl, o[dt]);
        }
      } else {
        const v8bf bq = *reinterpret_cast<const v8bf*>(Pl + l16 * C::PST + 2 * (32 * j + 8 * g));
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const int d = 128 * w + 16 * dt + l16;
          const v8bf av = *reinterpret_cast<const v8bf*>(Vt + d * C::VTST + 2 * (32 * j + 8 * g));
          o[dt] = mfma16x32_bf16(av, bq, o[dt]);
        }
      }
    }
    __syncthreads();  // (D) LDS free for the next tile
  };
  for (int ti = 0; ti + 1 < ntiles; ++ti) tile(std::true_type{}, ti);
  if (ntiles > 0) tile(std::false_type{}, ntiles - 1);

  // ---- finish: row sums across lanes and waves --------------------------------
  float l = l_run;
  l += shfl_xor_f(l, 16);
  l += shfl_xor_f(l, 32);
  if (g == 0) lsum[w * 16 + l16] = l;
  __syncthreads();
  const float Lsum = lsum[l16] + lsum[16 + l16] + lsum[32 + l16] + lsum[48 + l16];
  const float inv = Lsum > 0.f ? vscale / Lsum : 0.f;
  const int head = l16;
  if (slot < 0) {
    uint16_t* orow = p.out + ((int64_t)b * 16 + head) * kVDim;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int d = 128 * w + 16 * dt + 4 * g;
      const uint32_t lo = f32_to_bf16_bits(o[dt][0] * inv) | (f32_to_bf16_bits(o[dt][1] * inv) << 16);
      const uint32_t hi = f32_to_bf16_bits(o[dt][2] * inv) | (f32_to_bf16_bits(o[dt][3] * inv) << 16);
      *reinterpret_cast<uint2*>(orow + d) = make_uint2(lo, hi);
    }
  } else {
    float* prow = p.part_o + ((int64_t)slot * 16 + head) * kVDim;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int d = 128 * w + 16 * dt + 4 * g;
      *reinterpret_cast<float4*>(prow + d) =
          make_float4(o[dt][0] * inv, o[dt][1] * inv, o[dt][2] * inv, o[dt][3] * inv);
    }
    if (w == 0 && g == 0) p.part_lse[(int64_t)slot * 16 + head] = Lsum > 0.f ? m_run + __log2f(Lsum) : neg_inf();
  }
}

// ============================================================================
// H = 128.  4 waves; wave w owns heads 32w .. 32w+31 for every token of the
// work item and all 512 latent dims, so the softmax state and O^T never leave
// the wave.  Q^T (the QK B operand) stays in registers, O^T in accumulators.
// Cache rows are gathered straight into an LDS ring by LDS-DMA (no staging
// registers), S tiles deep; the PV A operand (V^T) is read from the row-major
// tile with ds_read_b64_tr_b8, so no transposed copy is ever written.
//   KF: 0 = fp8 K rows, V = same rows; 1 = fp4 K rows + e8m0, V = fp8 cache
// Online softmax is rescaled lazily: the exponent base m only moves when a
// head's tile max exceeds it by more than 8 (log2 units), so P <= 2^8 fits
// e4m3 and O^T is touched by VALU only on those (rare) tiles.
// ============================================================================
template <int KF>
struct H128 {
  static constexpr int NT = 256;
  static constexpr int KST = KF == 0 ? 592 : 304;              // K row stride in LDS
  static constexpr int KCH = KF == 0 ? 36 : 18;                // real 16-B chunks per K row
  static constexpr int VST = 528;                              // fp8 V row stride (KF == 1)
  static constexpr int KDMA = (kTile * KST + 1023) / 1024;     // 1-KiB DMA windows: 37 / 19
  static constexpr int VDMA = KF == 1 ? (kTile * VST + 1023) / 1024 : 0;  // 33
  static constexpr int DPW = (KDMA + VDMA + 3) / 4;            // windows per wave: 10 / 13
  static constexpr int STAGE = 4 * DPW * 1024;                 // ring stage bytes
  static constexpr int S = KF == 0 ? 3 : 2;                    // ring depth (tiles)
  static constexpr int OFF_V = KDMA * 1024;                    // V rows inside a stage (KF == 1)
  static constexpr int OFF_SLOT = S * STAGE;                   // [S][64] int32 cache slots
  static constexpr int OFF_VOTE = OFF_SLOT + S * 256;          // [2][4] restart votes
  static constexpr int LDS = OFF_VOTE + 16;
};

template <int KF, bool IDX>
__global__ __launch_bounds__(256, 1) void decode_h128_kernel(const DecodeParams p) {
  using C = H128<KF>;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[C::LDS];
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;

  const int32_t* plan = p.plan;
  if ((int)blockIdx.x >= plan[0]) return;
  const int4 it = reinterpret_cast<const int4*>(plan + kPlanHeader)[blockIdx.x];
  const int b = it.x, t_beg = it.y, t_end = it.z, slot = it.w;
  const int ntok = t_end - t_beg;
  const int ntiles = (ntok + kTile - 1) / kTile;

  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (feeds M0)
  const int lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int head = 32 * w + l32;

  // ---- Q^T B operand, K-step ks = dims 64ks .. +63 (fp4 K: partner order) -----
  v8i qv[9];
  {
    const uint8_t* qrow = p.q_fp8 + ((int64_t)b * 128 + head) * kQKDim;
#pragma unroll
    for (int ks = 0; ks < 9; ++ks) {
      const int d0 = KF == 0 ? 64 * ks + 32 * hh : 64 * ks + 16 * hh;
      const int d1 = KF == 0 ? d0 + 16 : d0 + 32;
      const uint4 lo = *reinterpret_cast<const uint4*>(qrow + d0);
      const uint4 hi = *reinterpret_cast<const uint4*>(qrow + d1);
      qv[ks] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    }
#pragma unroll
    for (int ks = 0; ks < 9; ++ks) asm volatile("" : "+v"(qv[ks]));
  }
  const float qs = p.q_scale[0];
  const float kvs = p.kv_scale[0];
  const float c = qs * (KF == 0 ? kvs : 1.0f) * p.sm_scale * kLog2e;
  const float vscale = kvs;  // the 2^8 carried by P' is folded into the PV scale exponent

  v16f o[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = v16f{};
  float m_ref = 0.f, l_run = 0.f;

  // ---- DMA issue helpers -------------------------------------------------------
  auto slot_of = [&](int st, int tok, int pos0) -> int {
    if constexpr (IDX) return reinterpret_cast<const int*>(smem + C::OFF_SLOT + st * 256)[tok];
    else return min(pos0 + tok, t_end - 1);
  };
  auto issue_slots = [&](int t) {  // wave 0: 64 slots of tile t (positions clamped into the item)
    if constexpr (IDX) {
      if (w == 0) {
        const int pos = min(t_beg + kTile * t + lane, t_end - 1);
        dma4_to_lds(p.kv_indices + pos, lds0 + C::OFF_SLOT + (t % C::S) * 256);
      }
    }
  };
  auto issue_rows = [&](int t) {  // this wave's DPW windows of tile t
    const int st = t % C::S;
    const int pos0 = t_beg + kTile * t;
    const uint32_t sbase = lds0 + st * C::STAGE;
#pragma unroll
    for (int k = 0; k < C::DPW; ++k) {
      const int u = w + 4 * k;  // window index within the stage
      const uint8_t* src;
      if (u < C::KDMA) {
        const int bb = 1024 * u + 16 * lane;
        int tok = bb / C::KST, pos = (bb - tok * C::KST) >> 4;
        if (tok >= kTile) { tok = kTile - 1; pos = 0; }
        src = p.k_cache + (int64_t)slot_of(st, tok, pos0) * p.k_row_stride + 16 * min(pos, C::KCH - 1);
      } else if (KF == 1 && u < C::KDMA + C::VDMA) {
        const int bb = 1024 * (u - C::KDMA) + 16 * lane;
        int tok = bb / C::VST, pos = (bb - tok * C::VST) >> 4;
        if (tok >= kTile) { tok = kTile - 1; pos = 0; }
        src = p.v_cache + (int64_t)slot_of(st, tok, pos0) * p.v_row_stride + 16 * min(pos, 31);
      } else {  // padding window: any valid source
        src = p.k_cache + (int64_t)slot_of(st, kTile - 1, pos0) * p.k_row_stride;
      }
      dma16_to_lds(src, sbase + 1024 * u);
    }
  };
  // fp4 K scales: lane (token u*32 + l32) needs blocks 2ks + hh, ks = 0..8
  uint32_t sc_nxt[2][9], sc_cur[2][9];
  auto load_scales = [&](int t) {
    if constexpr (KF == 1) {
      const int st = t % C::S;
      const int pos0 = t_beg + kTile * t;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint8_t* srow = p.k_scales + (int64_t)slot_of(st, 32 * u + l32, pos0) * p.k_scale_stride;
#pragma unroll
        for (int ks = 0; ks < 9; ++ks) sc_nxt[u][ks] = srow[2 * ks + hh];
      }
    }
  };

  auto prologue = [&]() {
    // prologue: slots(0) visible; rows(0) [+ scales(0)] in flight; slots(1), and for S = 3
    // rows(1) and slots(2), issued in the order the steady-state waits assume
    issue_slots(0);
    wait_vmcnt<0>();
    lds_barrier();
    issue_slots(1);
    issue_rows(0);
    load_scales(0);
    if constexpr (C::S == 3) {
      if (ntiles > 1) {
        wait_vmcnt<C::DPW>();  // slots(1) landed (rows(0) may still be in flight)
        lds_barrier();
        issue_slots(2);
        issue_rows(1);
      }
    }
  };

  // lane-constant parts of the transpose-read addresses (PV A operand)
  const int vrow_st = KF == 0 ? C::KST : C::VST;
  const int voff = KF == 0 ? 0 : C::OFF_V;
  int tr_off[4];
  {
    const int G = lane >> 4, m = (lane & 15) >> 1, oo = lane & 1;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const int k = 8 * cc + m;  // K-slot of this lane half
      const int T = 32 * (k >> 4) + 8 * ((k >> 2) & 3) + 4 * hh + (k & 3);
      tr_off[cc] = voff + T * vrow_st + 16 * (G & 1) + 8 * oo;
    }
  }

  // O^T accumulates sum_n V_n 2^(s_n - m_ref) against a fixed per-lane (head)
  // reference, the first tile's ceil(max); a tile's own offset rides on the
  // B-operand e8m0 scale of the PV MFMA, so the accumulators are never
  // rescaled.  A tile whose max lies more than kRebase above m_ref (the
  // accumulators could overflow) makes the whole block restart the item with
  // m_ref = the running max: a block-wide vote through LDS, one tile late.
  volatile uint8_t* vote = smem + C::OFF_VOTE;  // [2][4] wave flags, double-buffered by tile parity
  float m_seen = neg_inf();
  bool have_ref = false;
  for (;;) {
  if (ntiles > 0) prologue();
  bool restart = false;
  for (int ti = 0; ti < ntiles; ++ti) {
    const int st = ti % C::S;
    const int nval = min(kTile, ntok - kTile * ti);
    // tile ti landed (and slots for the tile issued next); see the prologue order
    if constexpr (C::S == 3) {
      if (ti + 1 < ntiles) wait_vmcnt<C::DPW>();
      else wait_vmcnt<0>();
    } else {
      wait_vmcnt<0>();
    }
    if constexpr (KF == 1) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int ks = 0; ks < 9; ++ks) sc_cur[u][ks] = sc_nxt[u][ks];
    }
    lds_barrier();  // tile ti visible; the stage of tile ti-1 is free
    if (ti > 0 && __builtin_amdgcn_readfirstlane(*reinterpret_cast<volatile uint32_t*>(vote + 4 * ((ti - 1) & 1))) != 0) {
      restart = true;
      break;
    }
    if (ti + C::S - 1 < ntiles) {
      issue_slots(ti + C::S);
      issue_rows(ti + C::S - 1);
      if constexpr (KF == 1) load_scales(ti + C::S - 1);
    }

    // ---- scores S^T: s0 = tokens 0..31, s1 = tokens 32..63 of the tile ------------
    const uint32_t sb = lds0 + st * C::STAGE;
    const uint8_t* kt = smem + st * C::STAGE;
    v16f s0 = v16f{}, s1 = v16f{};
    // one K-step of lookahead on the LDS fragments; sched_barrier keeps the
    // compiler from hoisting every fragment load (register blow-up)
    auto kfrag = [&](int ks, int u) -> v8i {
      if constexpr (KF == 0) return ld_v8(kt + (32 * u + l32) * C::KST + 64 * ks + 32 * hh);
      else return ld_v4_as_v8(kt + (32 * u + l32) * C::KST + 16 * (2 * ks + hh));
    };
    v8i a0n = kfrag(0, 0), a1n = kfrag(0, 1);
#pragma unroll
    for (int ks = 0; ks < 9; ++ks) {
      const v8i a0 = a0n, a1 = a1n;
      if (ks < 8) {
        a0n = kfrag(ks + 1, 0);
        a1n = kfrag(ks + 1, 1);
      }
      if constexpr (KF == 0) {
        s0 = mfma32_f8(a0, qv[ks], s0);
        s1 = mfma32_f8(a1, qv[ks], s1);
      } else {
        s0 = mfma32_f4f8(a0, (int)sc_cur[0][ks], qv[ks], s0);
        s1 = mfma32_f4f8(a1, (int)sc_cur[1][ks], qv[ks], s1);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    (void)sb;
    // s_u[r] = score(token 32u + 8(r/4) + 4hh + r%4, head)
    float mx = neg_inf();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int tk = 8 * (r >> 2) + 4 * hh + (r & 3);
      s0[r] = tk < nval ? s0[r] * c : neg_inf();
      s1[r] = 32 + tk < nval ? s1[r] * c : neg_inf();
      mx = fmaxf(mx, fmaxf(s0[r], s1[r]));
    }
    mx = fmaxf(mx, shfl_xor_f(mx, 32));
    // Fixed per-item reference m_ref (the first tile's ceil(max)); each tile's
    // offset rides on the B-operand e8m0 scale of the PV MFMA, so O^T is never
    // rescaled: O^T accumulates sum_n V_n 2^(s_n - m_ref).
    const float m_t = __builtin_ceilf(mx);
    if (!have_ref) m_ref = m_t;  // first tile of the first pass
    have_ref = true;
    m_seen = fmaxf(m_seen, m_t);
    const bool over = __any(m_t > m_ref + kRebase);
    if (lane == 0) vote[4 * (ti & 1) + w] = over ? 1 : 0;
    // P' = 2^(s - m_t) * 2^8 in fp8; the e8m0 B scale 2^(m_t - m_ref - 8) restores 2^(s - m_ref)
    const float dm = fminf(fmaxf(m_t - m_ref, -160.f), 160.f);
    const int pscale = min(max((int)dm - 8 + 127, 0), 254);
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s0[r] = exp2f(s0[r] - m_t);
      s1[r] = exp2f(s1[r] - m_t);
      psum += s0[r] + s1[r];
    }
    l_run += psum * exp2f(dm);
    // P'^T B operand: byte 16u + 4q + i <-> token 32u + 8q + 4hh + i; hi + lo fp8 terms
    v8i pbh, pbl;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t h0, l0, h1, l1;
      pack4_fp8_split(s0[4 * q] * kPScale, s0[4 * q + 1] * kPScale, s0[4 * q + 2] * kPScale,
                      s0[4 * q + 3] * kPScale, h0, l0);
      pack4_fp8_split(s1[4 * q] * kPScale, s1[4 * q + 1] * kPScale, s1[4 * q + 2] * kPScale,
                      s1[4 * q + 3] * kPScale, h1, l1);
      pbh[q] = (int)h0;
      pbl[q] = (int)l0;
      pbh[4 + q] = (int)h1;
      pbl[4 + q] = (int)l1;
    }
    // ---- O^T += V^T . P^T, V^T fragments by transpose reads of the row tile ------
    auto vfrag = [&](int dt) -> v8i {
      const uint32_t vb = lds0 + st * C::STAGE + 32 * dt;
      const v2i r0 = lds_read_tr8(vb + tr_off[0]);
      const v2i r1 = lds_read_tr8(vb + tr_off[1]);
      const v2i r2 = lds_read_tr8(vb + tr_off[2]);
      const v2i r3 = lds_read_tr8(vb + tr_off[3]);
      return v8i{r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
    };
    v8i avn = vfrag(0);
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) {
      const v8i av = avn;
      if (dt < 15) avn = vfrag(dt + 1);
      o[dt] = mfma32_f8_bscale(av, pbh, pscale, o[dt]);
      o[dt] = mfma32_f8_bscale(av, pbl, pscale, o[dt]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (!restart && ntiles > 0) {
    lds_barrier();  // the last tile's votes
    restart = __builtin_amdgcn_readfirstlane(*reinterpret_cast<volatile uint32_t*>(vote + 4 * ((ntiles - 1) & 1))) != 0;
  }
  if (!restart) break;
  // drain the ring (the prologue reuses it), then start over from m_ref = running max
  wait_vmcnt<0>();
  lds_barrier();
  m_ref = m_seen;
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = v16f{};
  l_run = 0.f;
  }

  // ---- finish ---------------------------------------------------------------------
  const float L = l_run + shfl_xor_f(l_run, 32);
  const float inv = L > 0.f ? vscale / L : 0.f;
  if (slot < 0) {
    uint16_t* orow = p.out + ((int64_t)b * 128 + head) * kVDim;
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int d = 32 * dt + 8 * q + 4 * hh;
        const uint32_t lo = f32_to_bf16_bits(o[dt][4 * q] * inv) | (f32_to_bf16_bits(o[dt][4 * q + 1] * inv) << 16);
        const uint32_t hi = f32_to_bf16_bits(o[dt][4 * q + 2] * inv) | (f32_to_bf16_bits(o[dt][4 * q + 3] * inv) << 16);
        *reinterpret_cast<uint2*>(orow + d) = make_uint2(lo, hi);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    float* prow = p.part_o + ((int64_t)slot * 128 + head) * kVDim;
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int d = 32 * dt + 8 * q + 4 * hh;
        *reinterpret_cast<float4*>(prow + d) = make_float4(o[dt][4 * q] * inv, o[dt][4 * q + 1] * inv,
                                                           o[dt][4 * q + 2] * inv, o[dt][4 * q + 3] * inv);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (hh == 0) p.part_lse[(int64_t)slot * 128 + head] = L > 0.f ? m_ref + __log2f(L) : neg_inf();
  }
}

// ============================================================================
// LSE combine: out[b,h,:] = sum_s 2^(lse_s - M) O_s / sum_s 2^(lse_s - M)
// grid (batch, H/16), 256 threads: thread = (head in group, 32-dim slice)
// ============================================================================
__global__ __launch_bounds__(256) void combine_kernel(const DecodeParams p) {
  const int b = blockIdx.x;
  const int H = p.num_heads;
  const int2* binfo = reinterpret_cast<const int2*>(p.plan + kPlanHeader + 4 * p.max_items);
  const int2 bi = binfo[b];
  if (bi.y <= 1) return;
  const int head = blockIdx.y * 16 + (threadIdx.x >> 4);
  const int d0 = (threadIdx.x & 15) * 32;
  float M = neg_inf();
  for (int s = 0; s < bi.y; ++s) M = fmaxf(M, p.part_lse[(int64_t)(bi.x + s) * H + head]);
  float acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) acc[i] = 0.f;
  float wsum = 0.f;
  if (M != neg_inf()) {
    for (int s = 0; s < bi.y; ++s) {
      const int64_t slot = bi.x + s;
      const float wgt = exp2f(p.part_lse[slot * H + head] - M);
      wsum += wgt;
      const float4* src = reinterpret_cast<const float4*>(p.part_o + (slot * H + head) * kVDim + d0);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float4 v = src[i];
        acc[4 * i + 0] += wgt * v.x;
        acc[4 * i + 1] += wgt * v.y;
        acc[4 * i + 2] += wgt * v.z;
        acc[4 * i + 3] += wgt * v.w;
      }
    }
  }
  const float inv = wsum > 0.f ? 1.0f / wsum : 0.f;
  uint16_t* orow = p.out + ((int64_t)b * H + head) * kVDim + d0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t lo = f32_to_bf16_bits(acc[4 * i] * inv) | (f32_to_bf16_bits(acc[4 * i + 1] * inv) << 16);
    const uint32_t hi = f32_to_bf16_bits(acc[4 * i + 2] * inv) | (f32_to_bf16_bits(acc[4 * i + 3] * inv) << 16);
    *reinterpret_cast<uint2*>(orow + 4 * i) = make_uint2(lo, hi);
  }
}

// ============================================================================
template <bool IDX>
static hipError_t launch_decode_t(const DecodeParams& p, int kv_mode, int grid, hipStream_t stream) {
  if (p.num_heads == 16) {
    switch (kv_mode) {
      case 0: hipLaunchKernelGGL((decode_h16_kernel<0, 0, IDX>), dim3(grid), dim3(256), 0, stream, p); break;
      case 1: hipLaunchKernelGGL((decode_h16_kernel<1, 2, IDX>), dim3(grid), dim3(256), 0, stream, p); break;
      case 2: hipLaunchKernelGGL((decode_h16_kernel<1, 1, IDX>), dim3(grid), dim3(256), 0, stream, p); break;
      default: return hipErrorInvalidValue;
    }
  } else if (p.num_heads == 128) {
    switch (kv_mode) {
      case 0: hipLaunchKernelGGL((decode_h128_kernel<0, IDX>), dim3(grid), dim3(256), 0, stream, p); break;
      case 2: hipLaunchKernelGGL((decode_h128_kernel<1, IDX>), dim3(grid), dim3(256), 0, stream, p); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_decode(const DecodeParams& p, int kv_mode, int grid, hipStream_t stream) {
  return p.kv_indices != nullptr ? launch_decode_t<true>(p, kv_mode, grid, stream)
                                 : launch_decode_t<false>(p, kv_mode, grid, stream);
}

hipError_t launch_combine(const DecodeParams& p, hipStream_t stream) {
  hipLaunchKernelGGL(combine_kernel, dim3(p.batch, p.num_heads / 16), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mla
