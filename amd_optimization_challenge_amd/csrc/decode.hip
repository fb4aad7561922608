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
// H = 128: 8 waves.  Wave w owns head group g4 = w & 3 (heads 32*g4 .. +31) and
// half = w >> 2: it scores token half `half` of each 64-token tile (32x32x64
// MFMAs over the 576 dims) and accumulates O^T for latent dims 256*half .. +255
// over all 64 tokens.  The two waves of a head group swap their tile maxima and
// their halves of P through LDS, so both run the same online softmax.
//   KF: 0 = fp8 K rows, V = same rows; 1 = fp4 K rows + e8m0, V = fp8 cache
// ============================================================================
template <int KF>
struct H128 {
  static constexpr int KROW = KF == 0 ? 576 : 288;
  static constexpr int KST = KROW + 16;
  static constexpr int OFF_K = 0;
  static constexpr int OFF_S = OFF_K + kTile * KST;
  static constexpr int OFF_VT = OFF_S + (KF == 1 ? kTile * 20 : 0);
  static constexpr int OFF_Q = OFF_VT + kVDim * 64;        // V^T rows of 64 bytes
  static constexpr int OFF_P = OFF_Q + 128 * kQKDim;       // [hi/lo][4 groups][64 lanes][32 B]
  static constexpr int OFF_MAX = OFF_P + 2 * 4 * 64 * 32;  // [2 halves][128] f32
  static constexpr int OFF_L = OFF_MAX + 2 * 128 * 4;      // [2 halves][128] f32
  static constexpr int LDS = OFF_L + 2 * 128 * 4;
  static constexpr int NT = 512;
};

// V^T row of latent dim d: token n sits at byte pos(n) = 32hh + 16u + 4q + i
// (n = 32u + 8q + 4hh + i), the order of the P operand built from the 32x32
// score accumulators.  The row's four 16-byte chunks are XOR-swizzled by
// ((d >> 2) ^ (d >> 4)) & 3 so that both the transposed writes (dims 16 apart)
// and the operand reads (consecutive dims) spread over the banks.
__device__ __forceinline__ int vt128_sw(int d) { return ((d >> 2) ^ (d >> 4)) & 3; }
__device__ __forceinline__ int vt128_quad_off(int d, int tq) {
  const int pos = 32 * (tq & 1) + 16 * (tq >> 3) + 4 * ((tq & 7) >> 1);
  return d * 64 + 16 * ((pos >> 4) ^ vt128_sw(d)) + (pos & 15);
}
// Q chunk swizzle: 16-byte chunk c (0..35) of head row h lives at chunk
// c ^ ((h >> 2) & 3), which stays inside the row (36 is a multiple of 4).  Rows
// are 36 chunks apart, so heads h and h+4 would otherwise hit the same banks.
__device__ __forceinline__ int q_off(int h, int c) { return h * kQKDim + 16 * (c ^ ((h >> 2) & 3)); }

template <int KF, bool IDX>
__global__ __launch_bounds__(512, 1) void decode_h128_kernel(const DecodeParams p) {
  using C = H128<KF>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[C::LDS];
  uint8_t* Klds = smem + C::OFF_K;
  uint8_t* Slds = smem + C::OFF_S;
  uint8_t* Vt = smem + C::OFF_VT;
  uint8_t* Qlds = smem + C::OFF_Q;
  uint8_t* Pex = smem + C::OFF_P;
  float* smax = reinterpret_cast<float*>(smem + C::OFF_MAX);
  float* lsum = reinterpret_cast<float*>(smem + C::OFF_L);

  const int32_t* plan = p.plan;
  if ((int)blockIdx.x >= plan[0]) return;
  const int4 it = reinterpret_cast<const int4*>(plan + kPlanHeader)[blockIdx.x];
  const int b = it.x, t_beg = it.y, t_end = it.z, slot = it.w;

  const int tid = threadIdx.x;
  const int w = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int g4 = w & 3, half = w >> 2;
  const int head = 32 * g4 + l32;

  // Q [128][576] fp8 -> LDS; visible after barrier (A)
  {
    const uint8_t* qb = p.q_fp8 + (int64_t)b * 128 * kQKDim;
    for (int k = tid; k < 128 * 36; k += C::NT) {
      const int h = k / 36, ch = k - h * 36;
      *reinterpret_cast<uint4*>(Qlds + q_off(h, ch)) = *reinterpret_cast<const uint4*>(qb + h * kQKDim + 16 * ch);
    }
  }
  const float qs = p.q_scale[0];
  const float kvs = p.kv_scale[0];
  const float c = qs * (KF == 0 ? kvs : 1.0f) * p.sm_scale * kLog2e;
  const float vscale = kvs / kPScale;

  v16f o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = v16f{};
  float m_run = neg_inf(), l_run = 0.f;

  TileLoader<C::NT, KF, KF == 1 ? 1 : 0, IDX> L;
  L.init(tid);
  auto vt_off = [](int d, int tq) { return vt128_quad_off(d, tq); };

  const int ntok = t_end - t_beg;
  const int ntiles = (ntok + kTile - 1) / kTile;
  const int last = t_end - 1;
  if (ntiles > 0) {
    int sl[4];
    L.load_idx(p, t_beg, last, sl);
    L.load_rows(p, sl, min(kTile, ntok));
    L.load_idx(p, t_beg + kTile, last, L.sl_nxt);
  }

  auto tile = [&](auto pf, int ti) {
    constexpr bool PF = decltype(pf)::value;
    const int t0 = ti * kTile;
    const int nval = min(kTile, ntok - t0);
    L.store_k(Klds, C::KST, Slds);
    L.store_v_fp8(Vt, vt_off);
    __syncthreads();  // (A) tile (and Q) visible
    if constexpr (PF) {
      L.load_rows(p, L.sl_nxt, min(kTile, ntok - t0 - kTile));
      L.load_idx(p, t_beg + t0 + 2 * kTile, last, L.sl_nxt);
    }

    // ---- scores S^T for tokens 32*half .. +31 of this tile, heads of g4 -------
    v16f s = v16f{};
    const int trow = 32 * half + l32;
#pragma unroll
    for (int ks = 0; ks < 9; ++ks) {
      // Q chunks of this lane's head for K-step ks: fp8 K pairs dims 64ks+32hh..+31;
      // fp4 K pairs dims 64ks+16hh..+15 and 64ks+32+16hh..+15 (f8f6f4 fp4 order)
      const int qc0 = KF == 0 ? 4 * ks + 2 * hh : 4 * ks + hh;
      const int qc1 = KF == 0 ? qc0 + 1 : qc0 + 2;
      v8i qf;
      {
        const uint4 a = *reinterpret_cast<const uint4*>(Qlds + q_off(head, qc0));
        const uint4 bq = *reinterpret_cast<const uint4*>(Qlds + q_off(head, qc1));
        qf[0] = a.x; qf[1] = a.y; qf[2] = a.z; qf[3] = a.w;
        qf[4] = bq.x; qf[5] = bq.y; qf[6] = bq.z; qf[7] = bq.w;
      }
      if constexpr (KF == 0) {
        s = mfma32_f8(ld_v8(Klds + trow * C::KST + 64 * ks + 32 * hh), qf, s);
      } else {
        const int blk = 2 * ks + hh;
        s = mfma32_f4f8(ld_v4_as_v8(Klds + trow * C::KST + 16 * blk), (int)Slds[trow * 20 + blk], qf, s);
      }
    }
    // s[r] = score(token 32*half + 8(r/4) + 4hh + r%4, head)
    float mx = neg_inf();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int tk = 32 * half + 8 * (r >> 2) + 4 * hh + (r & 3);
      s[r] = tk < nval ? s[r] * c : neg_inf();
      mx = fmaxf(mx, s[r]);
    }
    mx = fmaxf(mx, shfl_xor_f(mx, 32));
    if (hh == 0) smax[half * 128 + head] = mx;
    __syncthreads();  // (B) half maxima visible
    const float tmax = fmaxf(smax[head], smax[128 + head]);
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = exp2f(m_run - m_new);
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = exp2f(s[r] - m_new);
      psum += s[r];
    }
    l_run = l_run * alpha + psum;
    // this wave's half of the P^T B operand: bytes 16*half .. +15 of the lane's 32
    {
      uint4 ph, pl;
      pack4_fp8_split(s[0] * kPScale, s[1] * kPScale, s[2] * kPScale, s[3] * kPScale, ph.x, pl.x);
      pack4_fp8_split(s[4] * kPScale, s[5] * kPScale, s[6] * kPScale, s[7] * kPScale, ph.y, pl.y);
      pack4_fp8_split(s[8] * kPScale, s[9] * kPScale, s[10] * kPScale, s[11] * kPScale, ph.z, pl.z);
      pack4_fp8_split(s[12] * kPScale, s[13] * kPScale, s[14] * kPScale, s[15] * kPScale, ph.w, pl.w);
      *reinterpret_cast<uint4*>(Pex + (g4 * 64 + lane) * 32 + 16 * half) = ph;
      *reinterpret_cast<uint4*>(Pex + 8192 + (g4 * 64 + lane) * 32 + 16 * half) = pl;
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] *= alpha;
    __syncthreads();  // (C) both halves of P visible
    const v8i pbh = ld_v8(Pex + (g4 * 64 + lane) * 32);
    const v8i pbl = ld_v8(Pex + 8192 + (g4 * 64 + lane) * 32);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int d = 256 * half + 32 * dt + l32;
      const int sw = vt128_sw(d);
      v8i av;
      {
        const uint4 a0 = *reinterpret_cast<const uint4*>(Vt + d * 64 + 16 * ((2 * hh) ^ sw));
        const uint4 a1 = *reinterpret_cast<const uint4*>(Vt + d * 64 + 16 * ((2 * hh + 1) ^ sw));
        av[0] = a0.x; av[1] = a0.y; av[2] = a0.z; av[3] = a0.w;
        av[4] = a1.x; av[5] = a1.y; av[6] = a1.z; av[7] = a1.w;
      }
      o[dt] = mfma32_f8(av, pbh, o[dt]);
      o[dt] = mfma32_f8(av, pbl, o[dt]);
    }
    __syncthreads();  // (D) LDS free for the next tile
  };
  for (int ti = 0; ti + 1 < ntiles; ++ti) tile(std::true_type{}, ti);
  if (ntiles > 0) tile(std::false_type{}, ntiles - 1);

  // ---- finish: row sum over both lane halves and both half-waves ---------------
  float l = l_run + shfl_xor_f(l_run, 32);
  if (hh == 0) lsum[half * 128 + head] = l;
  __syncthreads();
  const float Lsum = lsum[head] + lsum[128 + head];
  const float inv = Lsum > 0.f ? vscale / Lsum : 0.f;
  if (slot < 0) {
    uint16_t* orow = p.out + ((int64_t)b * 128 + head) * kVDim;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int d = 256 * half + 32 * dt + 8 * q + 4 * hh;
        const uint32_t lo = f32_to_bf16_bits(o[dt][4 * q] * inv) | (f32_to_bf16_bits(o[dt][4 * q + 1] * inv) << 16);
        const uint32_t hi = f32_to_bf16_bits(o[dt][4 * q + 2] * inv) | (f32_to_bf16_bits(o[dt][4 * q + 3] * inv) << 16);
        *reinterpret_cast<uint2*>(orow + d) = make_uint2(lo, hi);
      }
    }
  } else {
    float* prow = p.part_o + ((int64_t)slot * 128 + head) * kVDim;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int d = 256 * half + 32 * dt + 8 * q + 4 * hh;
        *reinterpret_cast<float4*>(prow + d) = make_float4(o[dt][4 * q] * inv, o[dt][4 * q + 1] * inv,
                                                           o[dt][4 * q + 2] * inv, o[dt][4 * q + 3] * inv);
      }
    }
    if (hh == 0 && half == 0) p.part_lse[(int64_t)slot * 128 + head] = Lsum > 0.f ? m_run + __log2f(Lsum) : neg_inf();
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
      case 0: hipLaunchKernelGGL((decode_h128_kernel<0, IDX>), dim3(grid), dim3(512), 0, stream, p); break;
      case 2: hipLaunchKernelGGL((decode_h128_kernel<1, IDX>), dim3(grid), dim3(512), 0, stream, p); break;
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
