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
// H = 16
//   KF: 0 = fp8 K rows (576 B), 1 = packed fp4 K rows (288 B) + e8m0 scales
//   VF: 0 = fp8 V = K rows, 1 = fp8 V from its own cache, 2 = fp4 V = K rows
// ============================================================================
template <int KF, int VF>
struct H16 {
  static constexpr int KROW = KF == 0 ? 576 : 288;
  static constexpr int KCH = KROW / 16;               // 16-byte chunks per K row
  static constexpr int KST = KROW + 16;               // LDS row stride (bank spread)
  static constexpr bool VB16 = VF == 2;               // V^T / P held as bf16
  static constexpr int EV = VB16 ? 2 : 1;             // bytes per V^T / P element
  static constexpr int VTST = 64 * EV + 8 * EV;       // LDS bytes per latent dim row
  static constexpr int PST = 64 * EV + 8 * EV;
  static constexpr int OFF_K = 0;
  static constexpr int OFF_S = OFF_K + kTile * KST;
  static constexpr int OFF_VT = OFF_S + (KF == 1 ? kTile * 20 : 0);
  static constexpr int OFF_P = OFF_VT + kVDim * VTST;
  static constexpr int OFF_MAX = OFF_P + 16 * PST;
  static constexpr int OFF_L = OFF_MAX + 4 * 16 * 4;
  static constexpr int LDS = OFF_L + 4 * 16 * 4;
  // global->register items per thread per tile
  //   K rows: (token quad, 16-B chunk): 16 * KCH items
  //   V rows (VF == 1): 16 * 32 items of fp8 V
  static constexpr int KITEMS = 16 * KCH;
  static constexpr int KIT = (KITEMS + 255) / 256;
  static constexpr int VITEMS = VF == 1 ? 16 * 32 : 0;
  static constexpr int VIT = (VITEMS + 255) / 256;
};

template <int KF, int VF>
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
  v8i qv[5];
  {
    const uint8_t* qrow = p.q_fp8 + ((int64_t)b * 16 + l16) * kQKDim;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qv[ks] = ld_v8(qrow + 128 * ks + 32 * g);
    qv[4] = g < 2 ? ld_v8(qrow + 512 + 32 * g) : v8i{0, 0, 0, 0, 0, 0, 0, 0};
  }
  const float qs = p.q_scale[0];
  const float kvs = (KF == 0 || VF == 1) ? p.kv_scale[0] : 1.0f;
  const float c = qs * (KF == 0 ? kvs : 1.0f) * p.sm_scale * kLog2e;
  const float vscale = (VF == 2 ? 1.0f : kvs / kPScale);

  v4f o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = v4f{0.f, 0.f, 0.f, 0.f};
  float m_run = neg_inf(), l_run = 0.f;

  // ---- prefetch registers ----------------------------------------------------
  uint4 kr[C::KIT][4];
  uint4 vr[C::VIT > 0 ? C::VIT : 1][4];
  uint32_t sr[5];  // e8m0 bytes (fp4 K): token tid>>2, blocks (tid&3)+4j

  auto load_tile = [&](int t0, int nval) {
#pragma unroll
    for (int i = 0; i < C::KIT; ++i) {
      const int k = tid + 256 * i;
      const int tq = k / C::KCH, ch = k - tq * C::KCH;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tok = 4 * tq + r;
        if (k < C::KITEMS && tok < nval) {
          const int s = kv_slot(p.kv_indices, t0 + tok);
          kr[i][r] = ldg16(p.k_cache + (int64_t)s * p.k_row_stride + 16 * ch);
        } else {
          kr[i][r] = make_uint4(0, 0, 0, 0);
        }
      }
    }
    if constexpr (VF == 1) {
#pragma unroll
      for (int i = 0; i < C::VIT; ++i) {
        const int k = tid + 256 * i;
        const int tq = k >> 5, ch = k & 31;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tok = 4 * tq + r;
          if (tok < nval) {
            const int s = kv_slot(p.kv_indices, t0 + tok);
            vr[i][r] = ldg16(p.v_cache + (int64_t)s * p.v_row_stride + 16 * ch);
          } else {
            vr[i][r] = make_uint4(0, 0, 0, 0);
          }
        }
      }
    }
    if constexpr (KF == 1) {
      const int tok = tid >> 2, q4 = tid & 3;
      const int s = tok < nval ? kv_slot(p.kv_indices, t0 + tok) : 0;
      const uint8_t* srow = p.k_scales + (int64_t)s * p.k_scale_stride;
#pragma unroll
      for (int j = 0; j < 5; ++j) {
        const int blk = q4 + 4 * j;
        sr[j] = (tok < nval && blk < kMxBlocks) ? (uint32_t)srow[blk] : 127u;
      }
    }
  };

  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < C::KIT; ++i) {
      const int k = tid + 256 * i;
      if (k >= C::KITEMS) continue;
      const int tq = k / C::KCH, ch = k - tq * C::KCH;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *reinterpret_cast<uint4*>(Klds + (4 * tq + r) * C::KST + 16 * ch) = kr[i][r];
      if constexpr (VF == 0) {
        if (ch < 32) {  // latent dims 16ch .. 16ch+15 -> V^T[d][token]
          const uint32_t* x0 = reinterpret_cast<const uint32_t*>(&kr[i][0]);
          const uint32_t* x1 = reinterpret_cast<const uint32_t*>(&kr[i][1]);
          const uint32_t* x2 = reinterpret_cast<const uint32_t*>(&kr[i][2]);
          const uint32_t* x3 = reinterpret_cast<const uint32_t*>(&kr[i][3]);
#pragma unroll
          for (int wd = 0; wd < 4; ++wd) {
            uint32_t y[4];
            transpose4x4_bytes(x0[wd], x1[wd], x2[wd], x3[wd], y);
#pragma unroll
            for (int e = 0; e < 4; ++e)
              *reinterpret_cast<uint32_t*>(Vt + (16 * ch + 4 * wd + e) * C::VTST + 4 * tq) = y[e];
          }
        }
      }
      if constexpr (VF == 2) {
        if (ch < 16) {  // latent dims 32ch .. 32ch+31, scale block ch
          // e8m0 of block ch for the quad's 4 tokens (written to LDS by store_scales)
          float sc[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) sc[r] = e8m0_to_f32(Slds[(4 * tq + r) * 20 + ch]);
#pragma unroll
          for (int wd = 0; wd < 4; ++wd) {
            // word wd of each token row holds dims 32ch + 8wd .. +7 (4 bytes)
            uint32_t xw[4] = {reinterpret_cast<const uint32_t*>(&kr[i][0])[wd],
                              reinterpret_cast<const uint32_t*>(&kr[i][1])[wd],
                              reinterpret_cast<const uint32_t*>(&kr[i][2])[wd],
                              reinterpret_cast<const uint32_t*>(&kr[i][3])[wd]};
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
              const int d0 = 32 * ch + 8 * wd + 2 * bt;  // even dim, d0 + 1 odd
              uint2 ev = make_uint2(__builtin_amdgcn_perm(bf[1][bt], bf[0][bt], 0x05040100u),
                                    __builtin_amdgcn_perm(bf[3][bt], bf[2][bt], 0x05040100u));
              uint2 od = make_uint2(__builtin_amdgcn_perm(bf[1][bt], bf[0][bt], 0x07060302u),
                                    __builtin_amdgcn_perm(bf[3][bt], bf[2][bt], 0x07060302u));
              *reinterpret_cast<uint2*>(Vt + d0 * C::VTST + 2 * 4 * tq) = ev;
              *reinterpret_cast<uint2*>(Vt + (d0 + 1) * C::VTST + 2 * 4 * tq) = od;
            }
          }
        }
      }
    }
    if constexpr (VF == 1) {
#pragma unroll
      for (int i = 0; i < C::VIT; ++i) {
        const int k = tid + 256 * i;
        const int tq = k >> 5, ch = k & 31;
        const uint32_t* x0 = reinterpret_cast<const uint32_t*>(&vr[i][0]);
        const uint32_t* x1 = reinterpret_cast<const uint32_t*>(&vr[i][1]);
        const uint32_t* x2 = reinterpret_cast<const uint32_t*>(&vr[i][2]);
        const uint32_t* x3 = reinterpret_cast<const uint32_t*>(&vr[i][3]);
#pragma unroll
        for (int wd = 0; wd < 4; ++wd) {
          uint32_t y[4];
          transpose4x4_bytes(x0[wd], x1[wd], x2[wd], x3[wd], y);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            *reinterpret_cast<uint32_t*>(Vt + (16 * ch + 4 * wd + e) * C::VTST + 4 * tq) = y[e];
        }
      }
    }
  };

  auto store_scales = [&]() {
    if constexpr (KF == 1) {
      const int tok = tid >> 2, q4 = tid & 3;
#pragma unroll
      for (int j = 0; j < 5; ++j) {
        const int blk = q4 + 4 * j;
        if (blk < 20) Slds[tok * 20 + blk] = (uint8_t)sr[j];
      }
    }
  };

  const int ntok = t_end - t_beg;
  if (ntok > 0) load_tile(t_beg, min(kTile, ntok));

  for (int t0 = 0; t0 < ntok; t0 += kTile) {
    const int nval = min(kTile, ntok - t0);
    store_scales();
    if constexpr (VF == 2) __syncthreads();  // V dequant reads the scale copy
    store_tile();
    __syncthreads();                          // (A) tile visible
    if (t0 + kTile < ntok) load_tile(t_beg + t0 + kTile, min(kTile, ntok - t0 - kTile));

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
      const uint32_t pk = pack4_fp8(pv[0] * kPScale, pv[1] * kPScale, pv[2] * kPScale, pv[3] * kPScale);
      *reinterpret_cast<uint32_t*>(Pl + l16 * C::PST + 16 * w + 4 * g) = pk;
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
        const long bq = *reinterpret_cast<const long*>(Pl + l16 * C::PST + 32 * j + 8 * g);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const int d = 128 * w + 16 * dt + l16;
          const long av = *reinterpret_cast<const long*>(Vt + d * C::VTST + 32 * j + 8 * g);
          o[dt] = mfma16x32_f8(av, bq, o[dt]);
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
  }

  // ---- finish: row sums across lanes and waves --------------------------------
  float l = l_run;
  l += shfl_xor_f(l, 16);
  l += shfl_xor_f(l, 32);
  if (g == 0) lsum[w * 16 + l16] = l;
  __syncthreads();
  const float L = lsum[l16] + lsum[16 + l16] + lsum[32 + l16] + lsum[48 + l16];
  const float inv = L > 0.f ? vscale / L : 0.f;
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
    if (w == 0 && g == 0) p.part_lse[(int64_t)slot * 16 + head] = L > 0.f ? m_run + __log2f(L) : neg_inf();
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
  static constexpr int KCH = KROW / 16;
  static constexpr int KST = KROW + 16;
  static constexpr int VTST = 80;  // 64 token bytes + 16 pad per latent dim
  static constexpr int OFF_K = 0;
  static constexpr int OFF_S = OFF_K + kTile * KST;
  static constexpr int OFF_VT = OFF_S + (KF == 1 ? kTile * 20 : 0);
  static constexpr int OFF_Q = OFF_VT + kVDim * VTST;      // [128][576], 16-B chunks swizzled
  static constexpr int OFF_P = OFF_Q + 128 * kQKDim;       // [4 groups][64 lanes][32 B]
  static constexpr int OFF_MAX = OFF_P + 4 * 64 * 32;      // [2 halves][128] f32
  static constexpr int OFF_L = OFF_MAX + 2 * 128 * 4;      // [2 halves][128] f32
  static constexpr int LDS = OFF_L + 2 * 128 * 4;
  static constexpr int NT = 512;
  static constexpr int KITEMS = 16 * KCH;
  static constexpr int KIT = (KITEMS + NT - 1) / NT;
  static constexpr int VITEMS = KF == 1 ? 16 * 32 : 0;
  static constexpr int VIT = (VITEMS + NT - 1) / NT;
};

// V^T byte offset of token quad tq (tokens 4tq..4tq+3) in a latent-dim row: the
// order matches the P operand built from the 32x32 score accumulators, where
// lane half hh holds tokens 32u + 8q + 4hh + i as byte 16u + 4q + i.
__device__ __forceinline__ int vt128_quad_off(int tq) {
  return 32 * (tq & 1) + 16 * (tq >> 3) + 4 * ((tq & 7) >> 1);
}
// Q chunk swizzle: 16-byte chunk c of head row h lives at chunk c ^ (h & 7)
__device__ __forceinline__ int q_off(int h, int c) { return h * kQKDim + 16 * (c ^ (h & 7)); }

template <int KF>
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
      *reinterpret_cast<uint4*>(Qlds + q_off(h, ch)) =
          *reinterpret_cast<const uint4*>(qb + h * kQKDim + 16 * ch);
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

  uint4 kr[C::KIT][4];
  uint4 vr[C::VIT > 0 ? C::VIT : 1][4];
  uint32_t sr[3];  // fp4 K scales: token tid>>3, blocks (tid&7) + 8j

  auto load_tile = [&](int t0, int nval) {
#pragma unroll
    for (int i = 0; i < C::KIT; ++i) {
      const int k = tid + C::NT * i;
      const int tq = k / C::KCH, ch = k - tq * C::KCH;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tok = 4 * tq + r;
        if (k < C::KITEMS && tok < nval) {
          const int s = kv_slot(p.kv_indices, t0 + tok);
          kr[i][r] = ldg16(p.k_cache + (int64_t)s * p.k_row_stride + 16 * ch);
        } else {
          kr[i][r] = make_uint4(0, 0, 0, 0);
        }
      }
    }
    if constexpr (KF == 1) {
#pragma unroll
      for (int i = 0; i < C::VIT; ++i) {
        const int k = tid + C::NT * i;
        const int tq = k >> 5, ch = k & 31;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tok = 4 * tq + r;
          if (tok < nval) {
            const int s = kv_slot(p.kv_indices, t0 + tok);
            vr[i][r] = ldg16(p.v_cache + (int64_t)s * p.v_row_stride + 16 * ch);
          } else {
            vr[i][r] = make_uint4(0, 0, 0, 0);
          }
        }
      }
      const int tok = tid >> 3, q8 = tid & 7;
      const int s = tok < nval ? kv_slot(p.kv_indices, t0 + tok) : 0;
      const uint8_t* srow = p.k_scales + (int64_t)s * p.k_scale_stride;
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const int blk = q8 + 8 * j;
        sr[j] = (tok < nval && blk < kMxBlocks) ? (uint32_t)srow[blk] : 127u;
      }
    }
  };

  auto vt_store = [&](const uint4 (&x)[4], int tq, int ch) {
    const uint32_t* x0 = reinterpret_cast<const uint32_t*>(&x[0]);
    const uint32_t* x1 = reinterpret_cast<const uint32_t*>(&x[1]);
    const uint32_t* x2 = reinterpret_cast<const uint32_t*>(&x[2]);
    const uint32_t* x3 = reinterpret_cast<const uint32_t*>(&x[3]);
    const int qo = vt128_quad_off(tq);
#pragma unroll
    for (int wd = 0; wd < 4; ++wd) {
      uint32_t y[4];
      transpose4x4_bytes(x0[wd], x1[wd], x2[wd], x3[wd], y);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        *reinterpret_cast<uint32_t*>(Vt + (16 * ch + 4 * wd + e) * C::VTST + qo) = y[e];
    }
  };

  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < C::KIT; ++i) {
      const int k = tid + C::NT * i;
      if (k >= C::KITEMS) continue;
      const int tq = k / C::KCH, ch = k - tq * C::KCH;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *reinterpret_cast<uint4*>(Klds + (4 * tq + r) * C::KST + 16 * ch) = kr[i][r];
      if constexpr (KF == 0) {
        if (ch < 32) vt_store(kr[i], tq, ch);
      }
    }
    if constexpr (KF == 1) {
#pragma unroll
      for (int i = 0; i < C::VIT; ++i) {
        const int k = tid + C::NT * i;
        vt_store(vr[i], k >> 5, k & 31);
      }
      const int tok = tid >> 3, q8 = tid & 7;
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const int blk = q8 + 8 * j;
        if (blk < 20) Slds[tok * 20 + blk] = (uint8_t)sr[j];
      }
    }
  };

  const int ntok = t_end - t_beg;
  if (ntok > 0) load_tile(t_beg, min(kTile, ntok));

  for (int t0 = 0; t0 < ntok; t0 += kTile) {
    const int nval = min(kTile, ntok - t0);
    store_tile();
    __syncthreads();  // (A) tile (and Q) visible
    if (t0 + kTile < ntok) load_tile(t_beg + t0 + kTile, min(kTile, ntok - t0 - kTile));

    // ---- scores S^T for tokens 32*half .. +31 of this tile, heads of g4 -------
    v16f s = v16f{};
    const int trow = 32 * half + l32;
#pragma unroll
    for (int ks = 0; ks < 9; ++ks) {
      const int qc = 4 * ks + 2 * hh;  // Q chunks qc, qc+1 of this lane's head
      v8i qf;
      {
        const uint4 a = *reinterpret_cast<const uint4*>(Qlds + q_off(head, qc));
        const uint4 bq = *reinterpret_cast<const uint4*>(Qlds + q_off(head, qc + 1));
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
      uint4 pk;
      pk.x = pack4_fp8(s[0] * kPScale, s[1] * kPScale, s[2] * kPScale, s[3] * kPScale);
      pk.y = pack4_fp8(s[4] * kPScale, s[5] * kPScale, s[6] * kPScale, s[7] * kPScale);
      pk.z = pack4_fp8(s[8] * kPScale, s[9] * kPScale, s[10] * kPScale, s[11] * kPScale);
      pk.w = pack4_fp8(s[12] * kPScale, s[13] * kPScale, s[14] * kPScale, s[15] * kPScale);
      *reinterpret_cast<uint4*>(Pex + (g4 * 64 + lane) * 32 + 16 * half) = pk;
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] *= alpha;
    __syncthreads();  // (C) both halves of P visible
    const v8i pb = ld_v8(Pex + (g4 * 64 + lane) * 32);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int d = 256 * half + 32 * dt + l32;
      o[dt] = mfma32_f8(ld_v8(Vt + d * C::VTST + 32 * hh), pb, o[dt]);
    }
    __syncthreads();  // (D) LDS free for the next tile
  }

  // ---- finish: row sum over both lane halves and both half-waves ---------------
  float l = l_run + shfl_xor_f(l_run, 32);
  if (hh == 0) lsum[half * 128 + head] = l;
  __syncthreads();
  const float L = lsum[head] + lsum[128 + head];
  const float inv = L > 0.f ? vscale / L : 0.f;
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
    if (hh == 0 && half == 0) p.part_lse[(int64_t)slot * 128 + head] = L > 0.f ? m_run + __log2f(L) : neg_inf();
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
hipError_t launch_decode(const DecodeParams& p, int kv_mode, int grid, hipStream_t stream) {
  if (p.num_heads == 16) {
    switch (kv_mode) {
      case 0: hipLaunchKernelGGL((decode_h16_kernel<0, 0>), dim3(grid), dim3(256), 0, stream, p); break;
      case 1: hipLaunchKernelGGL((decode_h16_kernel<1, 2>), dim3(grid), dim3(256), 0, stream, p); break;
      case 2: hipLaunchKernelGGL((decode_h16_kernel<1, 1>), dim3(grid), dim3(256), 0, stream, p); break;
      default: return hipErrorInvalidValue;
    }
  } else if (p.num_heads == 128) {
    switch (kv_mode) {
      case 0: hipLaunchKernelGGL((decode_h128_kernel<0>), dim3(grid), dim3(512), 0, stream, p); break;
      case 2: hipLaunchKernelGGL((decode_h128_kernel<1>), dim3(grid), dim3(512), 0, stream, p); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_combine(const DecodeParams& p, hipStream_t stream) {
  hipLaunchKernelGGL(combine_kernel, dim3(p.batch, p.num_heads / 16), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mla
