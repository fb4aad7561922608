// Split-KV MLA absorbed decode for gfx950 with 16 heads, the launch switch for
// every head count and cache mode, and the log-sum-exp split combine.
//
// One work-group (4 waves) runs one work item {batch, token range, slot} from
// the on-device plan.  Cache rows are gathered by kv_indices (page tables are
// expanded to that form beforehand) straight from HBM into an LDS ring by
// LDS-DMA, slot indices one tile ahead of the rows they address.  Both
// products run on MFMA:
//   scores  S^T = K . Q^T   K = A operand from LDS, Q = B operand in registers
//   output  O^T = V^T . P^T V^T = A operand from LDS (transpose reads), P = B
// so every lane's accumulators belong to a single head and the softmax state
// is a per-lane scalar.  H = 16 runs here (below); H = 128 gives each wave 32
// heads of its own (decode_h128.hip).
//
// Numerics: scores are accumulated in f32 from the fp8/fp4/bf16 operands and
// scaled by q_scale * k_scale * sm_scale * log2(e); the softmax uses exp2 with
// a fixed per-item reference.  P enters the PV product as two fp8 terms (fp8
// V), or as bf16 (fp4 or bf16 V).  The row sum uses the f32 P.
//
// Behavioural reference: mixed-mla/asm_dumps/aiter_mla.py:149-470 (interface),
// mixed-mla/submission.py:122-250 (split-K online softmax), V5
// mixed-mla/versions/hip_mxfp4_v5/submission.py:214-714 (split + reduce).
#include <type_traits>

#include "mla_internal.hpp"
#include "mla_plan.hpp"

namespace mla {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kPScale = 256.0f;  // fp8 P = p * 256
constexpr float kRebase = 96.0f;   // max log2 distance of a tile max above the fixed reference

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

// waits until at most k groups of PER operations issued after the one waited
// for are still outstanding (k in 0..2: at most the ring depth minus one, S <= 3)
template <int PER>
__device__ __forceinline__ void wait_groups(int k) {
  if (k <= 0) wait_vmcnt<0>();
  else if (k == 1) wait_vmcnt<PER>();
  else wait_vmcnt<2 * PER>();
}

// ============================================================================
// H = 16.  4 waves; per 64-token tile wave w scores 16 tokens for all 16
// heads (16x16x128 MFMAs, Q^T in registers) and accumulates O^T for latent
// dims 128w .. 128w+127 over all 64 tokens.  Cache rows arrive by LDS-DMA in
// an S-stage ring (slots one tile ahead of the rows they address).
//   KF: 0 = fp8 K rows (576 B), 1 = packed fp4 K rows (288 B) + e8m0 scales
//   VF: 0 = fp8 V = K rows, 1 = fp8 V from its own cache, 2 = fp4 V = K rows
// fp8 V: P^T enters a block-scaled 16x16x128 MFMA as two fp8 terms whose e8m0
// B scale carries 2^(m_w - m_ref - 8): m_w is the wave's own (ceil) max for the
// head, m_ref a per-item reference, so no cross-wave max and no rescale of
// O^T per tile.  The A operand (V^T) comes from the row-major tile through
// ds_read_b64_tr_b8; K block g of the MFMA holds wave g's 16 tokens (+16 zeros).
// fp4 V: no dequantized copy of the tile.  Each wave reads its V^T fragments
// straight from the packed rows with ds_read_b64_tr_b4 (16 tokens of one latent
// dim per lane), widens the e2m1 codes to bf16 unscaled, and folds each token's
// e8m0 block scale into P instead: P'_j = P * 2^(e[t, j] - E_ref) for MX block j,
// with P = 2^(s - m_ref) in f32 shared through LDS and E_ref a per-item
// reference exponent; O^T is rescaled by 2^(E_ref - 127) at the end.  PV runs on
// 16x16x32 bf16 MFMAs.  The LDS this frees lets two work-groups share a CU.
// A tile max more than kRebase above m_ref, or (fp4 V) a V block exponent more
// than kVScaleSpan above E_ref, restarts the item from a higher reference
// (block-wide vote), so neither the accumulators nor P' can overflow.
// ============================================================================
// KF / VF: 0 / 0 fp8 K = V, 1 / 2 fp4 K = V, 1 / 1 fp4 K + fp8 V, 2 / 3 bf16 K =
// V (a16w16: 1152-byte rows, V = their first 512 dims; QK and PV on 16x16x32
// bf16 MFMAs, the V^T operand by ds_read_b64_tr_b16).
template <int KF, int VF>
struct H16 {
  static constexpr int KROW = KF == 0 ? 576 : (KF == 1 ? 288 : 1152);
  static constexpr int KST = KROW + 16;                        // LDS row stride: 592 / 304 / 1168
  static constexpr int KCPR = KST / 16;                        // 16-B chunks per LDS row: 37 / 19 / 73
  static constexpr int KCH = KROW / 16;                        // real chunks: 36 / 18 / 72
  static constexpr int VST = 528, VCPR = 33;                   // fp8 V rows (VF == 1): 512 B used
  static constexpr int KW = kTile * KST / 1024;                // 1-KiB DMA windows of K rows: 37 / 19
  static constexpr int VW = VF == 1 ? kTile * VST / 1024 : 0;  // of V rows: 33
  static constexpr int NW = KW + VW;
  static constexpr int STAGE = NW * 1024;
  // ring depth (tiles).  fp8 K = V: two stages; fp4 K = V: three stages of rows
  // and scales.  Both fit two work-groups per CU (LDS <= 80 KiB, <= 256
  // registers a wave), whose eight waves keep twice the row gathers in flight
  // and overlap one group's compute with the other's waits.  fp4 K + fp8 V
  // (two caches) runs one work-group per CU.
  static constexpr int S = KF != 1 ? 2 : (VF == 1 ? 2 : 3);
  static constexpr int BLOCKS_PER_CU = (VF == 1 || KF == 2) ? 1 : 2;
  // DMA issue: waves RW0..3 gather rows.  fp4 K + fp8 V: wave 0 gathers the
  // 18 scale bytes of every token (SCW = 1); fp4 K = V: every wave gathers rows
  // and scale dword columns j = w + 4k (SCW = 4), so no wave issues a long burst
  static constexpr int RW0 = (KF == 1 && VF == 1) ? 1 : 0;
  static constexpr int SCW = KF == 0 ? 0 : (VF == 1 ? 1 : 4);
  static constexpr int NRW = 4 - RW0;
  static constexpr int NA = (NW + NRW - 1) / NRW;              // windows per row wave: NA or NA - 1
  static constexpr int NAW = NW % NRW == 0 ? NRW : NW % NRW;   // row waves (from RW0) that issue NA
  static constexpr bool VB16 = VF == 2;                        // fp4 V, bf16 PV from registers
  static constexpr bool P32 = VF >= 2;                         // P shared as f32 [head][token] (bf16 PV)
  static constexpr int PST = 68;                               // f32 P row stride (P32): 64 tokens + 4
  static constexpr int NSL = 2 * S;                            // slot stages (slots lead rows by S tiles)
  static constexpr int OFF_SLOT = S * STAGE;                   // [NSL][64] int32 cache slots
  static constexpr int SCST = kScWin * 256;                    // e8m0 stage: [5][64 tokens] dwords
  static constexpr int OFF_SC = OFF_SLOT + NSL * 256;          // [S] e8m0 stages (KF == 1)
  static constexpr int OFF_P = OFF_SC + (KF == 1 ? S * SCST : 0);
  static constexpr int P_BYTES = P32 ? 16 * PST * 4 : 2 * 4 * 16 * 16;  // f32 [h][token] | fp8 [term][g][h][16]
  static constexpr int OFF_PS = OFF_P + P_BYTES;               // [g][h] e8m0 B scales
  static constexpr int OFF_X = OFF_PS + 64;                    // [4][16] f32 exchange
  static constexpr int OFF_E = OFF_X + 256;                    // [4] int exchange (V block exponents)
  static constexpr int OFF_VOTE = OFF_E + 16;
  static constexpr int LDS = OFF_VOTE + 16;
  static_assert(BLOCKS_PER_CU == 1 || LDS <= 80 * 1024, "two work-groups per CU");
};
constexpr int kVScaleSpan = 31;  // fp4 V: P' = P 2^(e - E_ref) <= 2^(96 + 31) stays finite in bf16


// QM: how Q arrives.  0: fp8 codes and their per-tensor scale (the staged
// path).  1: bf16, quantized here per tensor from the amax partials (a8w8).
// 2: bf16 with no tensor-wide scale (a16w8, fp8 K only): each head row is
// split here into two fp8 terms at a power-of-two row scale 2^e, hi =
// e4m3(q 2^-e) and lo = e4m3((q 2^-e - hi) 2^4), and QK runs one MFMA per term
// (the lo one with B scale 2^-4), about 8 significant bits of Q as bf16 has.
// 3: bf16, used as it is (a16w16, bf16 K).  4: bf16, quantized here per
// head row (the per-tensor rule with the row as the tensor; fp8 or fp4 K), so
// no tensor-wide amax pass has to run first.  5: as 4, the work-group's item
// planned here by the block (65 to 256 query rows).
template <int KF, int VF, bool IDX, int QM>
__global__ __launch_bounds__(256, (H16<KF, VF>::BLOCKS_PER_CU)) void decode_h16_kernel(const DecodeParams p) {
  using C = H16<KF, VF>;
  constexpr bool QB = QM != 0;
  static_assert(QM != 2 || KF == 0, "a16w8: fp8 K only");
  static_assert((QM == 3) == (KF == 2), "a16w16: bf16 Q with bf16 K");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[C::LDS];
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;

  const int32_t* plan = p.plan;
  int4 it;
  if (QM == 5 || (QM == 4 && p.plan_here)) {  // only the per-row Q route plans here
    // QM 4, up to 64 rows: wave 0 plans in registers and takes this
    // work-group's item; QM 5, up to 256: the block plans (its scratch on the
    // ring, which nothing has written yet) and the thread of the item's row
    // takes it (a variant of its own, so that the small batches' kernel does
    // not carry the block planner's code).  Work-group 0 also writes what the
    // combine reads of the plan.
    __shared__ int4 s_item;
    if constexpr (QM == 4) {
      if ((threadIdx.x >> 6) == 0) {
        const WavePlan P = plan_wave(p.kv_indptr, p.batch, p.plan_qlen, p.plan_target, p.plan_min_chunk,
                                     p.plan_max_splits);
        if (blockIdx.x == 0) plan_wave_write_rows(P, p.batch, p.max_items, const_cast<int32_t*>(plan));
        const int4 mine = plan_wave_item_uniform(P, (int)blockIdx.x);
        if ((threadIdx.x & 63) == 0) s_item = mine;
      }
    } else {
      const BlockPlan P = plan_block(p.kv_indptr, p.batch, p.plan_qlen, p.plan_target, p.plan_min_chunk,
                                     p.plan_max_splits, reinterpret_cast<uint64_t*>(smem),
                                     reinterpret_cast<int*>(smem + 2048), reinterpret_cast<int*>(smem + 3072));
      const int tid = threadIdx.x, i = blockIdx.x;
      if (blockIdx.x == 0) {
        int32_t* pl = const_cast<int32_t*>(plan);
        if (tid < p.batch) reinterpret_cast<int2*>(pl + kPlanHeader + 4 * p.max_items)[tid] = make_int2(P.first, P.nb);
        if (tid == 0) {
          pl[0] = P.n_items;
          pl[1] = P.chunk;
          pl[2] = (int)(64u * P.hi64 + P.lo64);
          pl[3] = p.batch;
          pl[4] = p.max_items;
        }
      }
      if (tid == 0 && i >= P.n_items) s_item = make_int4(-1, 0, 0, -1);
      if (tid < p.batch && P.first <= i && i < P.first + P.nb) {  // piece j of this row, as the planner emits it
        const unsigned j = (unsigned)(i - P.first), n = (unsigned)P.nb;
        const unsigned q = (unsigned)P.L / n, r = (unsigned)P.L - q * n;
        s_item = make_int4(tid, P.s0 + (int)(j * q + (j * r) / n), P.s0 + (int)((j + 1) * q + ((j + 1) * r) / n),
                           P.nb > 1 ? i : -1);
      }
    }
    __syncthreads();
    it = s_item;
    if (it.x < 0) return;  // past the plan's items (block-uniform)
  } else {
    if ((int)blockIdx.x >= plan[0]) return;
    it = reinterpret_cast<const int4*>(plan + kPlanHeader)[blockIdx.x];
  }
  const int b = it.x, t_beg = it.y, t_end = it.z, slot = it.w;
  const int ntok = t_end - t_beg;
  const int ntiles = (ntok + kTile - 1) / kTile;

  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (feeds M0)
  const int lane = tid & 63, l16 = lane & 15, g = lane >> 4;

  auto tok_of = [](int gg, int i) { return 16 * gg + i; };  // tile token of row i of wave gg's slice

  // ---- ring issue ----------------------------------------------------------
  // slots of tile t live in slot stage t % NSL
  auto slot_of = [&](int t, int tok) -> int __attribute__((always_inline)) {
    if constexpr (IDX) return reinterpret_cast<const int*>(smem + C::OFF_SLOT + (t % C::NSL) * 256)[tok];
    else return min(t_beg + kTile * t + tok, t_end - 1);
  };
  auto issue_slots = [&](int t) __attribute__((always_inline)) {  // wave 0: the 64 slots of tile t (positions clamped into the item)
    if constexpr (IDX) {
      if (w == 0) {
        const int pos = min(t_beg + kTile * t + lane, t_end - 1);
        dma4_to_lds(p.kv_indices + pos, lds0 + C::OFF_SLOT + (t % C::NSL) * 256);
      }
    }
  };
  auto issue_rows = [&](int t) __attribute__((always_inline)) {  // row waves: windows u = (w - RW0) + NRW k of tile t
    if (w < C::RW0) return;
    const int st = t % C::S;
    const uint32_t sbase = lds0 + st * C::STAGE;
    // all slot reads first: each DMA below is an asm barrier for memory ops
    int sl[C::NA], co[C::NA];
#pragma unroll
    for (int k = 0; k < C::NA; ++k) {
      const int u = (w - C::RW0) + C::NRW * k;
      if (u < C::KW) {
        const int e = 64 * u + lane;  // 16-B chunk index within the stage
        const int tok = e / C::KCPR, ch = e - tok * C::KCPR;
        sl[k] = slot_of(t, tok);
        co[k] = 16 * min(ch, C::KCH - 1);
      } else if (u < C::NW) {
        const int e = 64 * (u - C::KW) + lane;
        const int tok = e / C::VCPR, ch = e - tok * C::VCPR;
        sl[k] = slot_of(t, tok);
        co[k] = 16 * min(ch, 31);
      }
    }
#pragma unroll
    for (int k = 0; k < C::NA; ++k) {
      const int u = (w - C::RW0) + C::NRW * k;
      // slot x stride in one v_mad_u64_u32 (both below 2^31, checked on the host)
      if (u < C::KW)
        dma16_to_lds_nt(p.k_cache + ((uint64_t)(uint32_t)sl[k] * (uint32_t)p.k_row_stride + (uint32_t)co[k]),
                     sbase + 1024 * u);
      else if (u < C::NW)
        dma16_to_lds_nt(p.v_cache + ((uint64_t)(uint32_t)sl[k] * (uint32_t)p.v_row_stride + (uint32_t)co[k]),
                     sbase + 1024 * u);
    }
  };
  // fp4 K scales: the 18 e8m0 bytes of token `lane` of tile t as 5 dwords
  // (kScWin), dword j = blocks 4j .. 4j + 3 (j < 4) and blocks 14 .. 17 (j =
  // 4, from byte 14: every read stays inside the row); dword j lands at
  // j * 64 + lane of the tile's scale stage.  A row starts at any byte (the
  // scale stride is free), so these are unaligned dword reads, which gfx950
  // serves for global memory.  Columns j = w + SCW k are this wave's.
  auto issue_scales = [&](int t) __attribute__((always_inline)) {
    if constexpr (KF == 1) {
      if (w < C::SCW) {
        const uint8_t* srow = p.k_scales + (uint64_t)(uint32_t)slot_of(t, lane) * (uint32_t)p.k_scale_stride;
        const uint32_t sb = lds0 + C::OFF_SC + (t % C::S) * C::SCST;
#pragma unroll
        for (int k = 0; k < (kScWin + C::SCW - 1) / C::SCW; ++k) {
          const int j = w + C::SCW * k;
          if (j < kScWin) dma4_to_lds(srow + (j < 4 ? 4 * j : 14), sb + 256 * j);
        }
      }
    }
  };
  // this wave's wait for tile t's rows (and scales), k groups issued after them
  auto wait_tile = [&](int k) __attribute__((always_inline)) {
    constexpr int SL = IDX ? 1 : 0;  // wave 0 issues one slot DMA per group
    if constexpr (KF == 1 && C::SCW == 4) {
      // rows: NA for waves < NAW, else NA - 1; scale columns: 2 for wave 0, else 1
      static_assert(C::RW0 == 0 && C::NAW == 3 && kScWin == 5, "per-wave DMA counts");
      if (w == 0) wait_groups<C::NA + 2 + SL>(k);
      else if (w == 1) wait_groups<C::NA + 1>(k);
      else if (w == 2) wait_groups<C::NA + 1>(k);
      else wait_groups<C::NA - 1 + 1>(k);
    } else if constexpr (KF == 1) {
      // wave 0: one slot DMA + the 5 scale DMAs per group
      if (w == 0) wait_groups<kScWin + SL>(k);
      else if (w - C::RW0 < C::NAW) wait_groups<C::NA>(k);
      else wait_groups<C::NA - 1>(k);
    } else {
      if (w == 0) wait_groups<C::NA + SL>(k);
      else if (w < C::NAW) wait_groups<C::NA>(k);
      else wait_groups<C::NA - 1>(k);
    }
  };
  // group x = {slots(x + S), rows(x) | scales(x)}.  The prologue issues groups
  // 0 .. S-1 (every stage is free then, so the first S tiles are in flight
  // together: a short item pays one row round trip, not one per tile); the
  // pass of tile t >= 1 issues group t + S - 1 into the stage tile t - 1 used.
  // The slots of tile x arrive with group x - S (the prologue's wait covers
  // tiles 0 .. S-1), one barrier before the rows that read them are issued.
  // The first slot indices are in flight while Q is loaded (and quantized).
  if (ntiles > 0) {
#pragma unroll
    for (int j = 0; j < C::S; ++j) issue_slots(j);
  }

  // ---- Q^T (B operand): head l16, dims 128ks + 32g .. +31 -------------------
  // With fp4 K, the f8f6f4 MFMA pairs fp4 element e of lane group g (K =
  // 32g + e within the 128-step, one MX block) with fp8 byte i of lane group
  // g' where 32g + e = 16g' + (i & 15) + 64 (i >> 4); the fp8 Q operand is
  // gathered in that order.  With fp8 K both operands share one order.
  v8i qv[5];
  v8i qlo[QM == 2 ? 5 : 1];  // a16w8: the lo term of Q
  v8bf qbf[QM == 3 ? 18 : 1];  // a16w16: Q^T bf16, K-step ks = dims 32ks + 8g .. +7
  float c = 0.f;  // qs * kv scale (fp8 K) * sm_scale * log2(e), set once Q is resident
  const float kvs = (KF == 0 || VF == 1) ? p.kv_scale[0] : 1.0f;
  const float vscale = VF == 2 ? 1.0f : kvs;
  auto load_q = [&](const uint8_t* qrow) __attribute__((always_inline)) {
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
  };
  // QB: Q is quantized here, bit-exact with the quant kernel.  This sequence's
  // 16 x 576 bf16 Q (18 KiB) is gathered by LDS-DMA into the last ring stage
  // and the per-tensor amax partials are loaded, in flight with the first slot
  // indices; quantize_q folds the scale and quantizes in place once the first
  // prologue has issued the rows of every other stage, and the fp8 Q fragments
  // are read before the last stage's rows are issued.
  constexpr int QNV = 16 * kQKDim / 8, QNJ = (QNV + 255) / 256;  // 16-B bf16 chunks, per thread
  static_assert(C::STAGE >= 16 * kQKDim * 2, "bf16 Q fits one ring stage");
  const uint32_t qlds = lds0 + (C::S - 1) * C::STAGE;
  uint32_t qm = 0;
  if constexpr (QB) {
    const uint8_t* src = reinterpret_cast<const uint8_t*>(p.q_bf16 + (int64_t)b * 16 * kQKDim);
    for (int k = w; k < QNV / 64; k += 4) dma16_to_lds(src + 1024 * k + 16 * lane, qlds + 1024 * k);
    if constexpr (QM == 1)
      for (int i = tid; i < p.q_nparts; i += 256) qm = max(qm, p.q_partials[i]);
    (void)qm;
  } else {
    load_q(p.q_fp8 + ((int64_t)b * 16 + l16) * kQKDim);
    c = p.q_scale[0] * (KF == 0 ? kvs : 1.0f) * p.sm_scale * kLog2e;
  }
  auto quantize_q = [&]() __attribute__((always_inline)) {  // block-uniform; the loads have landed
    if constexpr (QM == 3) {
      const uint8_t* qrow = smem + (C::S - 1) * C::STAGE + l16 * (2 * kQKDim) + 16 * g;
#pragma unroll
      for (int ks = 0; ks < 18; ++ks) qbf[ks] = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4*>(qrow + 64 * ks));
#pragma unroll
      for (int ks = 0; ks < 18; ++ks) asm volatile("" : "+v"(qbf[ks]));  // keep resident, no reload
      c = p.sm_scale * kLog2e;
      lds_barrier();  // every wave holds its fragments before the stage is refilled
    } else if constexpr (QM == 2) {
      // per head row: |q| max (bf16 bits) -> row exponent e (q 2^-e <= 448),
      // then both terms written over the bf16 rows (hi at row r, lo 9 KiB on)
      uint8_t* qst = smem + (C::S - 1) * C::STAGE;
      uint32_t* rmax = reinterpret_cast<uint32_t*>(smem + C::OFF_X);  // [16] row maxima, then exponents
      if (tid < 16) rmax[tid] = 0;
      uint4 xv[QNJ];
#pragma unroll
      for (int j = 0; j < QNJ; ++j) {
        const int i = tid + 256 * j;
        if (i < QNV) xv[j] = *reinterpret_cast<const uint4*>(qst + 16 * i);
      }
      lds_barrier();  // rmax zeroed
#pragma unroll
      for (int j = 0; j < QNJ; ++j) {
        const int i = tid + 256 * j;
        if (i < QNV) {
          const uint32_t wv[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
          uint32_t m = 0;
#pragma unroll
          for (int k = 0; k < 4; ++k) m = max(m, max(wv[k] & 0x7FFFu, (wv[k] >> 16) & 0x7FFFu));
          atomicMax(&rmax[i / (kQKDim / 8)], m);
        }
      }
      lds_barrier();  // row maxima complete; every bf16 chunk read before the fp8 terms overwrite them
      if (tid < 16) {
        const float a = bf16_bits_to_f32(rmax[tid]);
        int e = a > 0.f ? (int)__builtin_ceilf(__log2f(a * (1.0f / 448.0f))) : 0;
        e = min(max(e, -126), 126);
        if (a * __builtin_amdgcn_ldexpf(1.0f, -e) > 448.0f) ++e;  // log2 rounding
        rmax[16 + tid] = (uint32_t)e;
      }
      lds_barrier();
#pragma unroll
      for (int j = 0; j < QNJ; ++j) {
        const int i = tid + 256 * j;
        if (i < QNV) {
          const float sc = __builtin_amdgcn_ldexpf(1.0f, -(int)rmax[16 + i / (kQKDim / 8)]);
          const uint32_t wv[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
          float y[8];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            y[2 * k] = bf16_bits_to_f32(wv[k] & 0xFFFFu) * sc;
            y[2 * k + 1] = bf16_bits_to_f32(wv[k] >> 16) * sc;
          }
          const uint32_t h0 = pack4_fp8(y[0], y[1], y[2], y[3]), h1 = pack4_fp8(y[4], y[5], y[6], y[7]);
          const v2f a0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h0, false), a1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h0, true);
          const v2f a2 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h1, false), a3 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h1, true);
          const uint32_t l0 = pack4_fp8((y[0] - a0[0]) * 16.f, (y[1] - a0[1]) * 16.f, (y[2] - a1[0]) * 16.f,
                                        (y[3] - a1[1]) * 16.f);
          const uint32_t l1 = pack4_fp8((y[4] - a2[0]) * 16.f, (y[5] - a2[1]) * 16.f, (y[6] - a3[0]) * 16.f,
                                        (y[7] - a3[1]) * 16.f);
          *reinterpret_cast<uint2*>(qst + 8 * i) = make_uint2(h0, h1);
          *reinterpret_cast<uint2*>(qst + 16 * kQKDim + 8 * i) = make_uint2(l0, l1);
        }
      }
      lds_barrier();
      load_q(qst + l16 * kQKDim);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) qlo[ks] = ld_v8(qst + 16 * kQKDim + l16 * kQKDim + 128 * ks + 32 * g);
      qlo[4] = g < 2 ? ld_v8(qst + 16 * kQKDim + l16 * kQKDim + 512 + 32 * g) : v8i{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int ks = 0; ks < 5; ++ks) asm volatile("" : "+v"(qlo[ks]));
      c = __builtin_amdgcn_ldexpf(1.0f, (int)rmax[16 + l16]) * kvs * p.sm_scale * kLog2e;
      lds_barrier();  // every wave holds its fragments (and its row exponent) before the stage is refilled
    } else if constexpr (QM == 4 || QM == 5) {
      // per head row: the per-tensor rule with the row as the tensor (|q| max,
      // bf16 scale amax / 448), every row quantized at its own scale.  Lane
      // group (w, lane / 16) holds head row 4w + lane / 16 and its lanes the
      // 16-B chunks lane % 16 + 16k of it (72 a row): the row max is a 16-lane
      // reduction and each lane forms its row's scale once.
      uint8_t* qst = smem + (C::S - 1) * C::STAGE;
      float* rsc = reinterpret_cast<float*>(smem + C::OFF_X);  // [16] row scales
      constexpr int CPR = kQKDim / 8, NK = (CPR + 15) / 16;
      const int qrow = 4 * w + (lane >> 4), c0 = lane & 15;
      uint4 xv[NK];
      uint32_t m = 0;
#pragma unroll
      for (int k = 0; k < NK; ++k) {
        const int cc = c0 + 16 * k;
        xv[k] = cc < CPR ? *reinterpret_cast<const uint4*>(qst + 16 * (qrow * CPR + cc)) : make_uint4(0, 0, 0, 0);
        const uint32_t wv[4] = {xv[k].x, xv[k].y, xv[k].z, xv[k].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) m = max(m, max(wv[e] & 0x7FFFu, (wv[e] >> 16) & 0x7FFFu));
      }
#pragma unroll
      for (int msk = 1; msk < 16; msk <<= 1) m = max(m, (uint32_t)__shfl_xor((int)m, msk, 64));
      const Fp8Quant qq = make_fp8_quant(fp8_scale_from_amax(m));
      if (c0 == 0) rsc[qrow] = qq.s;
      lds_barrier();  // every bf16 chunk read before the fp8 rows overwrite them
#pragma unroll
      for (int k = 0; k < NK; ++k) {
        const int cc = c0 + 16 * k;
        if (cc < CPR) *reinterpret_cast<uint2*>(qst + 8 * (qrow * CPR + cc)) = quant8_fp8(xv[k], qq);
      }
      lds_barrier();
      load_q(qst + l16 * kQKDim);
      c = rsc[l16] * (KF == 0 ? kvs : 1.0f) * p.sm_scale * kLog2e;
      lds_barrier();  // every wave holds its fragments and its row's scale before the stage is refilled
    } else if constexpr (QB) {
      uint8_t* qst = smem + (C::S - 1) * C::STAGE;
      uint32_t* xu = reinterpret_cast<uint32_t*>(smem + C::OFF_X);
      const uint32_t m = (uint32_t)wave_max((int)qm);
      if (lane == 0) xu[w] = m;
      uint4 xv[QNJ];
#pragma unroll
      for (int j = 0; j < QNJ; ++j) {
        const int i = tid + 256 * j;
        if (i < QNV) xv[j] = *reinterpret_cast<const uint4*>(qst + 16 * i);
      }
      lds_barrier();  // partial maxima exchanged; every bf16 chunk read before the fp8 rows overwrite them
      const float qs = fp8_scale_from_amax(max(max(xu[0], xu[1]), max(xu[2], xu[3])));
      const Fp8Quant qq = make_fp8_quant(qs);
#pragma unroll
      for (int j = 0; j < QNJ; ++j) {
        const int i = tid + 256 * j;
        if (i < QNV) *reinterpret_cast<uint2*>(qst + 8 * i) = quant8_fp8(xv[j], qq);
      }
      lds_barrier();
      load_q(qst + l16 * kQKDim);
      lds_barrier();  // every wave holds its fragments before the stage is refilled
      c = qs * (KF == 0 ? kvs : 1.0f) * p.sm_scale * kLog2e;
    }
  };

  v4f o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = v4f{0.f, 0.f, 0.f, 0.f};
  float m_ref = 0.f, m_seen = neg_inf(), l_part = 0.f;
  bool have_ref = false;
  int e_ref = 127, e_seen = 0;  // fp4 V: reference and running max of the V block exponents

  auto prologue = [&](bool slots_issued, bool quant) __attribute__((always_inline)) {
    if (!slots_issued) {
#pragma unroll
      for (int j = 0; j < C::S; ++j) issue_slots(j);
    }
    wait_vmcnt<0>();
    lds_barrier();
#pragma unroll
    for (int j = 0; j < C::S; ++j) {
      if (j >= ntiles) break;
      if (quant && j == C::S - 1) quantize_q();  // the other stages' rows are in flight
      issue_slots(j + C::S);
      issue_rows(j);
      issue_scales(j);
    }
    if (quant && ntiles < C::S) quantize_q();  // the last stage stays free
  };

  // ---- main loop ---------------------------------------------------------------
  int8_t* vote = reinterpret_cast<int8_t*>(smem + C::OFF_VOTE);
  float* xch = reinterpret_cast<float*>(smem + C::OFF_X);
  bool slots_issued = true;  // by the early issue above; a restart issues them again
  bool q_pending = QB;       // Q is quantized in the first prologue only
  for (;;) {
    bool restart = false;
    if (ntiles > 0) prologue(slots_issued, q_pending);
    slots_issued = false;
    q_pending = false;
    for (int ti = 0; ti < ntiles; ++ti) {
      const int st = ti % C::S;
      const int nval = min(kTile, ntok - kTile * ti);
      // groups issued after group ti: 1 .. S-1 at the first tile, then the
      // S-2 before this pass's own issue
      wait_tile(min(ti == 0 ? C::S - 1 : C::S - 2, ntiles - 1 - ti));
      lds_barrier();  // (1) tile ti and its scales visible; iteration ti-1 done everywhere
      if (ti >= 1 && ti + C::S - 1 < ntiles) {
        issue_slots(ti + 2 * C::S - 1);
        issue_rows(ti + C::S - 1);
        issue_scales(ti + C::S - 1);
      }
      const uint8_t* kt = smem + st * C::STAGE;
      // e8m0 of (token t, block j): byte j & 3 of dword (j >> 2, t) at 256 (j >> 2)
      // + 4 t (j < 16), byte j - 14 of dword (4, t) (j = 16, 17)
      const uint8_t* sct = smem + C::OFF_SC + st * C::SCST;

      // ---- scores: rows i = l16 of this wave's slice, 16x16x128 MFMAs ----------
      v4f s = v4f{0.f, 0.f, 0.f, 0.f};
      int e_w = 0;  // fp4 V: max V block exponent of this wave's 16 tokens
      {
        // all fragment reads first, then the MFMA chain
        const uint8_t* kp = kt + tok_of(w, l16) * C::KST;
        v8i ka[5];
        if constexpr (KF == 2) {
          // 18 steps of 32 dims, reads two steps ahead of their MFMA
          v8bf kb[18];
#pragma unroll
          for (int ks = 0; ks < 18; ++ks) kb[ks] = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4*>(kp + 64 * ks + 16 * g));
#pragma unroll
          for (int ks = 0; ks < 18; ++ks) s = mfma16x32_bf16(kb[ks], qbf[ks], s);
          (void)ka;
        } else if constexpr (KF == 0) {
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) ka[ks] = ld_v8(kp + 128 * ks + 32 * g);
          ka[4] = g < 2 ? ld_v8(kp + 512 + 32 * g) : v8i{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
          for (int ks = 0; ks < 5; ++ks) {
            s = mfma16_f8(ka[ks], qv[ks], s);
            if constexpr (QM == 2) s = mfma16_f8_bscale(ka[ks], qlo[ks], 127 - 4, s);
          }
        } else {
          const uint8_t* sp = sct + 4 * tok_of(w, l16);
          int ksc[5];
#pragma unroll
          for (int ks = 0; ks < 5; ++ks) {
            const int blk = 4 * ks + g;
            ka[ks] = blk < kMxBlocks ? ld_v4_as_v8(kp + 16 * blk) : v8i{0, 0, 0, 0, 0, 0, 0, 0};
            ksc[ks] = blk < kMxBlocks ? (int)sp[256 * ks + (ks < 4 ? g : 2 + g)] : 127;  // blk = 4 ks + g
          }
#pragma unroll
          for (int ks = 0; ks < 5; ++ks) s = mfma16_f4f8(ka[ks], ksc[ks], qv[ks], s);
          if constexpr (C::VB16) {  // V blocks 0..15 are K blocks 4ks + g, ks < 4
            e_w = wave_max(max(max(ksc[0], ksc[1]), max(ksc[2], ksc[3])));
            e_seen = max(e_seen, e_w);
          }
        }
      }
      // s[r] = score(token tok_of(w, 4g + r), head l16)
      float sv[4];
      float mx = neg_inf();
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sv[r] = tok_of(w, 4 * g + r) < nval ? s[r] * c : neg_inf();
        mx = fmaxf(mx, sv[r]);
      }
      mx = fmaxf(mx, shfl_xor_f(mx, 16));
      mx = fmaxf(mx, shfl_xor_f(mx, 32));
      const float m_w = mx == neg_inf() ? neg_inf() : __builtin_ceilf(mx);
      m_seen = fmaxf(m_seen, m_w);
      int* ex = reinterpret_cast<int*>(smem + C::OFF_E);
      if (!have_ref) {  // first tile of the first pass: references = tile maxima over the waves
        if (g == 0) xch[16 * w + l16] = m_w;
        if (C::VB16 && lane == 0) ex[w] = e_w;
        lds_barrier();
        m_ref = fmaxf(fmaxf(xch[l16], xch[16 + l16]), fmaxf(xch[32 + l16], xch[48 + l16]));
        if constexpr (C::VB16) e_ref = max(max(ex[0], ex[1]), max(ex[2], ex[3]));
        have_ref = true;
      }
      const bool over = __any(m_w > m_ref + kRebase) || (C::VB16 && e_w > e_ref + kVScaleSpan);
      if (lane == 0) vote[w] = over ? 1 : 0;

      if constexpr (!C::P32) {
        // P' = 2^(s - m_w) * 2^8 (two fp8 terms); B scale 2^(m_w - m_ref - 8)
        const float mw = m_w == neg_inf() ? m_ref : m_w;
        const float dm = fminf(fmaxf(mw - m_ref, -160.f), 160.f);
        float pv[4], ps = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pv[r] = __builtin_amdgcn_exp2f(sv[r] - mw);
          ps += pv[r];
        }
        l_part += ps * __builtin_amdgcn_exp2f(dm);
        uint32_t hi, lo;
        pack4_fp8_split(pv[0] * kPScale, pv[1] * kPScale, pv[2] * kPScale, pv[3] * kPScale, hi, lo);
        uint8_t* pl = smem + C::OFF_P + w * 256 + l16 * 16 + 4 * g;
        *reinterpret_cast<uint32_t*>(pl) = hi;
        *reinterpret_cast<uint32_t*>(pl + 4 * 256) = lo;
        if (g == 0) smem[C::OFF_PS + 16 * w + l16] = (uint8_t)min(max((int)dm - 8 + 127, 0), 254);
      } else {
        // f32 P = 2^(s - m_ref), row-major [head][token]
        float pw[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pw[r] = __builtin_amdgcn_exp2f(fminf(sv[r] - m_ref, 120.f));
          l_part += pw[r];
        }
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(smem + C::OFF_P) + l16 * C::PST + tok_of(w, 4 * g)) =
            make_float4(pw[0], pw[1], pw[2], pw[3]);
      }
      lds_barrier();  // (2) P, its scales and the votes visible
      if (__builtin_amdgcn_readfirstlane(*reinterpret_cast<const int*>(vote)) != 0) {
        restart = true;
        break;
      }

      // ---- O^T[dims 128w ..] += V^T . P^T ---------------------------------------
      if constexpr (VF == 3) {
        // bf16 V: two 32-token K steps of 16x16x32 bf16 MFMAs per 16-dim tile;
        // lane (m, g) holds tokens 32h + 8g .. +7 of step h in both operands.
        // V^T by ds_read_b64_tr_b16: within a 16-lane group, result lane j,
        // element i = element j & 3 of source lane 4i + (j >> 2); source lane
        // s reads token 8g + 4u + (s >> 2), dims 16dt + 4(s & 3) .. +3, so read
        // u gives lane m tokens 8g + 4u .. +3 of dim 16dt + m.
        const float* prow = reinterpret_cast<const float*>(smem + C::OFF_P) + l16 * C::PST;
        v8bf pb[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float4 pa = *reinterpret_cast<const float4*>(prow + 32 * h + 8 * g);
          const float4 pc = *reinterpret_cast<const float4*>(prow + 32 * h + 8 * g + 4);
          pb[h] = __builtin_bit_cast(v8bf, make_uint4(pack_bf16x2(pa.x, pa.y), pack_bf16x2(pa.z, pa.w),
                                                      pack_bf16x2(pc.x, pc.y), pack_bf16x2(pc.z, pc.w)));
        }
        const uint32_t vb = lds0 + st * C::STAGE + (8 * g + (l16 >> 2)) * C::KST + 2 * (128 * w + 4 * (l16 & 3));
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint32_t a = vb + (32 * h) * C::KST + 32 * dt;
            const v4s16 r0 = lds_read_tr16(a);
            const v4s16 r1 = lds_read_tr16(a + 4 * C::KST);
            const v8bf av = __builtin_bit_cast(v8bf, v8s16{r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3]});
            o[dt] = mfma16x32_bf16(av, pb[h], o[dt]);
          }
        }
      } else if constexpr (!C::VB16) {
        // The block-scaled MFMA takes fp8 byte j of lane group G as K index
        // 16G + (j & 15) + 64 (j >> 4), scaled by lane group K/32.  Wave gw's
        // 16 tokens therefore sit in K block gw: bytes 0-7 of group G hold
        // tokens 8(G & 1) .. +7 of wave G/2, bytes 16-23 those of wave G/2 + 2,
        // the other bytes are zero; lane group G supplies wave G's scale.
        const int g0 = g >> 1, g1 = (g >> 1) + 2, ih = 8 * (g & 1);
        const uint8_t* pb = smem + C::OFF_P + l16 * 16 + ih;
        const uint2 h0 = *reinterpret_cast<const uint2*>(pb + g0 * 256);
        const uint2 h1 = *reinterpret_cast<const uint2*>(pb + g1 * 256);
        const uint2 q0 = *reinterpret_cast<const uint2*>(pb + 1024 + g0 * 256);
        const uint2 q1 = *reinterpret_cast<const uint2*>(pb + 1024 + g1 * 256);
        const v8i ph = v8i{(int)h0.x, (int)h0.y, 0, 0, (int)h1.x, (int)h1.y, 0, 0};
        const v8i pl = v8i{(int)q0.x, (int)q0.y, 0, 0, (int)q1.x, (int)q1.y, 0, 0};
        const int bsc = smem[C::OFF_PS + 16 * g + l16];
        // transpose reads: row 16 g0 + ih + m (bytes 0-7) and 16 g1 + ih + m
        // (bytes 16-23), dims 128w + 16dt + 8(lane & 1)
        const int vst = VF == 1 ? C::VST : C::KST;
        const uint32_t vb = lds0 + st * C::STAGE + (VF == 1 ? C::KW * 1024 : 0) + 128 * w + 8 * (lane & 1);
        const int m = l16 >> 1;
        const uint32_t a0 = vb + (16 * g0 + ih + m) * vst, a1 = vb + (16 * g1 + ih + m) * vst;
        v2i r0[8], r1[8];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          r0[dt] = lds_read_tr8(a0 + 16 * dt);
          r1[dt] = lds_read_tr8(a1 + 16 * dt);
        }
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const v8i av = v8i{r0[dt][0], r0[dt][1], 0, 0, r1[dt][0], r1[dt][1], 0, 0};
          o[dt] = mfma16_f8_bscale(av, ph, bsc, o[dt]);
          o[dt] = mfma16_f8_bscale(av, pl, bsc, o[dt]);
        }
      } else {
        // Two 32-token K steps of 16x16x32 bf16 MFMAs per dim tile; lane (m, g)
        // holds tokens T(g, k) = 8g + k (step 0, k < 8) and 24 + 8g + k (step 1,
        // k >= 8) in both operands.  V^T: one 4-bit transpose read per 16-dim
        // tile whose source lane m' reads row T(g, m'), so result lane m gets
        // dim 16dt + m of those 16 tokens, widened to bf16 at unit scale.
        // P'^T: P of the same tokens times 2^(e[t, j] - E_ref) for the MX block
        // j of the tile's dims, in bf16.  The shift is applied in one step: a
        // small P whose token has a large block exponent would lose its mantissa
        // to f32 subnormals if P were scaled by 2^-E_ref first.
        const float* prow = reinterpret_cast<const float*>(smem + C::OFF_P) + l16 * C::PST;
        float pv[16];
        {
          const float4 p0 = *reinterpret_cast<const float4*>(prow + 8 * g);
          const float4 p1 = *reinterpret_cast<const float4*>(prow + 8 * g + 4);
          const float4 p2 = *reinterpret_cast<const float4*>(prow + 32 + 8 * g);
          const float4 p3 = *reinterpret_cast<const float4*>(prow + 36 + 8 * g);
          const float pa[16] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w,
                                p2.x, p2.y, p2.z, p2.w, p3.x, p3.y, p3.z, p3.w};
#pragma unroll
          for (int k = 0; k < 16; ++k) pv[k] = pa[k];
        }
        const int trow = l16 < 8 ? 8 * g + l16 : 24 + 8 * g + l16;
        const uint32_t va = lds0 + st * C::STAGE + trow * C::KST + 64 * w;
        // dword (w, t): the e8m0 of this wave's blocks 4w .. 4w + 3 (dims 128w ..)
        const int* se = reinterpret_cast<const int*>(sct) + 64 * w;
        const int4 e0 = *reinterpret_cast<const int4*>(se + 8 * g);
        const int4 e1 = *reinterpret_cast<const int4*>(se + 8 * g + 4);
        const int4 e2 = *reinterpret_cast<const int4*>(se + 32 + 8 * g);
        const int4 e3 = *reinterpret_cast<const int4*>(se + 36 + 8 * g);
        const uint32_t ed[16] = {(uint32_t)e0.x, (uint32_t)e0.y, (uint32_t)e0.z, (uint32_t)e0.w,
                                 (uint32_t)e1.x, (uint32_t)e1.y, (uint32_t)e1.z, (uint32_t)e1.w,
                                 (uint32_t)e2.x, (uint32_t)e2.y, (uint32_t)e2.z, (uint32_t)e2.w,
                                 (uint32_t)e3.x, (uint32_t)e3.y, (uint32_t)e3.z, (uint32_t)e3.w};
        // P of tokens (k, k + 1) as a bf16 pair with E_ref taken off both
        // exponent fields (16-bit lanes, mod 2^16); block jl then adds e << 7
        // per half, which is the exact bf16 of P 2^(e - E_ref) while that
        // stays a normal number.  P <= 2^kRebase and e <= E_ref + kVScaleSpan
        // keep every sum below 2^15, so a negative 16-bit result means the
        // scaled P fell below the normal range: it becomes 0.
        u16x2 pq[8];
        const u16x2 eoff = (u16x2)(unsigned short)(e_ref << 7);
#pragma unroll
        for (int k = 0; k < 16; k += 2) pq[k / 2] = __builtin_bit_cast(u16x2, pack_bf16x2(pv[k], pv[k + 1])) - eoff;
#pragma unroll
        for (int jl = 0; jl < 4; ++jl) {  // block 4w + jl (dims 32(4w + jl) ..): byte jl
          uint32_t bw[8];
#pragma unroll
          for (int k = 0; k < 16; k += 2) {
            // byte jl of tokens k and k + 1 into the low bytes of the two halves
            const uint32_t x = __builtin_amdgcn_perm(ed[k + 1], ed[k], jl | 0x0C00u | ((4u + jl) << 16) | 0x0C000000u);
            // (e << 7) + P per half in one packed multiply-add (the compiler
            // would shift and add); its operands and result are plain VGPRs
            uint32_t y;
            asm("v_pk_mad_u16 %0, %1, %2, %3" : "=v"(y) : "v"(x), "s"(0x00800080u), "v"(pq[k / 2]));
            bw[k / 2] = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(s16x2, y), (s16x2)0));
          }
          const v8bf b0 = __builtin_bit_cast(v8bf, make_uint4(bw[0], bw[1], bw[2], bw[3]));
          const v8bf b1 = __builtin_bit_cast(v8bf, make_uint4(bw[4], bw[5], bw[6], bw[7]));
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int dt = 2 * jl + h;
            const v2i r = lds_read_tr4(va + 8 * dt);
            const uint32_t x0 = (uint32_t)r[0], x1 = (uint32_t)r[1];
            const v8bf a0 = __builtin_bit_cast(
                v8bf, make_uint4(cvt_fp4_byte<0>(x0, 1.f), cvt_fp4_byte<1>(x0, 1.f), cvt_fp4_byte<2>(x0, 1.f),
                                 cvt_fp4_byte<3>(x0, 1.f)));
            const v8bf a1 = __builtin_bit_cast(
                v8bf, make_uint4(cvt_fp4_byte<0>(x1, 1.f), cvt_fp4_byte<1>(x1, 1.f), cvt_fp4_byte<2>(x1, 1.f),
                                 cvt_fp4_byte<3>(x1, 1.f)));
            o[dt] = mfma16x32_bf16(a0, b0, o[dt]);
            o[dt] = mfma16x32_bf16(a1, b1, o[dt]);
          }
        }
      }
    }
    if (!restart) break;
    // drain the ring (the prologue reuses it); m_ref = running max over the waves
    wait_vmcnt<0>();
    if (g == 0) xch[16 * w + l16] = m_seen;
    if (C::VB16 && lane == 0) reinterpret_cast<int*>(smem + C::OFF_E)[w] = e_seen;
    lds_barrier();
    m_ref = fmaxf(fmaxf(xch[l16], xch[16 + l16]), fmaxf(xch[32 + l16], xch[48 + l16]));
    if constexpr (C::VB16) {
      const int* ex = reinterpret_cast<const int*>(smem + C::OFF_E);
      e_ref = max(max(ex[0], ex[1]), max(ex[2], ex[3]));
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = v4f{0.f, 0.f, 0.f, 0.f};
    l_part = 0.f;
    lds_barrier();  // exchange read before any rewrite
  }

  // ---- finish: row sums across lanes and waves --------------------------------
  float l = l_part;
  l += shfl_xor_f(l, 16);
  l += shfl_xor_f(l, 32);
  if (g == 0) xch[16 * w + l16] = l;
  lds_barrier();
  const float L = xch[l16] + xch[16 + l16] + xch[32 + l16] + xch[48 + l16];
  const float vs = C::VB16 ? e8m0_to_f32((uint32_t)e_ref) : vscale;  // fp4 V: 2^(E_ref - 127)
  const float inv = L > 0.f ? vs / L : 0.f;
  const int head = l16;
  if (slot < 0) {
    if (p.lse_out != nullptr && w == 0 && g == 0)
      p.lse_out[(int64_t)b * 16 + head] = L > 0.f ? (m_ref + __log2f(L)) * kLn2 : neg_inf();
    uint16_t* orow = p.out + ((int64_t)b * 16 + head) * kVDim;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int d = 128 * w + 16 * dt + 4 * g;
      const uint32_t lo = pack_bf16x2(o[dt][0] * inv, o[dt][1] * inv);
      const uint32_t hi = pack_bf16x2(o[dt][2] * inv, o[dt][3] * inv);
      *reinterpret_cast<uint2*>(orow + d) = make_uint2(lo, hi);
    }
  } else {
    uint16_t* prow = p.part_o + ((int64_t)slot * 16 + head) * kVDim;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int d = 128 * w + 16 * dt + 4 * g;
      const uint32_t lo = pack_bf16x2(o[dt][0] * inv, o[dt][1] * inv);
      const uint32_t hi = pack_bf16x2(o[dt][2] * inv, o[dt][3] * inv);
      *reinterpret_cast<uint2*>(prow + d) = make_uint2(lo, hi);
    }
    if (w == 0 && g == 0) p.part_lse[(int64_t)slot * 16 + head] = L > 0.f ? m_ref + __log2f(L) : neg_inf();
  }
}

// ============================================================================
// LSE combine: out[b,h,:] = sum_s 2^(lse_s - M) O_s / sum_s 2^(lse_s - M)
// grid (batch, H/16, 4): block = 16 heads x 128 dims, thread = (head, 8 dims);
// the split partials are read in batches of 8 so their loads overlap
// ============================================================================
__global__ __launch_bounds__(256) void combine_kernel(const DecodeParams p) {
  const int b = blockIdx.x, H = p.num_heads;
  const int2 bi = reinterpret_cast<const int2*>(p.plan + kPlanHeader + 4 * p.max_items)[b];
  if (bi.y <= 1) return;
  const int head = blockIdx.y * 16 + (threadIdx.x >> 4);
  const int d0 = blockIdx.z * 128 + (threadIdx.x & 15) * 8;
  const float* lse = p.part_lse + (int64_t)bi.x * H + head;
  const uint16_t* po = p.part_o + ((int64_t)bi.x * H + head) * kVDim + d0;
  const int64_t sstride = (int64_t)H * kVDim;
  // one pass, 8 splits per batch: lse and partial loads of a batch are issued
  // together; the running max rescales what is accumulated so far
  float M = neg_inf(), wsum = 0.f;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  for (int s0 = 0; s0 < bi.y; s0 += 8) {
    uint4 v[8];  // 8 bf16 of split s0 + j
    float ls[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // only the splits that exist are loaded
      const bool ok = s0 + j < bi.y;
      v[j] = ok ? *reinterpret_cast<const uint4*>(po + (s0 + j) * sstride) : make_uint4(0, 0, 0, 0);
      ls[j] = ok ? lse[(int64_t)(s0 + j) * H] : neg_inf();
    }
    float mb = M;
#pragma unroll
    for (int j = 0; j < 8; ++j) mb = fmaxf(mb, ls[j]);
    if (mb == neg_inf()) continue;  // every piece so far is empty
    const float r = M == neg_inf() ? 0.f : exp2f(M - mb);
    wsum *= r;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] *= r;
    M = mb;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float wg = exp2f(ls[j] - M);  // 0 for padding slots (lse -inf)
      wsum += wg;
      const uint32_t wv[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] += wg * bf16_bits_to_f32(wv[i] & 0xFFFFu);
        acc[2 * i + 1] += wg * bf16_bits_to_f32(wv[i] >> 16);
      }
    }
  }
  const float inv = wsum > 0.f ? 1.0f / wsum : 0.f;
  if (p.lse_out != nullptr && blockIdx.z == 0 && (threadIdx.x & 15) == 0)
    p.lse_out[(int64_t)b * H + head] = wsum > 0.f ? (M + __log2f(wsum)) * kLn2 : neg_inf();
  uint32_t w4[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w4[i] = pack_bf16x2(acc[2 * i] * inv, acc[2 * i + 1] * inv);
  *reinterpret_cast<uint4*>(p.out + ((int64_t)b * H + head) * kVDim + d0) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
}

// ============================================================================
template <bool IDX, bool QB>
static hipError_t launch_decode_t(const DecodeParams& p, int kv_mode, int grid, hipStream_t stream) {
  if (p.num_heads == 16) {
    if (kv_mode == 3) {  // bf16 cache: bf16 Q, used as it is
      if (!QB) return hipErrorInvalidValue;
      hipLaunchKernelGGL((decode_h16_kernel<2, 3, IDX, 3>), dim3(grid), dim3(256), 0, stream, p);
      return hipGetLastError();
    }
    if (QB && p.q_per_row) {  // bf16 Q quantized per head row here (fp8 or mxfp4 cache)
      const bool blk = p.plan_here && p.batch > 64;  // the block plans in the kernel
      switch (kv_mode) {
        case 0:
          if (blk) hipLaunchKernelGGL((decode_h16_kernel<0, 0, IDX, 5>), dim3(grid), dim3(256), 0, stream, p);
          else hipLaunchKernelGGL((decode_h16_kernel<0, 0, IDX, 4>), dim3(grid), dim3(256), 0, stream, p);
          break;
        case 1:
          if (blk) hipLaunchKernelGGL((decode_h16_kernel<1, 2, IDX, 5>), dim3(grid), dim3(256), 0, stream, p);
          else hipLaunchKernelGGL((decode_h16_kernel<1, 2, IDX, 4>), dim3(grid), dim3(256), 0, stream, p);
          break;
        default: return hipErrorInvalidValue;
      }
      return hipGetLastError();
    }
    if (QB && p.q_nparts == 0) {  // bf16 Q with no tensor-wide scale: a16w8, fp8 K only
      if (kv_mode != 0) return hipErrorInvalidValue;
      hipLaunchKernelGGL((decode_h16_kernel<0, 0, IDX, 2>), dim3(grid), dim3(256), 0, stream, p);
      return hipGetLastError();
    }
    constexpr int QM = QB ? 1 : 0;
    switch (kv_mode) {
      case 0: hipLaunchKernelGGL((decode_h16_kernel<0, 0, IDX, QM>), dim3(grid), dim3(256), 0, stream, p); break;
      case 1: hipLaunchKernelGGL((decode_h16_kernel<1, 2, IDX, QM>), dim3(grid), dim3(256), 0, stream, p); break;
      case 2: hipLaunchKernelGGL((decode_h16_kernel<1, 1, IDX, QM>), dim3(grid), dim3(256), 0, stream, p); break;
      default: return hipErrorInvalidValue;
    }
  } else if (p.num_heads == 128) {
    if (QB) return hipErrorInvalidValue;  // the H = 128 kernel takes a quantized Q
    switch (kv_mode) {
      case 0: return launch_decode_h128f(p, grid, stream);
      case 2: return launch_decode_h128m(p, grid, stream);
      default: return hipErrorInvalidValue;
    }
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_decode(const DecodeParams& p, int kv_mode, int grid, hipStream_t stream) {
  const bool idx = p.kv_indices != nullptr, qb = p.q_bf16 != nullptr;
  if (idx) return qb ? launch_decode_t<true, true>(p, kv_mode, grid, stream)
                     : launch_decode_t<true, false>(p, kv_mode, grid, stream);
  return qb ? launch_decode_t<false, true>(p, kv_mode, grid, stream)
            : launch_decode_t<false, false>(p, kv_mode, grid, stream);
}

hipError_t launch_combine(const DecodeParams& p, hipStream_t stream) {
  hipLaunchKernelGGL(combine_kernel, dim3(p.batch, p.num_heads / 16, 4), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mla
