// MLA absorbed decode, 128 heads, for gfx950: the fp8 cache (K = V = the
// 576-byte rows), and the two-cache mode (mxfp4 K rows with their e8m0 block
// scales for QK, the fp8 cache's rows for V), which differs only in its LDS
// rings, its DMA schedule and its QK operands (see the end of this comment).
//
// Work split: one work-group of 4 waves per CU runs one work item {batch,
// token range, slot} of the on-device plan.  Wave w owns heads 32w .. 32w+31
// for every token of the item and all 512 latent dims: Q^T (the QK B operand,
// 72 VGPRs) stays in registers, O^T (the PV accumulator, 256 AGPRs) never
// leaves them, and the softmax needs no cross-wave exchange.  This split reads
// each K and V byte from LDS once per 32 heads, the fewest LDS reads of any
// split that keeps Q in registers.
//
// Tiles are 32 tokens, pairs of tiles 64.  Per tile a wave runs 9 QK MFMAs
// (32x32x64, S^T = K . Q^T); per pair 32 PV MFMAs (O^T += V^T . P'^T, K = the
// pair's 64 tokens): P' split into two fp8 terms, hi = e4m3(x) and lo =
// e4m3(x - hi), each its own MFMA against the same V^T fragment (16 dim tiles
// x 2 terms).  Each lane's own QK outputs are exactly the 16 tokens its P'^T
// bytes of that tile need, so P never crosses lanes.  The loop is a software
// pipeline: iteration t runs QK(t), softmax(t - 1) and half of the PV of the
// pair whose softmax ended before it (pair q - 2's second half in the even
// iteration of pair q, pair q - 1's first half in the odd one).
//
// A wave issues one MFMA per 64 cycles and only about a dozen other
// instructions fit beside each (one wave per SIMD), so the iteration is a
// static schedule of 25 MFMA slots (QK steps at slots 0, 3, .., 24, PV in
// between) with the other work spread one slice per slot: fragment loads four
// to six slots ahead of their MFMA, one of 22 softmax steps, one row DMA every
// two or three slots of the pair.  Addresses move once per tile, in place.
//
// LDS: a 4-stage ring of 64-row pairs (608-byte rows: 576 + 32 of padding,
// 16-byte chunks of row r XOR-swizzled by (r >> 2) & 7, which keeps both the K
// fragment reads (ds_read_b128) and the V^T transpose reads
// (ds_read_b64_tr_b8) near their bank-conflict floor).  Rows arrive by LDS-DMA
// (global_load_lds_dwordx4) two pairs ahead of use; a pair's 64 slot indices
// arrive by one dword LDS-DMA four pairs ahead of its rows.  Two work-group
// barriers per pair: one once every wave has read the last V^T of pair q - 2
// (its stage then takes pair q + 2's rows), one once pair q + 1 has landed.
// The LDS-DMA writes lane l of a 1 KiB window to position 64u + l of the
// pair's stage, so each lane fetches whichever chunk its position holds
// (padding positions re-fetch chunk 0 of their row, a cache hit).  Q comes the
// same way, into stages 2-3 before the first rows(2) land there.
//
// Softmax: per head a reference m_ref (the first tile's ceil max); a tile's
// P' = 2^(c s - m_t + 8) with m_t its ceil max, and the PV MFMA's e8m0 B scale
// carries 2^(m_t - m_ref - 8), so O^T accumulates sum V 2^(s - m_ref) with no
// rescale.  A tile max more than 96 above m_ref (the accumulators could
// overflow) is clamped and flagged; at the end of the item a flag from any
// wave makes the work-group run the item again with every head's m_ref set to
// its running max over the whole item, which no tile then exceeds.
//
// Two-cache mode: K and V rows come from different caches, so they have rings
// of their own, each sized to its lifetime: K rows (288 bytes of fp4, rows of
// 304 bytes, conflict-free for the 16-byte fragment reads) in 3 pair stages;
// V half rows (dims 256h .. +255, rows of 272 bytes, at their bank floor for
// the transpose reads, which then need one address register) in 4 half-pair
// stages, fetched one pair after their K (each half one iteration before its
// stage is needed); the 18 e8m0 bytes of each K row in 3 stages as five dword
// DMAs per pair (dword j of every row of the pair in plane j: bytes 4j .. 4j +
// 3 for j < 4, bytes 14 .. 17 for j = 4), so a lane's 9 scales of a tile are
// three LDS reads.  Every DMA of a pair has its own slot, and every pair issues all of
// them (past the item's end they re-fetch its last row), so each wave's
// outstanding-DMA count at the two barriers is a compile-time constant.  QK is
// the scaled f8f6f4 MFMA with fp4 A (K, 4 VGPRs), the lane's e8m0 byte as A
// scale (K step ks of lane half hh scales by byte 2ks + hh; the lanes of half 1
// shift their scale dwords down a byte, so every lane's scale of step ks sits
// at byte 2 (ks & 1) of dword ks >> 1, the byte the MFMA selects), and fp8 Q^T
// in the order that pairs with the fp4 K layout.
//
// Behavioural reference: mixed-mla/asm_dumps/aiter_mla.py:149-470 (interface,
// 128-head folding :318-353), TASK/reference.py:349-369 (numerics).
#include <type_traits>

#include "mla_internal.hpp"

namespace mla {
namespace {

constexpr float kLog2eF = 1.4426950408889634f;
constexpr float kLn2F = 0.6931471805599453f;
constexpr float kRebaseF = 96.0f;

struct G128 {
  static constexpr int RST = 608;               // LDS row stride
  static constexpr int CPR = RST / 16;          // 38 chunk positions per row (36 used)
  static constexpr int HT = 32;                 // tokens per tile
  static constexpr int TSTAGE = HT * RST;       // 19456 B per tile
  static constexpr int PSTAGE = 2 * TSTAGE;     // a pair of tiles: 38 one-KiB DMA windows
  static constexpr int WIN = PSTAGE / 1024;
  static constexpr int NP = 4;                  // pair stages: pairs q-1 (V), q (K), q+1, q+2 (in flight)
  static constexpr int NSL = 8;                 // slot stages (one per pair)
  static constexpr int DMAX = (WIN + 3) / 4;    // windows of waves 0, 1 (waves 2, 3: DMAX - 1)
  static constexpr int OFF_SLOT = NP * PSTAGE;
  static constexpr int OFF_FLAG = OFF_SLOT + NSL * 256;  // [4] per-wave overflow flags
  static constexpr int LDS = OFF_FLAG + 16;
  static constexpr int OFF_Q = 2 * PSTAGE;      // Q (prologue): pair stages 2-3
  static_assert(WIN == 38 && DMAX == 10, "DMA window split");
  static_assert(LDS <= 160 * 1024, "LDS");
};

// LDS of the two-cache mode (one pair = 64 rows per stage)
struct M128 {
  static constexpr int HT = 32;
  static constexpr int KST = 304;                 // fp4 K row: 18 chunks + 1 of padding
  static constexpr int KSTAGE = 2 * HT * KST;     // 19 one-KiB DMA windows
  static constexpr int NK = 3;                    // K stages: pairs q (QK), q + 1, q + 2
  static constexpr int VST = 272;                 // fp8 V half row: 16 chunks + 1 of padding
  static constexpr int VSTAGE = 2 * HT * VST;     // 17 one-KiB windows
  static constexpr int NV = 4;                    // V half stages
  static constexpr int SPLANES = 5;               // e8m0 dwords per row (bytes 0-15, then 14-17)
  static constexpr int SSTAGE = SPLANES * 2 * HT * 4;  // plane j: dword j of the pair's 64 rows
  static constexpr int NSL = 8;                   // slot stages (one per pair)
  static constexpr int OFF_V = NK * KSTAGE;
  static constexpr int OFF_S = OFF_V + NV * VSTAGE;
  static constexpr int OFF_SLOT = OFF_S + NK * SSTAGE;
  static constexpr int OFF_FLAG = OFF_SLOT + NSL * 256;
  static constexpr int LDS = OFF_FLAG + 16;
  static constexpr int OFF_Q = 2 * KSTAGE;        // Q (prologue): K stage 2 and the V stages
  static_assert(KSTAGE == 19 * 1024 && VSTAGE == 17 * 1024 && SSTAGE == 5 * 256, "DMA windows");
  static_assert(OFF_Q + 128 * kQKDim <= OFF_S, "Q staging stays clear of the e8m0 stages");
  static_assert(LDS <= 160 * 1024, "LDS");
};

__device__ __forceinline__ int g128_key(int r) { return (r >> 2) & 7; }
// LDS chunk position (0..35) of logical chunk c of row r; an involution
__device__ __forceinline__ int g128_pos(int r, int c) {
  const int x = g128_key(r);
  return c < 32 ? (c ^ x) : 32 + ((c - 32) ^ (x & 3));
}

__device__ __forceinline__ float ninf() { return -__builtin_inff(); }

// s_waitcnt vmcnt(N_w) for wave w (wave-uniform branch)
template <int N0, int N1, int N2, int N3>
__device__ __forceinline__ void wait_vmcnt_w(int w) {
  if (w == 0) wait_vmcnt<N0>();
  else if (w == 1) wait_vmcnt<N1>();
  else if (w == 2) wait_vmcnt<N2>();
  else wait_vmcnt<N3>();
}

// QK: 32x32x64 fp8 MFMA with its accumulator in VGPRs (O^T holds all AGPRs, and
// the builtin would give every MFMA of the kernel an AGPR accumulator).  All
// MFMAs are issued by asm so that each keeps its place in the source order
// (the builtins are pure values the compiler may move past the MFMAs they are
// meant to interleave with).  The compiler does not see these MFMAs, so the
// schedule provides their wait states: no VALU writes an MFMA operand within
// the 2 wait states before it (the fragments come from LDS, P' and its scales
// are built slots earlier), a result is read by VALU only 19 or more after it
// (16-pass XDL), no VALU touches an accumulator in flight, and a dependent
// chain on one accumulator needs none.  tests/test_isa_rules.py checks the
// built code object for both rules along every path.
__device__ __forceinline__ void qk_first(v16f& d, const v8i& a, const v8i& b) {
  asm volatile("v_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
}
__device__ __forceinline__ void qk_acc(v16f& d, const v8i& a, const v8i& b) {
  asm volatile("v_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
}
// the same with fp4 A (4 VGPRs: 32 e2m1 values) at the lane's e8m0 scale: byte
// 0 (HI = false) or byte 2 (HI = true) of sa (the A scale's byte select is
// op_sel[0] + 2 op_sel_hi[0]); fp8 B at unit scale
template <bool HI>
__device__ __forceinline__ void qk4_first(v16f& d, const v4i& a, const v8i& b, int sa) {
  if constexpr (HI)
    asm volatile("v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, 0, %3, %4 op_sel_hi:[1,0,0] cbsz:4"
                 : "=&v"(d) : "v"(a), "v"(b), "v"(sa), "v"(127));
  else
    asm volatile("v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, 0, %3, %4 op_sel_hi:[0,0,0] cbsz:4"
                 : "=&v"(d) : "v"(a), "v"(b), "v"(sa), "v"(127));
}
template <bool HI>
__device__ __forceinline__ void qk4_acc(v16f& d, const v4i& a, const v8i& b, int sa) {
  if constexpr (HI)
    asm volatile("v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel_hi:[1,0,0] cbsz:4"
                 : "+v"(d) : "v"(a), "v"(b), "v"(sa), "v"(127));
  else
    asm volatile("v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel_hi:[0,0,0] cbsz:4"
                 : "+v"(d) : "v"(a), "v"(b), "v"(sa), "v"(127));
}
__device__ __forceinline__ void drain_v(v16f& x) { asm volatile("s_nop 15\n\ts_nop 15" : "+v"(x)); }
// PV: O^T += V^T . P'^T with an e8m0 scale on B (one per lane: its head), A at
// unit scale; accumulator in AGPRs
__device__ __forceinline__ void pv_mfma(v16f& acc, const v8i& a, const v8i& b, int bscale) {
  asm volatile("v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel_hi:[0,0,0]"
               : "+a"(acc)
               : "v"(a), "v"(b), "v"(127), "v"(bscale));
}
// v_permlane32_swap of x with itself: each lane ends with its own value and
// its partner's (lane +- 32)
__device__ __forceinline__ float xhalf_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// max of three scores (no NaN canonicalization: the scores are MFMA outputs)
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
// x = -inf where pos >= lim (one compare into VCC and one select, so masking
// a tile holds no per-element lane masks)
__device__ __forceinline__ float mask_ge(float x, int pos, int lim) {
  asm("v_cmp_le_i32 vcc, %2, %1\n\tv_cndmask_b32 %0, %0, %3, vcc"
      : "+v"(x)
      : "v"(pos), "v"(lim), "v"(ninf())
      : "vcc");
  return x;
}
// {hi, lo}: hi = e4m3(x), lo = e4m3(x - hi) of four values in [0, 448)
__device__ __forceinline__ int2 split4(float a, float b, float c, float d) {
  const uint32_t h = pack4_fp8(a, b, c, d);
  const v2f h01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h, false);
  const v2f h23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h, true);
  return make_int2((int)h, (int)pack4_fp8(a - h01[0], b - h01[1], c - h23[0], d - h23[1]));
}

template <int I>
using Ic = std::integral_constant<int, I>;

template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(Ic<B>{});
    static_for<B + 1, E>(f);
  }
}

// The static schedule of one pair of iterations: 50 MFMA slots, slot i of an
// iteration (0..24) issues QK step i / 3 when i % 3 == 0, else PV dim tile
// 2 (i / 3) + i % 3 - 1.  A wave issues one MFMA per 64 cycles and about a
// dozen other instructions fit beside each one, so the other work is spread
// one slice per slot: fragment loads a few slots ahead of their MFMA, one
// softmax step, one DMA every fourth slot of the pair.
struct H128Sched {
  static constexpr int kSlots = 25;
  static constexpr bool is_qk(int i) { return i % 3 == 0; }
  // PV slot i: group g = i / 3 (dim tile 8h + g of the iteration's half h of
  // the pair's PV), term i % 3 - 1 (0: hi, 1: lo), both terms on one V^T fragment
  // K fragment loaded at slot i: step g = 2..8 of this tile six slots ahead of
  // QK g, steps 0 and 1 of the next tile (returned as 9, 10) at slots 20, 22
  static constexpr int kload(int i) {
    if (i <= 18 && i % 3 == 0) return i / 3 + 2;
    if (i == 20) return 9;
    if (i == 22) return 10;
    return -1;
  }
  // V^T fragment of group g loaded at slot 3g - 3 (g = 1..7), group 0 of the
  // next iteration (returned as 8) at slot 22
  static constexpr int vload(int i) {
    if (i <= 18 && i % 3 == 0) return i / 3 + 1;
    if (i == 22) return 8;
    return -1;
  }
  // K addresses move to the next tile after the last K load of the tile; V^T
  // addresses to the next pair in iteration 0, after its last V^T load
  static constexpr int kRebaseK = 19, kRebaseV = 21;
  // softmax step k of the previous tile at iteration slot k + 2
  static constexpr int kSoftSteps = 22;
  // pair slots: the slot-index DMA; the barrier after the last V^T read of
  // pair q - 2 (its stage then takes the rows of pair q + 2); row DMA k at
  // dma_slot(k), its slot index read two slots before; the built P' becomes
  // the PV operand at the start of iteration 1; the barrier that publishes
  // pair q + 1 (iteration 1, slot 20, before that slot's K load: the first
  // read of the next pair)
  static constexpr int kSlotDma = 1;
  static constexpr int kStageFree = 20;
  static constexpr int dma_slot(int k) { return 21 + 5 * (k / 2) + 2 * (k % 2); }
  static constexpr int row_dma(int s) {
    for (int k = 0; k < 10; ++k)
      if (dma_slot(k) == s) return k;
    return -1;
  }
  static constexpr int row_read(int s) {
    for (int k = 0; k < 10; ++k)
      if (dma_slot(k) - 2 == s) return k;
    return -1;
  }
  static constexpr int kCopy = 25;
  static constexpr int kBarrier = 45;
};

// The two-cache mode's DMAs of pair q, one per pair slot, each window's slot
// index read two slots before: V(q) half 0 (type 0) at slots 3 + 4m, half 1
// (type 1) at 24 + 4m, K(q + 2) rows (type 2) at 5, 13, 22, 30, 38, their e8m0
// dwords (type 3, five windows: m = 0 on every wave, m = 1 on wave 0) at 9 and
// 17; window m of a type is the wave's window w + 4m of the stage.  Half 0 goes into the stage freed at the
// barrier that ends pair q - 1, half 1 into the one freed at slot 20; K and
// e8m0 into the stage of pair q - 1, free since that barrier too.
struct MixSched {
  static constexpr int at(int type, int m) {
    return type == 0 ? 3 + 4 * m : type == 1 ? 24 + 4 * m : type == 2 ? (m < 2 ? 5 + 8 * m : 6 + 8 * m)
                                                                       : (m < 2 ? 9 + 8 * m : 10 + 8 * m);
  }
  // windows per stage: V 17, K 19, e8m0 5; wave w has window m iff w + 4m is one of them
  static constexpr int windows(int type) { return type < 2 ? 17 : type == 2 ? 19 : M128::SPLANES; }
  static constexpr bool has(int type, int m, int w) { return w + 4 * m < windows(type); }
  // 8 type + m of the DMA at pair slot s (a window some wave has), or -1
  static constexpr int dma(int s) {
    for (int ty = 0; ty < 4; ++ty)
      for (int m = 0; m < 5; ++m)
        if (has(ty, m, 0) && at(ty, m) == s) return 8 * ty + m;
    return -1;
  }
  static constexpr int read(int s) {
    for (int ty = 0; ty < 4; ++ty)
      for (int m = 0; m < 5; ++m)
        if (has(ty, m, 0) && at(ty, m) - 2 == s) return 8 * ty + m;
    return -1;
  }
  // DMAs wave w issues at pair slots [lo, hi) (with the slot-index DMA of wave 0)
  static constexpr int issued(int w, bool idx, int lo, int hi) {
    int c = (idx && w == 0 && lo <= H128Sched::kSlotDma && H128Sched::kSlotDma < hi) ? 1 : 0;
    for (int ty = 0; ty < 4; ++ty)
      for (int m = 0; m < 5; ++m)
        if (has(ty, m, w) && lo <= at(ty, m) && at(ty, m) < hi) ++c;
    return c;
  }
  // outstanding DMAs allowed at the slot-20 barrier (V(q - 1) half 0 landed:
  // it publishes that half) and at the slot-45 barrier (every DMA of pair q - 1
  // landed: V(q - 1) half 1, K(q + 1), e8m0(q + 1))
  static constexpr int left_free(int w, bool idx) { return issued(w, idx, 20, 50) + issued(w, idx, 0, 20); }
  static constexpr int left_pub(int w, bool idx) { return issued(w, idx, 43, 50) + issued(w, idx, 0, 45); }
  // K and e8m0 windows of one pair that wave w issues
  static constexpr int ks_per_pair(int w) {
    int c = 0;
    for (int m = 0; m < 5; ++m) c += (has(2, m, w) ? 1 : 0) + (has(3, m, w) ? 1 : 0);
    return c;
  }
  static_assert(H128Sched::kStageFree == 20 && H128Sched::kBarrier == 45, "barrier slots");
};

// What each iteration of a pair runs: QK, softmax and PV are 1 (always), 0
// (never) or 2 (where the tile or pair exists: a runtime test per MFMA and
// softmax step, which costs the schedule about a thousand cycles per
// iteration); softmax 3 = never, but its half of the P' operand is zeroed
// (the pair's PV reads it).  K1: the second iteration runs (1), is skipped
// (0) or runs while q <= npair (2).
template <int Q0, int S0, int P0, int Q1, int S1, int P1, int K1>
struct PairKind {
  static constexpr int qk(int it) { return it ? Q1 : Q0; }
  static constexpr int sm(int it) { return it ? S1 : S0; }
  static constexpr int pv(int it) { return it ? P1 : P0; }
  static constexpr int k1 = K1;
  static constexpr bool edge = !(Q0 == 1 && S0 == 1 && P0 == 1 && Q1 == 1 && S1 == 1 && P1 == 1 && K1 == 1);
};

// MIX: the two-cache mode (fp4 K + e8m0, fp8 V); else the fp8 cache
template <bool IDX, bool MIX>
__global__ __launch_bounds__(256, 1) void decode_h128_kernel(const DecodeParams p) {
  using C = std::conditional_t<MIX, M128, G128>;
  using SC = H128Sched;
  using MS = MixSched;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[C::LDS];
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;

  // the item count and this item are read together (no dependent round trip;
  // the plan has room for max_items >= gridDim.x items)
  const int32_t* plan = p.plan;
  const int nitems = plan[0];
  const int item = xcd_item<2>((int)blockIdx.x, (int)gridDim.x);  // a row's pieces, and its Q, share an L2
  const int4 it = reinterpret_cast<const int4*>(plan + kPlanHeader)[item];
  if (item >= nitems) return;
  const int b = it.x, t_beg = it.y, t_end = it.z, slot = it.w;
  const int ntok = t_end - t_beg;
  const int n = (ntok + C::HT - 1) / C::HT;  // 32-token tiles
  const int npair = (n + 1) / 2;             // pairs of tiles (the DMA and barrier unit)

  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (feeds M0)
  const int lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int head = 32 * w + l32;

  // ---- slot indices of pairs 0, 1 first: their round trip overlaps the Q load -
  // wave 0: the 64 slot indices of pair q (positions clamped into the item:
  // pairs past its end fetch valid slots too, so every pair issues the same
  // DMAs and the vmcnt counts are uniform)
  auto issue_slots = [&](int q) __attribute__((always_inline)) {
    if constexpr (IDX) {
      asm volatile("" : "+s"(q));  // the address is formed at the call, not kept live from the entry
      if (w == 0) {
        const int pos = min(t_beg + 64 * q + lane, t_end - 1);
        dma4_to_lds(p.kv_indices + pos, lds0 + C::OFF_SLOT + (q % C::NSL) * 256);
      }
    }
  };
  // ---- Q: wave w's 32 head rows (18 KiB, contiguous in memory) go by LDS-DMA
  // into ring stages that the pipeline first writes only after the barrier
  // that follows the Q^T register reads (pair stages 2-3; in the two-cache
  // mode K stage 2 and the V stages); Q then needs no compiler-tracked global
  // load (whose conservative wait would also drain the row DMAs)
  constexpr int kQWin = 32 * kQKDim / 1024;  // 18 one-KiB windows per wave
  const uint32_t q_lds = lds0 + C::OFF_Q + w * 32 * kQKDim;
  auto issue_q = [&]() __attribute__((always_inline)) {
    const uint8_t* qsrc = p.q_fp8 + ((int64_t)b * 128 + 32 * w) * kQKDim + 16 * lane;
    asm volatile("" : "+v"(qsrc));  // the window addresses are formed here, not kept live from the entry
#pragma unroll
    for (int k = 0; k < kQWin; ++k) dma16_to_lds(qsrc + 1024 * k, q_lds + 1024 * k);
  };
  // Q^T B operand: K-step ks = dims 64ks .. +63; lane half hh holds dims
  // 32hh .. +31 (fp8 K) or, paired with fp4 K, dims 16hh .. +15 and 32 + 16hh
  // .. +15 (the f8f6f4 MFMA pairs fp4 element e of lane half hh, K index 32hh
  // + e, with fp8 byte i of lane half hh', K index 16hh' + (i & 15) + 32 (i >> 4))
  v8i qv[9];
  auto read_q = [&]() __attribute__((always_inline)) {
    typedef __attribute__((address_space(3))) v4i lds_v4i_q;
    const uint32_t a = q_lds + l32 * kQKDim + (MIX ? 16 : 32) * hh;
#pragma unroll
    for (int ks = 0; ks < 9; ++ks) {
      const v4i lo = *(const lds_v4i_q*)(uintptr_t)(a + 64 * ks);
      const v4i hi = *(const lds_v4i_q*)(uintptr_t)(a + 64 * ks + (MIX ? 32 : 16));
      qv[ks] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  };
  // fp4 K: its e8m0 block scales ride on the QK MFMA's A scale
  const float c = p.q_scale[0] * (MIX ? 1.0f : p.kv_scale[0]) * p.sm_scale * kLog2eF;
  const float vscale = p.kv_scale[0];

  // ---- DMA maps ---------------------------------------------------------------
  // fp8 cache: window u = w + 4k of a pair stage puts lane l at chunk position
  // 64u + l = (row r of the pair, position j); it fetches logical chunk
  // g128_pos(r, j) (chunk 0 for the two padding positions); packed (r << 10 |
  // byte offset), two windows per register.
  // Two-cache mode: window m of each type (the wave's window u = w + 4m of the
  // stage) puts lane l at position e = 64u + l: K, chunk e of the stage = row
  // e / 19, chunk e % 19 (the padding chunk re-fetches chunk 0); V half, row e /
  // 17, chunk e % 17 (likewise); e8m0, plane u, row l: the dword at byte 4u (u <
  // 4) or 14 (u = 4) of the row's scales.  Packed (r << 9 | source byte offset
  // in the row), entries K 0..4, e8m0 5..9, V 10..14.
  constexpr int kMaps = MIX ? 8 : G128::DMAX / 2;
  uint32_t dmap[kMaps];
  if constexpr (MIX) {
    uint32_t ent[16];
#pragma unroll
    for (int m = 0; m < 5; ++m) {
      const int e = 64 * (w + 4 * m) + lane;
      const int rk = min(e / 19, 63), ck = e - 19 * (e / 19);
      ent[m] = ((uint32_t)rk << 9) | (uint32_t)(16 * (ck < 18 ? ck : 0));
      const int u = w + 4 * m;
      ent[5 + m] = u < M128::SPLANES ? ((uint32_t)lane << 9) | (uint32_t)(u < 4 ? 4 * u : 14) : 0u;
      const int rv = min(e / 17, 63), cv = e - 17 * (e / 17);
      ent[10 + m] = ((uint32_t)rv << 9) | (uint32_t)(16 * (cv < 16 ? cv : 0));
    }
    ent[15] = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) dmap[k] = ent[2 * k] | (ent[2 * k + 1] << 16);
  } else {
#pragma unroll
    for (int k = 0; k < G128::DMAX; ++k) {
      const int pidx = min(64 * (w + 4 * k) + lane, 64 * G128::WIN - 1);
      const int r = pidx / G128::CPR, j = pidx - G128::CPR * r;
      const uint32_t e = ((uint32_t)r << 10) | (uint32_t)(16 * (j < 36 ? g128_pos(r, j) : 0));
      if (k % 2 == 0) dmap[k / 2] = e;
      else dmap[k / 2] |= e << 16;
    }
  }
  // Window k of pair rq: its slot (read from the pair's slot-ring stage at
  // sbase) and its DMA into the pair's stage (stage_w: the stage plus 1 KiB w;
  // window k lands 4 KiB k further).  k is a compile-time constant at every
  // call: the map register and its half are fixed.
  // (each use first marks its map register as rewritten, which costs no
  // instruction, so that no decode is hoisted out of the loop and kept live)
  auto row_slot = [&](int k, int rq, uint32_t sbase) __attribute__((always_inline)) -> int {
    asm volatile("" : "+v"(dmap[k / 2]));
    const uint32_t r = (dmap[k / 2] >> (10 + 16 * (k % 2))) & 63u;
    if constexpr (IDX) {
      typedef __attribute__((address_space(3))) int lds_int;
      return *(const lds_int*)(uintptr_t)(sbase + 4 * r);  // entry r of the ring stage
    } else {
      return min(t_beg + 64 * rq + (int)r, t_end - 1);
    }
  };
  auto row_dma = [&](int k, int sl, uint32_t stage_w) __attribute__((always_inline)) {
    if (k < G128::DMAX - 1 || w < 2) {
      asm volatile("" : "+v"(dmap[k / 2]));
      const uint32_t off = (dmap[k / 2] >> (16 * (k % 2))) & 1023u;
      const uint8_t* src = p.k_cache + ((uint64_t)(uint32_t)sl * (uint32_t)p.k_row_stride + off);
      uint32_t saved;  // M0 saved and restored, one wait state before the DMA; nt as in dma16_to_lds_nt
      asm volatile("s_mov_b32 %0, m0\n\ts_add_u32 m0, %1, %2\n\ts_mov_b32 %0, %0\n\t"
                   "global_load_lds_dwordx4 %3, off nt\n\ts_mov_b32 m0, %0"
                   : "=&s"(saved)
                   : "s"(stage_w), "i"(4096 * k), "v"(src)
                   : "memory", "scc");
    }
  };
  auto stage_of = [&](int q) __attribute__((always_inline)) -> uint32_t {  // pair q's stage + 1 KiB w
    return __builtin_amdgcn_readfirstlane(lds0 + (q % G128::NP) * G128::PSTAGE + 1024 * w);
  };
  auto sring_of = [&](int q) __attribute__((always_inline)) -> uint32_t {  // pair q's slot-ring stage
    return __builtin_amdgcn_readfirstlane(lds0 + C::OFF_SLOT + (q % C::NSL) * 256);
  };
  auto issue_rows = [&](int q) __attribute__((always_inline)) {
    const uint32_t stw = stage_of(q), sb = sring_of(q);
    int sl[G128::DMAX];
#pragma unroll
    for (int k = 0; k < G128::DMAX; ++k) sl[k] = row_slot(k, q, sb);  // every read before the first DMA
#pragma unroll
    for (int k = 0; k < G128::DMAX; ++k) row_dma(k, sl[k], stw);
  };
  // rows(q) have landed once the DMAs issued after them are all that is
  // outstanding: the next pair's slot indices (wave 0) and its rows (ten
  // windows for waves 0 and 1, nine for waves 2 and 3)
  auto wait_rows = [&]() __attribute__((always_inline)) {
    if (w == 0) wait_vmcnt<IDX ? G128::DMAX + 1 : G128::DMAX>();
    else if (w == 1) wait_vmcnt<G128::DMAX>();
    else wait_vmcnt<G128::DMAX - 1>();
  };
  // the same near the end of the item, where no rows follow (only the slot
  // indices of wave 0)
  auto wait_rows_last = [&]() __attribute__((always_inline)) {
    if (IDX && w == 0) wait_vmcnt<1>();
    else wait_vmcnt<0>();
  };
  // two-cache mode: the slot of map entry k's row in pair pq (ring stage sbase)
  auto mix_slot = [&](int k, int pq, uint32_t sbase) __attribute__((always_inline)) -> int {
    asm volatile("" : "+v"(dmap[k / 2]));
    const uint32_t r = (dmap[k / 2] >> (9 + 16 * (k % 2))) & 63u;
    if constexpr (IDX) {
      typedef __attribute__((address_space(3))) int lds_int;
      return *(const lds_int*)(uintptr_t)(sbase + 4 * r);
    } else {
      return min(t_beg + 64 * pq + (int)r, t_end - 1);
    }
  };
  // window m of type ty (0, 1: V half; 2: K; 3: e8m0) from slot sl into the
  // stage at base (the stage plus this wave's first window)
  auto mix_dma = [&](int ty, int m, int sl, uint32_t base) __attribute__((always_inline)) {
    if (MS::has(ty, m, w)) {
      const int k = ty < 2 ? 10 + m : ty == 2 ? m : 5 + m;
      asm volatile("" : "+v"(dmap[k / 2]));
      const uint32_t off = (dmap[k / 2] >> (16 * (k % 2))) & 511u;
      if (ty == 3) {
        const uint8_t* src = p.k_scales + ((uint64_t)(uint32_t)sl * (uint32_t)p.k_scale_stride + off);
        uint32_t saved;
        asm volatile("s_mov_b32 %0, m0\n\ts_add_u32 m0, %1, %2\n\ts_mov_b32 %0, %0\n\t"
                     "global_load_lds_dword %3, off\n\ts_mov_b32 m0, %0"
                     : "=&s"(saved)
                     : "s"(base), "i"(1024 * m), "v"(src)
                     : "memory", "scc");
      } else {
        const uint8_t* src = ty == 2 ? p.k_cache + ((uint64_t)(uint32_t)sl * (uint32_t)p.k_row_stride + off)
                                     : p.v_cache + ((uint64_t)(uint32_t)sl * (uint32_t)p.v_row_stride +
                                                    (uint32_t)(256 * ty) + off);
        uint32_t saved;
        asm volatile("s_mov_b32 %0, m0\n\ts_add_u32 m0, %1, %2\n\ts_mov_b32 %0, %0\n\t"
                     "global_load_lds_dwordx4 %3, off nt\n\ts_mov_b32 m0, %0"
                     : "=&s"(saved)
                     : "s"(base), "i"(4096 * m), "v"(src)
                     : "memory", "scc");
      }
    }
  };
  auto kstage_of = [&](int x) __attribute__((always_inline)) -> uint32_t {  // K stage of pair x + 1 KiB w
    return __builtin_amdgcn_readfirstlane(lds0 + (x % M128::NK) * M128::KSTAGE + 1024 * w);
  };
  auto sstage_of = [&](int x) __attribute__((always_inline)) -> uint32_t {  // e8m0 stage + 256 w
    return __builtin_amdgcn_readfirstlane(lds0 + M128::OFF_S + (x % M128::NK) * M128::SSTAGE + 256 * w);
  };
  auto vstage_of = [&](int hx) __attribute__((always_inline)) -> uint32_t {  // half stage hx & 3 + 1 KiB w
    return __builtin_amdgcn_readfirstlane(lds0 + M128::OFF_V + (hx & 3) * M128::VSTAGE + 1024 * w);
  };
  // K rows and e8m0 bytes of pair x (the prologue), every slot read first
  auto mix_issue_ks = [&](int x) __attribute__((always_inline)) {
    const uint32_t sb = sring_of(x), kb = kstage_of(x), eb = sstage_of(x);
    int sl[10];
#pragma unroll
    for (int k = 0; k < 10; ++k) sl[k] = mix_slot(k, x, sb);
#pragma unroll
    for (int m = 0; m < 5; ++m) mix_dma(2, m, sl[m], kb);
#pragma unroll
    for (int m = 0; m < 5; ++m) mix_dma(3, m, sl[5 + m], eb);
  };

  // ---- lane-constant fragment offsets -----------------------------------------
  // fp8 cache.  K fragment (QK A operand) of K-step ks: row l32 of the tile,
  // logical chunks 4ks + 2hh + {0, 1} (ks < 8) or 32 + 2hh + {0, 1} (ks = 8).
  // Rows r and r + 32 share a key, so the offsets hold for both tiles of a pair.
  // ka[2 (ks & 1) + j] + 128 (ks >> 1) (ks < 8), ka[4 + j] (ks = 8): LDS
  // addresses of the current K tile, moved along the ring in place.
  // Two-cache mode.  K fragment of step ks: chunk 2ks + hh of row l32 of the
  // tile, at ka[0] + 32ks; the row's e8m0 dword j at ka[1] + 256j.
  uint32_t ka[MIX ? 2 : 6];
  // (the init lambdas derive everything from an opaque copy of the lane id, so
  // the addresses are formed where they are needed, not kept live from the entry)
  auto init_ka = [&]() __attribute__((always_inline)) {
    int ln = lane;
    asm volatile("" : "+v"(ln));
    if constexpr (MIX) {  // pair 0: stage 0, tile 0
      const int r = ln & 31, h = ln >> 5;
      ka[0] = lds0 + r * M128::KST + 16 * h;
      ka[1] = lds0 + M128::OFF_S + 4 * r;
    } else {
      const int r = ln & 31, h2 = (ln >> 5) * 2, x = g128_key(r);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        ka[j] = lds0 + r * G128::RST + 16 * ((h2 + j) ^ x);
        ka[2 + j] = lds0 + r * G128::RST + 16 * ((4 + h2 + j) ^ x);
        ka[4 + j] = lds0 + r * G128::RST + 16 * (32 + ((h2 + j) ^ (x & 3)));
      }
    }
  };
  // V^T fragment (PV A operand) of dim tile dt (dims 32dt .. +31) over the 64
  // tokens of a pair: four ds_read_b64_tr_b8, read cc of lane (G, m, oo) is
  // row T0 + 16cc of the pair's first tile (bytes 8cc .. +7) and of its second
  // tile (bytes 16 + 8cc .. +7), T0 = 8(m >> 2) + 4hh + (m & 3), logical chunk
  // 2dt + (G & 1), byte 8oo: byte 16u + 4q + i <-> token 8q + 4hh + i of tile
  // u, the order of the lane's own scores.  fp8 cache: row T0 + 16cc has key
  // x0 ^ 4cc, x0 = T0 >> 2; va[4cc + (dt & 3)] + 128 (dt >> 2) (+ TSTAGE): LDS
  // addresses of the PV pair's first (second) tile.  Two-cache mode: half rows
  // of 17 chunks, unswizzled (the 16 rows T0 fall on 16 distinct chunk
  // positions), so every read of dim tile 8h + g is va[0] + 32g + (32u + 16cc)
  // 272, va[0] in the half stage of the iteration.
  uint32_t va[MIX ? 1 : 8];
  auto init_va = [&]() __attribute__((always_inline)) {
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int G = ln >> 4, m = (ln & 15) >> 1, oo = ln & 1;
    const int T0 = 8 * (m >> 2) + 4 * (ln >> 5) + (m & 3);
    if constexpr (MIX) {  // iteration 0 reads half stage 1 (never by an MFMA)
      va[0] = lds0 + M128::OFF_V + M128::VSTAGE + T0 * M128::VST + 16 * (G & 1) + 8 * oo;
    } else {
      const int x0 = T0 >> 2;
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
#pragma unroll
        for (int e = 0; e < 4; ++e)  // pair -2: stage 2 (never read by an MFMA)
          va[4 * cc + e] = lds0 + 2 * G128::PSTAGE + (T0 + 16 * cc) * G128::RST +
                           16 * ((2 * e + (G & 1)) ^ (x0 ^ (4 * cc))) + 8 * oo;
    }
  };
  typedef __attribute__((address_space(3))) v4i lds_v4i;
  typedef __attribute__((address_space(3))) int lds_i32;
  v8i kf[3];
  v4i kf4[3];                  // two-cache mode: fp4 K fragments
  // two-cache mode: e8m0 dwords of the K tile (steps 0..3, 4..7, 8), each
  // shifted down by 8 hh once loaded (byte 2 (ks & 1) of dword ks >> 1, byte 2 of sc8)
  int sc_lo[2] = {0x7F7F7F7F, 0x7F7F7F7F}, sc_hi[2] = {0x7F7F7F7F, 0x7F7F7F7F};
  int sc8 = 0x7F7F7F7F;
  const int sc_shift = 8 * hh;
  auto kload = [&](int g) __attribute__((always_inline)) {  // K fragment of step g (0..8) into kf[g % 3]
    if constexpr (MIX) {
      kf4[g % 3] = *(const lds_v4i*)(uintptr_t)(ka[0] + 32 * g);
    } else {
      const uint32_t a0 = g < 8 ? ka[2 * (g & 1)] + 128 * (g >> 1) : ka[4];
      const uint32_t a1 = g < 8 ? ka[2 * (g & 1) + 1] + 128 * (g >> 1) : ka[5];
      const v4i lo = *(const lds_v4i*)(uintptr_t)a0;
      const v4i hi = *(const lds_v4i*)(uintptr_t)a1;
      kf[g % 3] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  };
  // V^T fragment of group g (dim tile dt = 8h + g) into vf[g % 2]
  v8i vf[2];
  auto vload = [&](int h, int g) __attribute__((always_inline)) {
    if constexpr (MIX) {
      const uint32_t a = va[0] + 32 * g;
      const v2i r0 = lds_read_tr8(a);
      const v2i r1 = lds_read_tr8(a + 16 * M128::VST);
      const v2i r2 = lds_read_tr8(a + 32 * M128::VST);
      const v2i r3 = lds_read_tr8(a + 48 * M128::VST);
      vf[g % 2] = v8i{r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
    } else {
      const int dt = 8 * h + g;
      const uint32_t a0 = va[dt & 3] + 128 * (dt >> 2), a1 = va[4 + (dt & 3)] + 128 * (dt >> 2);
      const v2i r0 = lds_read_tr8(a0);
      const v2i r1 = lds_read_tr8(a1);
      const v2i r2 = lds_read_tr8(a0 + G128::TSTAGE);
      const v2i r3 = lds_read_tr8(a1 + G128::TSTAGE);
      vf[g % 2] = v8i{r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
    }
  };
  // two-cache mode: the e8m0 dwords of the current K tile (ka[1]), and their
  // per-lane-half shift (a separate step, placed slots after the read)
  auto scload_lo = [&]() __attribute__((always_inline)) {
    sc_lo[0] = *(const lds_i32*)(uintptr_t)ka[1];
    sc_lo[1] = *(const lds_i32*)(uintptr_t)(ka[1] + 256);
  };
  auto scload_hi = [&]() __attribute__((always_inline)) {
    sc_hi[0] = *(const lds_i32*)(uintptr_t)(ka[1] + 512);
    sc_hi[1] = *(const lds_i32*)(uintptr_t)(ka[1] + 768);
  };
  auto scload_8 = [&]() __attribute__((always_inline)) { sc8 = *(const lds_i32*)(uintptr_t)(ka[1] + 1024); };
  // (asm, so that the shift stays in its slot: a plain shift is a value the
  // compiler may recompute right before its MFMA, inside the wait states)
  auto shr = [&](int& x) __attribute__((always_inline)) {
    asm volatile("v_lshrrev_b32 %0, %1, %0" : "+v"(x) : "v"(sc_shift));
  };
  auto scshift_lo = [&]() __attribute__((always_inline)) {
    shr(sc_lo[0]);
    shr(sc_lo[1]);
  };
  auto scshift_hi = [&]() __attribute__((always_inline)) {
    shr(sc_hi[0]);
    shr(sc_hi[1]);
  };
  auto scshift_8 = [&]() __attribute__((always_inline)) { shr(sc8); };
  // two-cache mode: outstanding-DMA waits of the two barriers
  auto mix_wait_free = [&]() __attribute__((always_inline)) {
    wait_vmcnt_w<MS::left_free(0, IDX), MS::left_free(1, IDX), MS::left_free(2, IDX), MS::left_free(3, IDX)>(w);
  };
  auto mix_wait_pub = [&]() __attribute__((always_inline)) {
    wait_vmcnt_w<MS::left_pub(0, IDX), MS::left_pub(1, IDX), MS::left_pub(2, IDX), MS::left_pub(3, IDX)>(w);
  };

  v16f o[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = v16f{};
  float m_ref = 0.f, l_run = 0.f, m_seen = ninf();
  bool have_ref = false, overflow = false;

  // ---- softmax of tile t (scores s, one lane = one head, 16 tokens) ------------
  // s[r] = raw score(token 8(r >> 2) + 4hh + (r & 3)); output: bytes 16u + 4q + i
  // of the pair's P'^T B operands (u = t & 1: the tile's half) = the hi term
  // (in w_hi) and the lo term (in w_lo) of token 8q + 4hh + i, and the tile's
  // B scale (lane half u of wsc: the scale of K block u).  22 steps of a few
  // VALU ops, one per MFMA slot.
  v8i w_hi = v8i{}, w_lo = v8i{}, r_hi = v8i{}, r_lo = v8i{};  // P' being built / the PV operand
  int wsc = 127, rsc = 127;
  float mx = 0.f, sh = 0.f, ps = 0.f;  // tile max (then its clamped exponent), 8 - exponent, row sum
  auto softmax_body = [&](auto K, auto U, int t, v16f& s, v8i& bh, v8i& bl) __attribute__((always_inline)) {
    constexpr int u = decltype(U)::value;
    constexpr int k = decltype(K)::value;
    if constexpr (k == 0) {
      // the tile's last QK MFMA issued two slots back: slots 0 and 1 hold at
      // least 13 instructions (MFMAs, fragment loads), and these 7 complete the
      // 19 a VALU read of its result needs, with one to spare
      asm volatile("s_nop 6" : "+v"(s));
      const int nval = ntok - C::HT * t;
      if (nval < C::HT) {  // token 8(r >> 2) + (r & 3) (+ 4hh) >= nval: a constant vs the lane limit
        const int lim = nval - 4 * hh;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = mask_ge(s[r], 8 * (r >> 2) + (r & 3), lim);
      }
      mx = max3f(max3f(s[0], s[1], s[2]), max3f(s[3], s[4], s[5]), s[6]);
      mx = max3f(mx, s[7], s[8]);
    } else if constexpr (k == 1) {
      mx = max3f(max3f(mx, s[9], s[10]), max3f(s[11], s[12], s[13]), max3f(s[14], s[15], s[15]));
    } else if constexpr (k == 2) {
      mx = __builtin_ceilf(xhalf_max(mx) * c);  // the tile's ceil max (finite: every tile holds a token)
    } else if constexpr (k == 3) {
      if (!have_ref) {
        m_ref = mx;
        have_ref = true;
      }
      m_seen = fmaxf(m_seen, mx);
      overflow = overflow || mx > m_ref + kRebaseF;
      mx = fminf(mx, m_ref + kRebaseF);  // the exponent, clamped: a flagged pass is run again
    } else if constexpr (k == 4) {
      const int psc = min(max((int)fmaxf(mx - m_ref, -160.f) - 8 + 127, 0), 254);
      if constexpr (u == 0) wsc = psc;
      else wsc = hh ? psc : wsc;
      sh = 8.f - mx;
      ps = 0.f;
    } else if constexpr (k <= 12) {  // P' = 2^(c s - m_t + 8) of two scores (at most 2^8 unless flagged)
      constexpr int r = 2 * (k - 5);
      s[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], c, sh));
      s[r + 1] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r + 1], c, sh));
      if constexpr (r > 0) ps += s[r - 2] + s[r - 1];  // the previous step's pair (no transcendental wait)
    } else if constexpr (k == 13) {
      ps += s[14] + s[15];
      l_run = __builtin_fmaf(ps, __builtin_amdgcn_exp2f(fmaxf(mx - m_ref, -160.f) - 8.f), l_run);
    } else {  // steps 14..21: quad qd, hi term then lo term (the hi codes decoded again)
      constexpr int qd = (k - 14) / 2;
      if constexpr ((k - 14) % 2 == 0) {
        bh[4 * u + qd] = (int)pack4_fp8_over((uint32_t)bh[4 * u + qd], s[4 * qd], s[4 * qd + 1], s[4 * qd + 2], s[4 * qd + 3]);
      } else {
        const v2f h01 = __builtin_amdgcn_cvt_pk_f32_fp8(bh[4 * u + qd], false);
        const v2f h23 = __builtin_amdgcn_cvt_pk_f32_fp8(bh[4 * u + qd], true);
        bl[4 * u + qd] = (int)pack4_fp8_over((uint32_t)bl[4 * u + qd], s[4 * qd] - h01[0], s[4 * qd + 1] - h01[1],
                                               s[4 * qd + 2] - h23[0], s[4 * qd + 3] - h23[1]);
      }
    }
  };
  auto softmax_step = [&](auto K, auto U, int t, v16f& s, v8i& bh, v8i& bl) __attribute__((always_inline)) {
    // register fences: the step's work stays in its slot (neither hoisted
    // above the previous MFMA nor sunk below the next)
    asm volatile("" : "+v"(s), "+v"(mx), "+v"(l_run), "+v"(ps), "+v"(sh));
    softmax_body(K, U, t, s, bh, bl);
    asm volatile("" : "+v"(s), "+v"(bh), "+v"(bl), "+v"(mx), "+v"(l_run), "+v"(ps), "+v"(sh));
  };

  // ---- one pair of iterations -------------------------------------------------
  // iteration t = 2q + IT: QK(t) | softmax(t - 1) | half IT ^ 1 of the PV of pair
  // q - 2 + IT (dims 256 (1 - IT) .. +255: the pair's second half in iteration
  // 0, the next pair's first half in iteration 1), a PV pair being the 64
  // tokens of its two tiles, whose softmax ended the iteration before.
  v16f sa, sb;  // QK accumulators of tiles of parity 0 / 1
  int rs[2] = {0, 0};  // slots of the next row DMAs (read two slots ahead)
  int mrs = 0;         // two-cache mode: the same (one at a time)
  // Kind (PairKind): which QK, softmax and PV parts run; at the edges of the
  // pipeline a part runs only where its tile (pair) exists: t < n; 1 <= t <=
  // n; pair j >= 0, 2j < n.  Fragment loads and slot-index DMAs run everywhere
  // (their addresses stay inside the ring and the item).  DM: the rows of pair
  // q + 2 (which exist iff q + 2 < npair) are fetched always (1), never (0), or
  // as that test says (2).
  auto pair = [&](auto kind_tag, auto dm_tag, int q) __attribute__((always_inline)) {
    using PK = decltype(kind_tag);
    constexpr bool GUARD = PK::edge;
    constexpr int DM = decltype(dm_tag)::value;
    asm volatile("" : "+s"(q));  // nothing that depends on q is precomputed (and kept live) outside the pair
    const bool dmas = DM == 1 || (DM == 2 && q + 2 < npair);
    // two-cache mode: a pair past the item's last (draining the pipeline)
    // issues no DMAs, and its barriers wait for every DMA still in flight
    const bool live = !GUARD || q < npair;
    uint32_t stw = 0, sring = 0, sring_v = 0, kb = 0, eb = 0, vb0 = 0, vb1 = 0;
    if constexpr (MIX) {  // K and e8m0 of pair q + 2, V halves of pair q
      sring = sring_of(q + 2);
      sring_v = sring_of(q);
      kb = kstage_of(q + 2);
      eb = sstage_of(q + 2);
      vb0 = vstage_of(2 * q);
      vb1 = vstage_of(2 * q + 1);
    } else {
      stw = stage_of(q + 2);
      sring = sring_of(q + 2);
    }
    auto slot = [&](auto S) __attribute__((always_inline)) {
      constexpr int ps_ = decltype(S)::value;  // slot of the pair
      constexpr int IT = ps_ / SC::kSlots;      // iteration of the pair (tile t = 2q + IT)
      constexpr int i = ps_ % SC::kSlots;       // slot of the iteration
      constexpr int H = 1 - IT;                 // PV half of the iteration
      const int t = 2 * q + IT;
      const int j = q - 2 + IT;                 // PV pair of the iteration
      v16f& s_qk = IT == 0 ? sa : sb;  // tile t
      v16f& s_sm = IT == 0 ? sb : sa;  // tile t - 1
      // 0. the built P' (pair q - 1) becomes the PV operand
      if constexpr (ps_ == SC::kCopy) {
        r_hi = w_hi;
        r_lo = w_lo;
        rsc = wsc;
      }
      constexpr int KQ = PK::qk(IT), KS = PK::sm(IT), KP = PK::pv(IT);
      // 1. the slot's MFMA
      if constexpr (SC::is_qk(i) && KQ != 0) {
        constexpr int g = i / 3;
        if (KQ == 1 || t < n) {
          if constexpr (MIX) {
            const int sa = g < 4 ? sc_lo[(g >> 1) & 1] : g < 8 ? sc_hi[(g >> 1) & 1] : sc8;
            constexpr bool HI = g == 8 || (g & 1) != 0;  // byte 2 (odd steps, step 8), else byte 0
            if constexpr (g == 0) qk4_first<HI>(s_qk, kf4[0], qv[0], sa);
            else qk4_acc<HI>(s_qk, kf4[g % 3], qv[g], sa);
          } else {
            if constexpr (g == 0) qk_first(s_qk, kf[0], qv[0]);
            else qk_acc(s_qk, kf[g % 3], qv[g]);
          }
        }
      } else if constexpr (!SC::is_qk(i) && KP != 0) {
        constexpr int g = i / 3, term = i % 3 - 1;
        if (KP == 1 || (j >= 0 && 2 * j < n)) pv_mfma(o[8 * H + g], vf[g % 2], term == 0 ? r_hi : r_lo, rsc);
      }
      // 2. barriers: pair q - 2's stage free (every wave's last V^T read of it
      // done); pair q + 1 published (its rows landed)
      if constexpr (ps_ == SC::kStageFree) {
        if constexpr (MIX) {  // and V(q - 1) half 0 published
          if (live) mix_wait_free();
          else wait_vmcnt<0>();
        }
        lds_barrier();
      }
      if constexpr (ps_ == SC::kBarrier) {
        if constexpr (MIX) {
          if (live) mix_wait_pub();
          else wait_vmcnt<0>();
        } else if constexpr (DM == 1) {
          wait_rows();
        } else if constexpr (DM == 0) {
          wait_rows_last();
        } else {
          if (dmas) wait_rows();
          else wait_rows_last();
        }
        lds_barrier();
      }
      // 3. slot indices of pair q + 4, rows of pair q + 2
      if constexpr (ps_ == SC::kSlotDma) issue_slots(q + 4);
      if constexpr (MIX) {  // every DMA of a live pair (uniform vmcnt counts)
        constexpr int ev = MS::dma(ps_);
        if constexpr (ev >= 0) {
          constexpr int ty = ev / 8, m = ev % 8;
          if (live) mix_dma(ty, m, mrs, ty == 0 ? vb0 : ty == 1 ? vb1 : ty == 2 ? kb : eb);
        }
        constexpr int rv = MS::read(ps_);
        if constexpr (rv >= 0) {
          constexpr int ty = rv / 8, m = rv % 8;
          if (live) {
            if constexpr (ty < 2) mrs = mix_slot(10 + m, q, sring_v);
            else mrs = mix_slot(ty == 2 ? m : 5 + m, q + 2, sring);
          }
        }
      } else {
        if constexpr (SC::row_dma(ps_) >= 0) {
          constexpr int k = SC::row_dma(ps_);
          if (dmas) row_dma(k, rs[k % 2], stw);
        }
        if constexpr (SC::row_read(ps_) >= 0) {
          constexpr int k = SC::row_read(ps_);
          if constexpr (DM != 0) rs[k % 2] = row_slot(k, q + 2, sring);
        }
      }
      // 4. fragment loads, address moves
      if constexpr (SC::kload(i) >= 0) kload(SC::kload(i) % 9);
      if constexpr (MIX) {  // e8m0: steps 0..7 of the next tile once its QK is past them, step 8 after;
        // each shifted two to four slots after its read, and two or more MFMA
        // slots before its first MFMA (steps 0, 4 and 8: slots 0, 12, 24)
        if constexpr (i == 20) scload_lo();
        if constexpr (i == 22) scshift_lo();
        if constexpr (i == 22) scload_hi();
        if constexpr (i == 1) scload_8();
        if constexpr (i == 2) scshift_hi();
        if constexpr (i == 5) scshift_8();
      }
      if constexpr (SC::vload(i) >= 0) {
        constexpr int g = SC::vload(i);
        if constexpr (g < 8) vload(H, g);
        else vload(IT, 0);  // group 0 of the next iteration (half IT ^ 1 ^ 1)
      }
      if constexpr (i == SC::kRebaseK) {
        if constexpr (MIX) {  // K and e8m0 tiles: + 32 rows, or on to the next pair's stage
          const int step = (q % 3 == 2) ? -2 : 1;
          const int dk = IT == 0 ? 32 * M128::KST : step * M128::KSTAGE - 32 * M128::KST;
          const int ds = IT == 0 ? 32 * 4 : step * M128::SSTAGE - 32 * 4;
          ka[0] += dk;
          ka[1] += ds;
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) asm volatile("" : "+v"(ka[jj]));
        } else {
          const int dk = IT == 0 ? G128::TSTAGE : (((q + 1) & 3) - (q & 3)) * G128::PSTAGE - G128::TSTAGE;
#pragma unroll
          for (int jj = 0; jj < 6; ++jj) {
            ka[jj] += dk;
            asm volatile("" : "+v"(ka[jj]));
          }
        }
      }
      if constexpr (MIX && i == SC::kRebaseV) {  // half stage (t + 1) & 3 -> (t + 2) & 3
        const int dv = (IT == 0 && (q & 1)) ? -3 * M128::VSTAGE : M128::VSTAGE;
        va[0] += dv;
        asm volatile("" : "+v"(va[0]));
      }
      if constexpr (!MIX && IT == 0 && i == SC::kRebaseV) {  // pair q - 2 -> q - 1
        const int dv = (((q - 1) & 3) - ((q - 2) & 3)) * G128::PSTAGE;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          va[jj] += dv;
          asm volatile("" : "+v"(va[jj]));
        }
      }
      // 5. one softmax step of tile t - 1 (a tile past the item leaves its half
      // of the operand zero)
      if constexpr (i >= 2 && i < 2 + SC::kSoftSteps && KS != 0) {
        auto zero_half = [&]() __attribute__((always_inline)) {
#pragma unroll
          for (int qd = 0; qd < 4; ++qd) {
            w_hi[4 * (1 - IT) + qd] = 0;
            w_lo[4 * (1 - IT) + qd] = 0;
          }
        };
        // an iteration with no PV has no MFMA in slot 1: 8 more wait states
        // before the first read of the QK result
        if constexpr (i == 2 && KP == 0) asm volatile("s_nop 7" : "+v"(s_sm));
        if constexpr (KS == 1) {
          softmax_step(Ic<i - 2>{}, Ic<1 - IT>{}, t - 1, s_sm, w_hi, w_lo);
        } else if constexpr (KS == 2) {
          if (t >= 1 && t <= n) softmax_step(Ic<i - 2>{}, Ic<1 - IT>{}, t - 1, s_sm, w_hi, w_lo);
          else if constexpr (i == 2) zero_half();
        } else if constexpr (i == 2) {
          zero_half();
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    static_for<0, SC::kSlots>(slot);
    // the last pair's second iteration has no work (no QK, softmax or PV tile)
    if (PK::k1 == 1 || (PK::k1 == 2 && q <= npair)) static_for<SC::kSlots, 2 * SC::kSlots>(slot);
  };
  const PairKind<1, 1, 1, 1, 1, 1, 1> N{};  // full pairs
  const Ic<0> Z{};
  const Ic<1> A{};
  const Ic<2> R{};

  bool first = true;
  for (;;) {
    if (n > 0) {
      // prologue: slots(0), slots(1) (and Q on the first pass); then what pair
      // -1 would have issued (slots(2) before rows(0); slots(3) and rows(1) after)
      issue_slots(0);
      issue_slots(1);
      if (first) {
        issue_q();
        if (IDX && w == 0) wait_vmcnt<kQWin>();  // the slot indices, not Q
      } else {
        wait_vmcnt<0>();
      }
      lds_barrier();
      issue_slots(2);
      if constexpr (MIX) mix_issue_ks(0);
      else issue_rows(0);
      issue_slots(3);
      if constexpr (MIX) mix_issue_ks(1);
      else issue_rows(1);
      // two-cache mode: K and e8m0 windows of a pair per wave (MS::ks_per_pair)
      constexpr int S0 = IDX ? 1 : 0;
      if (first) {  // this wave's Q rows landed (issued before the DMAs since)
        if constexpr (MIX) {
          wait_vmcnt_w<2 * S0 + 2 * MS::ks_per_pair(0), 2 * MS::ks_per_pair(1), 2 * MS::ks_per_pair(2),
                       2 * MS::ks_per_pair(3)>(w);
        } else {
          if (w == 0) wait_vmcnt<IDX ? 2 * G128::DMAX + 2 : 2 * G128::DMAX>();
          else if (w == 1) wait_vmcnt<2 * G128::DMAX>();
          else wait_vmcnt<2 * G128::DMAX - 2>();
        }
        read_q();
      }
      if constexpr (MIX)  // K and e8m0 of pair 0
        wait_vmcnt_w<S0 + MS::ks_per_pair(0), MS::ks_per_pair(1), MS::ks_per_pair(2), MS::ks_per_pair(3)>(w);
      else wait_rows();
      lds_barrier();  // pair 0 visible; every wave's Q^T reads done (its stages reusable)
      init_ka();
      init_va();
      kload(0);
      kload(1);
      if constexpr (MIX) {  // tile 0's steps 0..3 (shifted here), 4..7 (shifted at slot 2); step 8 at slot 1
        scload_lo();
        scload_hi();
        scshift_lo();
        // the shifted dwords are MFMA sources: two wait states before the first QK
        asm volatile("s_nop 1" : "+v"(sc_lo[0]), "+v"(sc_lo[1]));
      }
      vload(1, 0);
      // pairs: the first two (pipeline fill), the steady ones (every part of
      // both iterations runs: PV pairs q - 2 >= 0 and q - 1, QK tiles 2q + 1 < n),
      // then those that drain the pipeline (the last PV pair, npair - 1, runs in
      // pairs npair and npair + 1)
      int q = 0;
      // Edge pairs, valid for every n >= 1: QK runs unconditionally (a tile past
      // the item only fills an accumulator whose softmax never runs), PV runs
      // wherever its pair exists (j >= 0 is fixed per pair; in the tail every
      // PV pair has 0 <= 2j < n), and only the softmax keeps a runtime test.
      pair(PairKind<1, 0, 0, 1, 1, 0, 1>{}, R, 0);
      pair(PairKind<1, 2, 0, 1, 2, 1, 1>{}, R, 1);
      for (q = 2; q + 2 < npair; ++q) pair(N, A, q);  // q + 2 < npair implies 2q + 1 < n
      for (; 2 * q + 1 < n; ++q) pair(N, Z, q);
      for (; q <= npair + 1; ++q) pair(PairKind<1, 2, 1, 1, 2, 1, 2>{}, R, q);
    }
    // a flagged head on any wave: run the item again from the running maxima
    wait_vmcnt<0>();
    if (lane == 0) smem[C::OFF_FLAG + w] = __any(overflow) ? 1 : 0;
    lds_barrier();
    const bool again = __builtin_amdgcn_readfirstlane(*reinterpret_cast<const int*>(smem + C::OFF_FLAG)) != 0;
    lds_barrier();  // flags read before anyone rewrites them
    if (!again) break;
    m_ref = m_seen;
    overflow = false;
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = v16f{};
    l_run = 0.f;
    first = false;
  }

  // ---- finish: normalize, transpose O^T through LDS, coalesced row stores ------
  // (16-byte stores of whole row segments: 8-byte stores straight from the
  // accumulators touch 32 rows per instruction and issue far slower)
  asm volatile("s_nop 15\n\ts_nop 15" ::: "memory");  // last PV MFMAs retired before O^T is read
  const float L = xhalf_sum(l_run);
  const float inv = L > 0.f ? vscale / L : 0.f;
  wait_vmcnt<0>();
  lds_barrier();  // every wave done with the ring
  // wave w's O^T tile -> bf16 [32 heads][512 dims] at 32.5 KiB w (rows of
  // 1 KiB + 16 B against bank conflicts)
  constexpr int ORST = 1040;
  uint8_t* ob = smem + w * 32 * ORST;
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int d = 32 * dt + 8 * q + 4 * hh;
      const uint32_t lo = pack_bf16x2(o[dt][4 * q] * inv, o[dt][4 * q + 1] * inv);
      const uint32_t hi = pack_bf16x2(o[dt][4 * q + 2] * inv, o[dt][4 * q + 3] * inv);
      *reinterpret_cast<uint2*>(ob + l32 * ORST + 2 * d) = make_uint2(lo, hi);
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's rows written (only it reads them)
  const float lse2 = L > 0.f ? m_ref + __log2f(L) : ninf();
  uint16_t* dst = slot < 0 ? p.out + ((int64_t)b * 128 + 32 * w) * kVDim
                           : p.part_o + ((int64_t)slot * 128 + 32 * w) * kVDim;
#pragma unroll 8
  for (int h = 0; h < 32; ++h) {
    const uint4 v = *reinterpret_cast<const uint4*>(ob + h * ORST + 16 * lane);
    *reinterpret_cast<uint4*>(dst + (int64_t)h * kVDim + 8 * lane) = v;
  }
  if (hh == 0) {
    if (slot < 0) {
      if (p.lse_out != nullptr) p.lse_out[(int64_t)b * 128 + head] = L > 0.f ? lse2 * kLn2F : ninf();
    } else {
      p.part_lse[(int64_t)slot * 128 + head] = lse2;
    }
  }
}

}  // namespace

hipError_t launch_decode_h128f(const DecodeParams& p, int grid, hipStream_t stream) {
  if (p.kv_indices != nullptr)
    hipLaunchKernelGGL((decode_h128_kernel<true, false>), dim3(grid), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((decode_h128_kernel<false, false>), dim3(grid), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_decode_h128m(const DecodeParams& p, int grid, hipStream_t stream) {
  if (p.kv_indices != nullptr)
    hipLaunchKernelGGL((decode_h128_kernel<true, true>), dim3(grid), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((decode_h128_kernel<false, true>), dim3(grid), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mla
