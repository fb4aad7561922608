"""CPU oracle for the MLA absorbed-decode hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or as the timed CPU baseline).  The product path never routes through
it: ``amd_optimization_challenge_amd`` raises if its HIP library is missing.

What it restates (all citations relative to the reference checkout; ``TASK/``
stands for competitor_submissions/mi355x_reference/, the in-tree copy of the
task files):

* ``quantize_fp8_per_tensor``  -- TASK/reference.py:65-80 (``quantize_fp8``),
  with torch's bf16 arithmetic made explicit: |x| max in bf16, clamp(min=1e-12)
  in bf16, ``amax / 448`` rounded to bf16, ``x / scale`` rounded to bf16,
  clamp to +-448, round-to-nearest-even cast to float8_e4m3fn.
* ``pack_mxfp4``               -- TASK/reference.py:88-113 -> AITER
  ``dynamic_mxfp4_quant``, whose algorithm the reference restates at
  mxfp4-mm/submission_v18_custom_fused.py:26-108 (``_mxfp4_quant_op``).
  AITER itself is not vendored (un-pinned HEAD clone, setup.sh:52-61), so the
  restatement there is the anchor.
* ``quantize_fp8_per_row``     -- quantize_fp8_per_tensor with each row as the
  tensor (this build's per-row Q route; no reference counterpart at row
  granularity).
* ``quantize_fp8_with_scale`` / ``append_kv`` -- the element step of
  TASK/reference.py:79-80 at a given scale, and the row-scatter cache writer
  built from it and ``pack_mxfp4`` (the incremental form of reference.py:318-321).
* ``dequant_fp8`` / ``dequant_mxfp4`` -- TASK/reference.py:73-74 and
  TASK/reference.py:116-154; e2m1 table from mixed-mla/triton_mla_mxfp4.py:21-31,
  e8m0 = 2^(e-127) from mixed-mla/triton_mla_mxfp4.py:59.
* ``mla_decode``               -- the dequantize-then-fp32
  softmax(Q K^T * sm_scale) V that ``ref_kernel`` (TASK/reference.py:349-369)
  approximates through AITER, gathered through ``kv_indices`` (page size 1).
* ``expand_pages`` / ``page_table`` -- AITER's paged-cache arguments
  (kv_indptr over pages, page ids, kv_last_page_lens, page_size;
  mixed-mla/asm_dumps/aiter_mla.py:149-175) as the reference builds them from
  per-sequence token counts (mixed-mla/submission.py:449-456, :538-544), and
  their expansion to the token rows of the cache viewed as [pages * P, row].
* ``absorb_q`` / ``v_up_proj``  -- the neighbouring per-head products the
  reference names but does not implement (mixed-mla/README.md:213-217): the
  W_UK absorption that produces the decode's 576-wide Q and the v_up_proj
  lift of its 512-wide output, in float32 from bf16 operands.

Independence from the kernels: the element encoders here are *table searches*
(nearest representable value, ties to the even code), not the bit tricks the
HIP kernels and the reference use, so agreement between the two is evidence.

Parity pins (see tests/test_oracle_*.py):
  fp8 quant   -- exhaustive against torch's own float8_e4m3fn cast (the
                 third-party routine the reference calls), plus closed-form
                 invariants; per row: each row equals the per-tensor result
                 on that row alone, rows 2^20 apart keep their codes, a row
                 scaled by a power of two keeps its codes and scales its scale.
  mxfp4 pack  -- exhaustive element encoding against the reference's bit-trick
                 formula (restated in the test), scale-rule known answers,
                 round trip.
  append      -- identity slots with the whole-buffer scale reproduce
                 quantize_fp8_per_tensor / pack_mxfp4; permuted slots give a
                 row permutation; saturation and exact-grid closed forms.
  attention   -- float64 brute force on tiny shapes, closed forms (kv_len=1,
                 identical keys), permutation/split invariance.
  neighbours  -- float64 brute force on tiny shapes; identity-block weights
                 reproduce the input columns; the rope columns pass through.
  paging      -- page_table then expand_pages returns every token's row (a
                 round trip through a random page placement); page_size 1 is
                 the identity.
"""
from __future__ import annotations

import math
import os
import time

import numpy as np

QK_DIM = 576
V_DIM = 512
MX_BLOCK = 32
FP8_MAX = 448.0
BF16_1E_12 = 0x2B8D  # torch: tensor(0., bf16).clamp(min=1e-12) -> bits 0x2b8d

# ----------------------------------------------------------------------------
# bf16 <-> f32
# ----------------------------------------------------------------------------


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 values (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest, ties to even.

    Finite inputs are rounded by a neighbour comparison on the magnitude: the
    two bf16 candidates are the truncation and the next value up (2^128, i.e.
    +inf, above the largest finite bf16), both exact in float64; the closer
    one wins, a tie goes to the one whose last mantissa bit is 0, so values at
    or past the midpoint below 2^128 overflow to inf.  +-inf map to +-inf and a
    NaN to a quiet NaN of the same sign, explicitly (no arithmetic on them).
    """
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    sign = (u >> 16) & 0x8000
    mag = u & 0x7FFFFFFF
    finite = mag < 0x7F800000
    lo = np.where(finite, mag >> 16, 0).astype(np.uint32)
    e = (lo >> 7).astype(np.int64)
    vlo = (lo << 16).view(np.float32).astype(np.float64)
    gap = np.where(e == 0, 2.0 ** -133, np.ldexp(1.0, np.maximum(e, 1) - 134))  # one bf16 ulp at lo
    vhi = vlo + gap
    xd = np.where(finite, mag, 0).astype(np.uint32).view(np.float32).astype(np.float64)
    dlo = xd - vlo
    dhi = vhi - xd
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((lo & 1) == 1))
    out = lo + pick_hi.astype(np.uint32)
    nonfinite = np.where(mag > 0x7F800000, (mag >> 16) | 0x40, mag >> 16)  # inf stays inf; NaN stays quiet NaN
    out = np.where(finite, out, nonfinite)
    return (out | sign).astype(np.uint16)


# ----------------------------------------------------------------------------
# float8 e4m3fn (OCP) -- decode table and RNE encode by table search
# ----------------------------------------------------------------------------


def _e4m3fn_table() -> np.ndarray:
    vals = np.zeros(256, dtype=np.float64)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 0x7
        if e == 0xF and m == 0x7:
            vals[c] = np.nan
        elif e == 0:
            vals[c] = s * (m / 8.0) * 2.0 ** -6
        else:
            vals[c] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return vals


E4M3FN = _e4m3fn_table()
_E4M3_POS = E4M3FN[:127]  # codes 0x00..0x7E, monotone increasing 0..448


def e4m3fn_to_f32(codes: np.ndarray) -> np.ndarray:
    return E4M3FN[np.asarray(codes, dtype=np.uint8)].astype(np.float32)


def f32_to_e4m3fn(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn code, nearest value, ties to even code; |x| > 448 saturates.

    Callers clamp to +-448 first (TASK/reference.py:79), so saturation is never
    reached on the reference path.
    """
    x = np.asarray(x, dtype=np.float64)
    a = np.minimum(np.abs(x), FP8_MAX)
    hi = np.searchsorted(_E4M3_POS, a, side="left")  # first value >= a
    hi = np.minimum(hi, 126)
    lo = np.maximum(hi - 1, 0)
    vlo = _E4M3_POS[lo]
    vhi = _E4M3_POS[hi]
    dlo = a - vlo
    dhi = vhi - a
    exact = vhi == a
    pick_hi = exact | (dhi < dlo) | ((dhi == dlo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    sign = (np.signbit(x)).astype(np.uint8) << 7
    return code | sign


# ----------------------------------------------------------------------------
# a2: per-tensor FP8 quantization (TASK/reference.py:65-80)
# ----------------------------------------------------------------------------


def fp8_scale_from_amax_bits(amax_bits: int) -> tuple[int, float]:
    """bf16 amax bits -> (bf16 scale bits, f32 scale) as torch computes it.

    TASK/reference.py:77-78: ``amax.clamp(min=1e-12)`` then ``amax / finfo.max``,
    both in bf16.  The division result is rounded to bf16.
    """
    amax_bits = max(int(amax_bits), BF16_1E_12) if amax_bits <= 0x7F80 else int(amax_bits)
    a = float(bf16_to_f32(np.array([amax_bits], dtype=np.uint16))[0])
    s_bits = int(f32_to_bf16(np.array([np.float32(a) / np.float32(FP8_MAX)], dtype=np.float32))[0])
    return s_bits, float(bf16_to_f32(np.array([s_bits], dtype=np.uint16))[0])


def quantize_fp8_per_tensor(x_bits: np.ndarray) -> tuple[np.ndarray, float]:
    """bf16 bits (any shape) -> (e4m3fn codes, same shape; float32 scale).

    Restates TASK/reference.py:76-80 step by step:
      amax   = bf16 max|x|                      (exact)
      amax   = max(amax, bf16(1e-12))           (clamp in bf16)
      scale  = bf16(amax / 448)
      y      = bf16(x / scale)                  (f32 divide, RNE to bf16)
      y      = clamp(y, -448, 448)
      codes  = e4m3fn_rne(y)
      return codes, float32(scale)
    """
    bits = np.asarray(x_bits, dtype=np.uint16)
    mag = (bits & 0x7FFF).astype(np.uint32)
    amax_bits = int(mag.max()) if mag.size else 0
    s_bits, scale = fp8_scale_from_amax_bits(amax_bits)
    return quantize_fp8_with_scale(bits, scale), np.float32(scale)


def quantize_fp8_per_row(x_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """bf16 bits [..., D] -> (e4m3fn codes, same shape; float32 scales [...]):
    quantize_fp8_per_tensor (TASK/reference.py:76-80) with each row of D as
    the tensor.  The reference's small-shape MXFP4 route scales Q per 32-element
    block for the same reason (no tensor-wide pass, mixed-mla/submission.py:
    330-334); this build's per-row route keeps the fp8 rule at row granularity."""
    bits = np.asarray(x_bits, dtype=np.uint16)
    rows = bits.reshape(-1, bits.shape[-1])
    codes = np.empty_like(rows, dtype=np.uint8)
    scales = np.empty(rows.shape[0], dtype=np.float32)
    for r in range(rows.shape[0]):
        codes[r], scales[r] = quantize_fp8_per_tensor(rows[r])
    return codes.reshape(bits.shape), scales.reshape(bits.shape[:-1])


def quantize_fp8_with_scale(x_bits: np.ndarray, scale: float) -> np.ndarray:
    """The element step of TASK/reference.py:79-80 for a given f32 scale:
    e4m3fn_rne(clamp(bf16(x / scale), -448, 448)).  With the whole buffer's
    scale this is what ``quantize_fp8`` writes for any subset of its rows."""
    xf = bf16_to_f32(np.asarray(x_bits, dtype=np.uint16))
    with np.errstate(over="ignore"):  # an f32 quotient past the range is +-inf, as torch's division gives
        q = xf / np.float32(scale)
    y = bf16_to_f32(f32_to_bf16(q))
    return f32_to_e4m3fn(np.clip(y, -FP8_MAX, FP8_MAX))


def append_kv(x_bits, slots, fp8_cache=None, fp8_scale=None, fp4_cache=None, fp4_scales=None):
    """Write tokens x_bits [n, 576] (bf16 bits) into cache rows ``slots`` in place.

    The incremental form of the cache build at TASK/reference.py:318-321:
    fp8 rows with a fixed per-tensor scale (``quantize_fp8_with_scale``), mxfp4
    rows with their own block scales (``pack_mxfp4`` of the row; scale columns
    beyond 18 untouched).  ``slots`` None = rows 0..n-1; a negative slot skips.
    Returns the bf16 bits of max|x| over the written tokens (0 if none).
    """
    x = np.asarray(x_bits, dtype=np.uint16).reshape(-1, QK_DIM)
    n = x.shape[0]
    idx = np.arange(n) if slots is None else np.asarray(slots, dtype=np.int64).reshape(n)
    keep = idx >= 0
    xs, rows = x[keep], idx[keep]
    if fp8_cache is not None:
        fp8_cache.reshape(fp8_cache.shape[0], -1)[rows, :QK_DIM] = quantize_fp8_with_scale(xs, fp8_scale)
    if fp4_cache is not None:
        packed, e8 = pack_mxfp4(xs)
        fp4_cache.reshape(fp4_cache.shape[0], -1)[rows, :QK_DIM // 2] = packed
        fp4_scales[rows, :QK_DIM // MX_BLOCK] = e8
    return int((xs & 0x7FFF).max()) if xs.size else 0


def dequant_fp8(codes: np.ndarray, scale: float) -> np.ndarray:
    """TASK/reference.py:73-74 (``fp8.to(bf16) * scale``), computed in float32."""
    return e4m3fn_to_f32(codes) * np.float32(scale)


# ----------------------------------------------------------------------------
# a4: MXFP4 (e2m1 values, e8m0 scale per 32 elements)
# ----------------------------------------------------------------------------

E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float64)


def mxfp4_block_scale(amax: np.ndarray) -> np.ndarray:
    """Per-block e8m0 byte from the block's float32 |x| max.

    mxfp4-mm/submission_v18_custom_fused.py:50-57: round amax up to the next
    power of two when its mantissa is >= 1.75 (add 2^21 to the f32 bits, drop
    the mantissa), take floor(log2) - 2, clamp to [-127, 127], bias by 127.
    A block of zeros gives 0.  A round-up that overflows the exponent gives
    +inf, whose clamp is 127 (byte 254).
    """
    a = np.asarray(amax, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((a + 0x200000) & 0xFF800000).astype(np.uint64)
    expf = (r >> 23) & 0xFF
    # floor(log2(r)): r is a power of two (or 0 / denormal-free after the mask)
    unb = np.where(r == 0, -1000, expf.astype(np.int64) - 127)
    unb = np.where(expf == 0xFF, 1000, unb)  # +inf
    e = np.clip(unb - 2, -127, 127)
    return (e + 127).astype(np.uint8)


def f32_to_e2m1(q: np.ndarray) -> np.ndarray:
    """float -> e2m1 nibble: nearest grid value, ties to the even code, >= 6 -> 7.

    Sign in bit 3 (mxfp4-mm/submission_v18_custom_fused.py:96-98); -0 keeps it.
    """
    q = np.asarray(q, dtype=np.float64)
    a = np.abs(q)
    hi = np.searchsorted(E2M1, a, side="left")
    hi = np.minimum(hi, 7)
    lo = np.maximum(hi - 1, 0)
    dlo = a - E2M1[lo]
    dhi = E2M1[hi] - a
    exact = E2M1[hi] == a
    pick_hi = exact | (dhi < dlo) | ((dhi == dlo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo)
    code = np.where(a >= 6.0, 7, code).astype(np.uint8)
    sign = np.signbit(q).astype(np.uint8) << 3
    return code | sign


def pack_mxfp4(x_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """bf16 bits [rows, cols] -> (packed uint8 [rows, cols/2], e8m0 uint8 [rows, cols/32]).

    Pack order: low nibble = even element (TASK/README.md:78;
    mxfp4-mm/submission_v18_custom_fused.py:100-106).
    """
    bits = np.asarray(x_bits, dtype=np.uint16)
    rows, cols = bits.shape
    assert cols % MX_BLOCK == 0
    x = bf16_to_f32(bits).reshape(rows, cols // MX_BLOCK, MX_BLOCK)
    amax = np.abs(x).max(axis=-1)
    e8 = mxfp4_block_scale(amax)
    unb = e8.astype(np.int64) - 127
    q = x.astype(np.float64) * np.exp2(-unb.astype(np.float64))[..., None]
    q = q.astype(np.float32)  # x * 2^-e is exact in f32 for every finite bf16 block
    codes = f32_to_e2m1(q).reshape(rows, cols)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    return packed, e8


def dequant_mxfp4(packed: np.ndarray, scales: np.ndarray, cols: int) -> np.ndarray:
    """TASK/reference.py:116-154: e2m1 value * 2^(e8m0-127), float32.

    ``scales`` may carry padding columns (TASK/reference.py:146-148); only the
    first cols/32 are used.
    """
    packed = np.asarray(packed, dtype=np.uint8)
    rows = packed.shape[0]
    lo = packed & 0xF
    hi = packed >> 4
    codes = np.empty((rows, cols), dtype=np.uint8)
    codes[:, 0::2] = lo[:, : cols // 2]
    codes[:, 1::2] = hi[:, : cols // 2]
    mag = E2M1[codes & 7]
    val = np.where(codes & 8, -mag, mag)
    sc = np.exp2(np.asarray(scales[:, : cols // MX_BLOCK], dtype=np.float64) - 127.0)
    val = val.reshape(rows, cols // MX_BLOCK, MX_BLOCK) * sc[..., None]
    return val.reshape(rows, cols).astype(np.float32)


# ----------------------------------------------------------------------------
# a7/a8: attention over the dequantized cache
# ----------------------------------------------------------------------------


def dequant_kv(kv_mode: str, fp8_codes=None, fp8_scale=None, fp4_packed=None,
               fp4_scales=None, bf16_bits=None) -> tuple[np.ndarray, np.ndarray]:
    """Return (K [T,576] f32, V [T,512] f32) for a kv_mode.

    fp8          : K = V-source = fp8 cache (V = first 512 dims)
    mxfp4        : K = mxfp4 cache, V = first 512 dims of the same cache
    mxfp4k_fp8v  : K = mxfp4 cache (576), V = fp8 cache (first 512 dims)
    bf16         : K = the bf16 cache as it is (TASK/reference.py:55-58
                   KV_DTYPE = bf16, kv_data["bf16"] of :311-327), V = first 512
    """
    if kv_mode == "bf16":
        k = bf16_to_f32(np.asarray(bf16_bits, dtype=np.uint16).reshape(-1, QK_DIM))
        return k, k[:, :V_DIM]
    if kv_mode == "fp8":
        k = dequant_fp8(fp8_codes.reshape(-1, QK_DIM), fp8_scale)
        return k, k[:, :V_DIM]
    if kv_mode == "mxfp4":
        k = dequant_mxfp4(fp4_packed.reshape(-1, QK_DIM // 2), fp4_scales, QK_DIM)
        return k, k[:, :V_DIM]
    if kv_mode == "mxfp4k_fp8v":
        k = dequant_mxfp4(fp4_packed.reshape(-1, QK_DIM // 2), fp4_scales, QK_DIM)
        v = dequant_fp8(fp8_codes.reshape(-1, QK_DIM), fp8_scale)[:, :V_DIM]
        return k, v
    raise ValueError(kv_mode)


def page_table(lengths, page_size, page_ids_for):
    """Per-sequence token counts -> AITER's page table, as mixed-mla/submission.py
    :449-456 and :538-544 build it: ceil(L / P) pages per sequence, last-page
    length L % P (P when 0).  ``page_ids_for(b, n)`` chooses the n page ids of
    sequence b.  Returns (page_indptr [B+1], page_ids, last_page_lens [B]) int32.
    """
    P = int(page_size)
    npages = [(int(L) + P - 1) // P for L in lengths]
    indptr = np.concatenate([[0], np.cumsum(npages)]).astype(np.int32)
    ids = np.concatenate([np.asarray(page_ids_for(b, n), dtype=np.int64) for b, n in enumerate(npages)] +
                         [np.zeros(0, np.int64)]).astype(np.int32)
    last = np.array([(int(L) % P) or P for L in lengths], dtype=np.int32)
    return indptr, ids, last


def expand_pages(page_indptr, page_ids, last_page_lens, page_size):
    """AITER's page table -> token-level (kv_indptr [B+1], kv_indices [T]) over
    the cache viewed as [pages * P, row]: sequence b has (n_b - 1) P + last_b
    tokens for n_b > 0 pages (last_b clamped to [1, P]); its token j is row
    page_ids[indptr[b] + j // P] * P + j % P (aiter_mla.py:149-175 with the
    kv_buffer [pages, page, 1, 576] view of mixed-mla/submission.py:508-509)."""
    P = int(page_size)
    indptr = np.asarray(page_indptr, dtype=np.int64)
    ids = np.asarray(page_ids, dtype=np.int64)
    last = np.asarray(last_page_lens, dtype=np.int64)
    lens, rows = [], []
    for b in range(len(indptr) - 1):
        n = int(indptr[b + 1] - indptr[b])
        L = (n - 1) * P + min(max(int(last[b]), 1), P) if n > 0 else 0
        lens.append(L)
        j = np.arange(L, dtype=np.int64)
        rows.append(ids[indptr[b] + j // P] * P + j % P)
    kv_indptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    kv_indices = np.concatenate(rows + [np.zeros(0, np.int64)]).astype(np.int32)
    return kv_indptr, kv_indices


def row_ranges(kv_indptr, q_seq_len=1):
    """(start, length) of the keys each query row attends to.

    Rows are (sequence b, query i) in order, q_seq_len per sequence; query i
    sees the causal prefix of length L_b - (q_seq_len - 1 - i) (clamped at 0):
    the uniform-qo_len causal decode of competitor_submissions/mi355x_reference/
    reference.py:188-193 (is_causal=True, uni_seqlen_qo=q_seq_len).  With
    q_seq_len = 1 this is simply [indptr[b], indptr[b+1]).
    """
    indptr = np.asarray(kv_indptr, dtype=np.int64)
    out = []
    for b in range(len(indptr) - 1):
        L = int(indptr[b + 1] - indptr[b])
        for i in range(q_seq_len):
            out.append((int(indptr[b]), max(L - (q_seq_len - 1 - i), 0)))
    return out


def mla_decode(q_deq, k_deq, v_deq, kv_indptr, kv_indices, sm_scale, threads=None, q_seq_len=1,
               return_lse=False):
    """out[r,h,:] = softmax(q[r,h] . K[keys_r]^T * sm_scale) V[keys_r], float32.

    q_deq [rows,H,576] f32 with rows = sequences * q_seq_len; k_deq [T,576];
    v_deq [T,512]; kv_indices maps each logical token to a cache row (page
    size 1); keys_r as in row_ranges.  A row with no keys yields 0 (and
    lse -inf).  With return_lse, also lse[r,h] = ln sum exp(sm_scale q.k)
    (natural log).  Computed with torch on the CPU (fp32 GEMM), one row at a time.
    """
    import torch

    if threads:
        torch.set_num_threads(threads)
    q = torch.as_tensor(np.ascontiguousarray(q_deq), dtype=torch.float32)
    k = torch.as_tensor(np.ascontiguousarray(k_deq), dtype=torch.float32)
    v = torch.as_tensor(np.ascontiguousarray(v_deq), dtype=torch.float32)
    idx = torch.as_tensor(np.asarray(kv_indices, dtype=np.int64))
    R, H, _ = q.shape
    ranges = row_ranges(kv_indptr, q_seq_len)
    assert len(ranges) == R, "q rows must equal sequences * q_seq_len"
    out = torch.zeros((R, H, V_DIM), dtype=torch.float32)
    lse = torch.full((R, H), float("-inf"), dtype=torch.float32)
    for r, (s0, n) in enumerate(ranges):
        if n <= 0:
            continue
        rows = idx[s0:s0 + n]
        kb = k.index_select(0, rows)
        vb = v.index_select(0, rows)
        s = (q[r] @ kb.T) * float(sm_scale)
        p = torch.softmax(s, dim=-1)
        out[r] = p @ vb
        lse[r] = torch.logsumexp(s, dim=-1)
    return (out.numpy(), lse.numpy()) if return_lse else out.numpy()


def mla_decode_f64(q_deq, k_deq, v_deq, kv_indptr, kv_indices, sm_scale, q_seq_len=1, return_lse=False):
    """Float64 pure-numpy brute force (small shapes only), explicit max-shifted softmax."""
    q = np.asarray(q_deq, np.float64)
    R, H, _ = q.shape
    out = np.zeros((R, H, V_DIM), np.float64)
    lse = np.full((R, H), -np.inf)
    for r, (s0, n) in enumerate(row_ranges(kv_indptr, q_seq_len)):
        for h in range(H):
            if n <= 0:
                continue
            rows = np.asarray(kv_indices[s0:s0 + n], np.int64)
            sc = np.array([np.dot(q[r, h], np.asarray(k_deq[t], np.float64)) for t in rows]) * sm_scale
            mx = sc.max()
            w = np.exp(sc - mx)
            lse[r, h] = mx + np.log(w.sum())
            w /= w.sum()
            out[r, h] = sum(w[i] * np.asarray(v_deq[t], np.float64) for i, t in enumerate(rows))
    return (out, lse) if return_lse else out


def reference_path(q_bits, kv_mode, caches, kv_indptr, kv_indices, sm_scale, threads=None, q_seq_len=1,
                   return_lse=False, q_dtype="fp8"):
    """The full CPU restatement of the reference path for one decode call.

    quantize Q (a2) -> dequantize Q and KV -> fp32 attention -> bf16 bits.
    q_dtype "bf16" is the a16w8 route (TASK/reference.py:55-58 Q_DTYPE, the
    bf16-Q paths of mixed-mla/submission.py:414-520): Q enters as its bf16
    values, unquantized; "fp8_row" quantizes Q per head row
    (``quantize_fp8_per_row``).
    ``caches`` = dict(fp8_codes, fp8_scale, fp4_packed, fp4_scales) (numpy).
    Returns (out_bf16_bits [rows,H,512], out_f32[, lse [rows,H] natural log]).
    """
    if q_dtype == "bf16":
        q_deq = bf16_to_f32(np.asarray(q_bits, dtype=np.uint16))
    elif q_dtype == "fp8_row":
        qc, qs = quantize_fp8_per_row(q_bits)
        q_deq = e4m3fn_to_f32(qc) * qs[..., None]
    else:
        qc, qs = quantize_fp8_per_tensor(q_bits)
        q_deq = dequant_fp8(qc, qs)
    k, v = dequant_kv(kv_mode, **caches)
    res = mla_decode(q_deq, k, v, kv_indptr, kv_indices, sm_scale, threads=threads, q_seq_len=q_seq_len,
                     return_lse=return_lse)
    if return_lse:
        out, lse = res
        return f32_to_bf16(out), out, lse
    return f32_to_bf16(res), res


def time_reference_path(q_bits, kv_mode, caches, kv_indptr, kv_indices, sm_scale,
                        reps=3, threads=None):
    """Median wall time (s) of ``reference_path`` after one warm-up; KV dequant included,
    cache construction excluded.  Returns (median_s, threads_used)."""
    import torch

    threads = threads or os.cpu_count() or 1
    torch.set_num_threads(threads)
    reference_path(q_bits, kv_mode, caches, kv_indptr, kv_indices, sm_scale)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter_ns()
        reference_path(q_bits, kv_mode, caches, kv_indptr, kv_indices, sm_scale)
        ts.append((time.perf_counter_ns() - t0) * 1e-9)
    ts.sort()
    return ts[len(ts) // 2], threads


def bf16_tensor_bits(t) -> np.ndarray:
    """torch bf16 tensor (any device) -> numpy uint16 bits."""
    import torch

    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def default_sm_scale() -> float:
    return 1.0 / math.sqrt(QK_DIM)


# ----------------------------------------------------------------------------
# Neighbouring steps: W_UK absorption (upstream) and v_up_proj (downstream)
# ----------------------------------------------------------------------------
def absorb_q(q_nope_bits: np.ndarray, q_rope_bits: np.ndarray, w_uk_bits: np.ndarray) -> np.ndarray:
    """bf16 bits q_nope [B, H, 128], q_rope [B, H, 64], w_uk [H, 128, 512] ->
    float32 Q [B, H, 576] = [q_nope[b, h] @ w_uk[h], q_rope[b, h]]."""
    qn = bf16_to_f32(q_nope_bits).astype(np.float32)
    w = bf16_to_f32(w_uk_bits).astype(np.float32)
    lat = np.einsum("bhk,hkn->bhn", qn, w, optimize=True).astype(np.float32)
    return np.concatenate([lat, bf16_to_f32(q_rope_bits).astype(np.float32)], axis=-1)


def v_up_proj(o_bits: np.ndarray, w_uv_bits: np.ndarray) -> np.ndarray:
    """bf16 bits o [B, H, 512], w_uv [H, 512, 128] -> float32 [B, H, 128]
    = o[b, h] @ w_uv[h]."""
    o = bf16_to_f32(o_bits).astype(np.float32)
    w = bf16_to_f32(w_uv_bits).astype(np.float32)
    return np.einsum("bhk,hkn->bhn", o, w, optimize=True).astype(np.float32)

