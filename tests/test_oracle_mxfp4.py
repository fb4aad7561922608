"""Pins the oracle's MXFP4 pack (TASK/reference.py:88-113 -> AITER
dynamic_mxfp4_quant, restated at mxfp4-mm/submission_v18_custom_fused.py:26-108).

AITER is not importable here and no golden vectors ship with the reference, so
the oracle (nearest-grid table search) is checked against the reference's own
bit-trick formula, restated below as a second, independent implementation,
plus closed-form known answers for the scale rule and a round-trip bound.
"""
import numpy as np
import torch

from oracle import mla_oracle as O


def reference_e2m1_bits(qx: np.ndarray) -> np.ndarray:
    """mxfp4-mm/submission_v18_custom_fused.py:60-98 element path, in numpy uint32."""
    qx = np.asarray(qx, np.float32)
    u = qx.view(np.uint32).astype(np.uint64)
    s = u & 0x80000000
    u = u ^ s
    a = u.astype(np.uint32).view(np.float32)
    sat = a >= 6.0
    den = (~sat) & (a < 1.0)
    # denormal: add 2^22 in f32 (numpy f32 add rounds to nearest even)
    d = (a + np.float32(4194304.0)).view(np.uint32).astype(np.int64) - (149 << 23)
    # normal: RNE on the mantissa
    odd = (u >> 22) & 1
    val_to_add = ((1 - 127) << 23) + (1 << 21) - 1
    nrm = ((u.astype(np.int64) + val_to_add + odd.astype(np.int64)) & 0xFFFFFFFF) >> 22
    code = np.where(sat, 7, np.where(den, d, nrm)) & 0xFF
    return (code | (s >> 28).astype(np.int64)).astype(np.uint8)


def test_e2m1_encoding_matches_reference_formula_on_all_bf16_below_8():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    v = O.bf16_to_f32(bits)
    v = v[np.isfinite(v) & (np.abs(v) < 8.0)]
    assert np.array_equal(O.f32_to_e2m1(v), reference_e2m1_bits(v))


def test_e2m1_known_answers():
    q = np.array([0.0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 5.5, 6.0, 7.9, -0.0, -0.3, -2.6])
    codes = O.f32_to_e2m1(q)
    #          0    .25->0 .75->1.0 1.25->1 1.75->2 2.5->2 3.5->4 5->4 5.5->6 6  >=6->6 -0  -.3->-.5 -2.6->-3
    assert list(codes) == [0, 0, 2, 2, 4, 4, 6, 6, 7, 7, 7, 8, 9, 13]


def test_scale_rule_known_answers():
    amax = np.array([0.0, 1.0, 1.74, 1.75, 6.0, 7.0, 2.0 ** -130, 3.0e38], np.float32)
    e8 = O.mxfp4_block_scale(amax)
    # 0 -> 0 (clamp); 1.0 -> 2^0 -> e=-2; 1.74 keeps 2^0; 1.75 rounds to 2^1 -> e=-1;
    # 6.0 (1.5*4) -> e=0; 7.0 (1.75*4) rounds to 8 -> e=1; tiny -> clamp -127;
    # 3e38 rounds past the largest exponent to +inf -> clamp 127
    assert list(e8) == [0, 125, 125, 126, 127, 128, 0, 254]


def test_pack_layout_low_nibble_even():
    x = np.zeros((1, 32), np.float32)
    x[0, 0], x[0, 1] = 1.0, 2.0  # amax 2 -> e = -1, q = x*2 -> 2.0 (code 4), 4.0 (code 6)
    packed, e8 = O.pack_mxfp4(O.f32_to_bf16(x))
    assert packed[0, 0] == (4 | (6 << 4)) and e8[0, 0] == 126
    assert np.all(packed[0, 1:] == 0)


def test_round_trip_bound_and_zero_block():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((64, 576)) * np.exp(rng.uniform(-8, 8, (64, 1)))).astype(np.float32)
    x[5, 32:64] = 0.0
    bits = O.f32_to_bf16(x)
    packed, e8 = O.pack_mxfp4(bits)
    assert e8[5, 1] == 0 and np.all(packed[5, 16:32] == 0)
    deq = O.dequant_mxfp4(packed, e8, 576)
    xf = O.bf16_to_f32(bits).reshape(64, 18, 32)
    step = np.exp2(e8.astype(np.float64) - 127.0)[..., None]  # one unit of 2^e
    err = np.abs(deq.reshape(64, 18, 32) - xf)
    assert np.all(err <= step + 1e-30)  # <= 2^e: half spacing (<=0.5*2^e*2) or the 6..8 saturation
    # values already on the grid come back exactly
    grid = (O.E2M1[rng.integers(0, 8, (8, 576))] * rng.choice([-1, 1], (8, 576)) * 2.0 ** -2)
    grid[:, ::32] = 6.0 * 2.0 ** -2  # pin every block's amax to 6*2^e with e = -2
    gb = O.f32_to_bf16(grid.astype(np.float32))
    p2, s2 = O.pack_mxfp4(gb)
    assert np.array_equal(O.dequant_mxfp4(p2, s2, 576), O.bf16_to_f32(gb))


def test_dequant_matches_torch_native_dtypes():
    # torch's own fp4x2 / e8m0 decoders (the dtypes the reference's tensors carry)
    rng = np.random.default_rng(4)
    packed = rng.integers(0, 256, (16, 288), dtype=np.uint8)
    e8 = rng.integers(100, 150, (16, 18), dtype=np.uint8)
    sc = torch.from_numpy(e8).view(torch.float8_e8m0fnu).float().numpy()
    assert np.array_equal(sc, np.exp2(e8.astype(np.float64) - 127).astype(np.float32))
    deq = O.dequant_mxfp4(packed, e8, 576)
    lo, hi = packed & 0xF, packed >> 4
    mag = np.array([0, .5, 1, 1.5, 2, 3, 4, 6], np.float64)
    dec = lambda c: np.where(c & 8, -1, 1) * mag[c & 7]
    ref = np.empty((16, 576))
    ref[:, 0::2], ref[:, 1::2] = dec(lo), dec(hi)
    ref = (ref.reshape(16, 18, 32) * sc[..., None]).reshape(16, 576)
    assert np.array_equal(deq, ref.astype(np.float32))
