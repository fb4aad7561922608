"""Pins the oracle's per-tensor FP8 quantizer (TASK/reference.py:65-80).

The reference's quantize_fp8 is a sequence of torch ops; torch's own
float8_e4m3fn cast is the third-party routine it rests on.  The oracle is a
table-search restatement, so agreement with torch on every bf16 input is
evidence, not a tautology.
"""
import numpy as np
import pytest
import torch

from oracle import mla_oracle as O

ALL_BF16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)
FINITE = ALL_BF16[(ALL_BF16 & 0x7F80) != 0x7F80]  # drop inf/nan


def torch_quantize_fp8(t: torch.Tensor):
    """The reference's quantize_fp8 body, evaluated by torch on the CPU."""
    finfo = torch.finfo(torch.float8_e4m3fn)
    amax = t.abs().amax().clamp(min=1e-12)
    scale = amax / finfo.max
    fp8 = (t / scale).clamp(min=finfo.min, max=finfo.max).to(torch.float8_e4m3fn)
    return fp8.view(torch.uint8).numpy(), scale.to(torch.float32).reshape(1).item()


def bits_to_torch(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def test_e4m3fn_table_matches_torch():
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    ours = O.e4m3fn_to_f32(np.arange(256))
    both_nan = np.isnan(codes) & np.isnan(ours)
    assert np.array_equal(np.where(both_nan, 0, codes), np.where(both_nan, 0, ours))
    assert np.isnan(ours[0x7F]) and np.isnan(ours[0xFF])
    assert ours[0x7E] == 448.0 and ours[0x01] == 2.0 ** -9


def test_f32_to_e4m3fn_exhaustive_over_bf16_inputs():
    # every finite bf16 value in [-448, 448] through the table search vs torch's cast
    v = O.bf16_to_f32(FINITE)
    v = v[np.abs(v) <= 448.0]
    ours = O.f32_to_e4m3fn(v)
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)


def test_f32_to_e4m3fn_ties_and_random_f32():
    rng = np.random.default_rng(0)
    grid = O.E4M3FN[:127]
    mids = ((grid[:-1] + grid[1:]) / 2).astype(np.float32)  # exact ties (all representable in f32)
    x = np.concatenate([mids, -mids, rng.uniform(-448, 448, 200000).astype(np.float32),
                        (rng.standard_normal(100000) * 2.0 ** -7).astype(np.float32)])
    ours = O.f32_to_e4m3fn(x)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)


def test_f32_to_bf16_matches_torch():
    rng = np.random.default_rng(1)
    u = rng.integers(0, 2 ** 32, 500000, dtype=np.uint64).astype(np.uint32)
    u = u[((u >> 23) & 0xFF) != 0xFF]  # finite
    ties = (rng.integers(0, 2 ** 16, 10000, dtype=np.uint32) << 16) | 0x8000
    x = np.concatenate([u, ties.astype(np.uint32)]).view(np.float32)
    x = x[np.isfinite(x)]
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16(x), ref)


def test_f32_to_bf16_overflow_edge_and_nonfinite():
    """Every f32 from just below the largest finite bf16 up to the largest
    finite f32 (the last 2^16 + 2^15 patterns, both signs): below the midpoint
    to 2^128 they round to 0x7F7F, from it on to inf, as torch rounds them;
    +-inf stay +-inf and NaN stays a NaN of its sign, with no floating-point
    warning raised on the way."""
    import warnings

    top = np.arange(0x7F7F0000, 0x7F800000, dtype=np.uint32)
    x = np.concatenate([top, top | 0x80000000]).view(np.float32)
    special = np.array([np.inf, -np.inf, np.nan, -np.nan], dtype=np.float32)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        got = O.f32_to_bf16(x)
        got_s = O.f32_to_bf16(special)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    assert (got == 0x7F80).sum() == (got == 0xFF80).sum() == 0x8000  # from the midpoint 0x7F7F8000 on
    assert got_s[0] == 0x7F80 and got_s[1] == 0xFF80
    assert (got_s[2] & 0x7FFF) > 0x7F80 and (got_s[3] & 0x7FFF) > 0x7F80
    assert (got_s[2] >> 15) == (special.view(np.uint32)[2] >> 31)


def test_scalar_divide_semantics_agree():
    # torch on GPU evaluates `amax / 448` as amax * fl(1/448); on CPU as a true
    # divide.  After rounding to bf16 both agree for every positive finite amax.
    a = O.bf16_to_f32(FINITE[(FINITE & 0x8000) == 0])
    div = O.f32_to_bf16(a / np.float32(448.0))
    mul = O.f32_to_bf16(a * (np.float32(1.0) / np.float32(448.0)))
    assert np.array_equal(div, mul)


@pytest.mark.parametrize("seed,shape,mult", [(0, (4, 16, 576), 1.0), (1, (3, 7, 33), 37.0),
                                             (2, (1000,), 1e-3), (3, (64, 576), 3e4)])
def test_quantize_matches_torch_expression(seed, shape, mult):
    g = torch.Generator().manual_seed(seed)
    t = (torch.randn(shape, generator=g) * mult).to(torch.bfloat16)
    ref_codes, ref_scale = torch_quantize_fp8(t)
    codes, scale = O.quantize_fp8_per_tensor(O.bf16_tensor_bits(t))
    assert np.float32(scale) == np.float32(ref_scale)
    assert np.array_equal(codes.reshape(-1), ref_codes.reshape(-1))


def test_quantize_exhaustive_bf16_at_fixed_amax():
    # all finite bf16 inputs at once: amax is bf16 max, scale is its /448
    t = bits_to_torch(FINITE)
    ref_codes, ref_scale = torch_quantize_fp8(t)
    codes, scale = O.quantize_fp8_per_tensor(FINITE)
    assert scale == ref_scale and np.array_equal(codes, ref_codes)
    # and the small-magnitude half alone (different scale, exercises subnormals)
    small = FINITE[(FINITE & 0x7FFF) < 0x3F80]
    ref_codes, ref_scale = torch_quantize_fp8(bits_to_torch(small))
    codes, scale = O.quantize_fp8_per_tensor(small)
    assert scale == ref_scale and np.array_equal(codes, ref_codes)


def test_quantize_invariants():
    rng = np.random.default_rng(5)
    for _ in range(20):
        x = (rng.standard_normal(4096) * rng.uniform(1e-3, 1e3)).astype(np.float32)
        bits = O.f32_to_bf16(x)
        codes, scale = O.quantize_fp8_per_tensor(bits)
        i = int(np.argmax(np.abs(O.bf16_to_f32(bits))))
        assert codes[i] & 0x7F == 0x7E  # the amax element lands on +-448
        deq = O.dequant_fp8(codes, scale)
        assert np.all(np.abs(deq) <= 448 * scale * (1 + 1e-6))
    zb = np.array([0x0000, 0x8000, 0x0000], np.uint16)
    z, s = O.quantize_fp8_per_tensor(zb)
    assert list(z) == [0x00, 0x80, 0x00]  # zeros stay zero, -0 keeps its sign
    ref_codes, ref_scale = torch_quantize_fp8(bits_to_torch(zb))  # amax clamped to bf16(1e-12)
    assert s == np.float32(ref_scale) and list(ref_codes) == [0x00, 0x80, 0x00]


def test_per_row_quantization_is_per_tensor_on_each_row():
    """quantize_fp8_per_row: each row equals quantize_fp8_per_tensor on that
    row alone (the reshape keeps rows whole: a transposed or flattened axis
    would mix rows); rows 2^20 apart in magnitude keep all their codes, where
    one tensor-wide scale flushes the small row; a row scaled by a power of
    two keeps its codes and scales its scale by the same power."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn((3, 4, 576), generator=g).to(torch.bfloat16)
    x[1, 2] *= 2.0 ** -20
    x[2, 0] *= 2.0 ** 7
    bits = O.bf16_tensor_bits(x)
    codes, scales = O.quantize_fp8_per_row(bits)
    assert codes.shape == bits.shape and scales.shape == (3, 4)
    for b in range(3):
        for h in range(4):
            c, s = O.quantize_fp8_per_tensor(bits[b, h])
            assert np.array_equal(codes[b, h], c) and scales[b, h] == s
    small = codes[1, 2]
    assert np.count_nonzero(small & 0x7F) > 500  # per row: the small row is not flushed
    whole, _ = O.quantize_fp8_per_tensor(bits)
    assert np.count_nonzero(whole[1, 2] & 0x7F) < 10  # one tensor-wide scale flushes it
    y = (x[0, 1].float() * 8.0).to(torch.bfloat16)
    cy, sy = O.quantize_fp8_per_row(O.bf16_tensor_bits(y)[None])
    assert np.array_equal(cy[0], codes[0, 1]) and sy[0] == np.float32(8.0) * scales[0, 1]


def test_reciprocal_product_rounds_like_the_division():
    """The device quantizer forms bf16(x / s) as bf16(x * r), r the correctly
    rounded f32 reciprocal of s, with no near-tie fallback: x and s are both
    bf16, so x / s is never within 2^-17 (relative) of a bf16 rounding tie
    while x * r is within 2^-23 of x / s.  Checked here in f32 arithmetic
    against the reference's f32 division for every finite bf16 x and every
    16th bf16 scale the per-tensor rule can produce (amax clamped to 1e-12,
    at most the bf16 maximum: s in [2.2e-15, 7.6e35]); the values beyond 448
    clamp alike.  (Every scale, run once: no mismatch either.)"""
    def bf16_rne(f):
        u = f.view(np.uint32).astype(np.uint64)
        u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF
        return ((u >> 16) << 16).astype(np.uint32).view(np.float32)

    x = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    x = x[np.isfinite(x)]
    s_all = (np.arange(0x7F80, dtype=np.uint32) << 16).view(np.float32)
    s_all = s_all[(s_all >= np.float32(2.2e-15)) & (s_all <= np.float32(7.6e35))]
    with np.errstate(over="ignore"):
        for s in s_all[::16]:
            r = np.float32(1.0) / s
            a = np.clip(bf16_rne((x * r).astype(np.float32)), -448, 448)
            b = np.clip(bf16_rne((x / s).astype(np.float32)), -448, 448)
            assert np.array_equal(a, b), float(s)
