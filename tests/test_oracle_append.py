"""Pins the oracle's KV-cache writer (``append_kv``, ``quantize_fp8_with_scale``)
and the host-side bookkeeping of ``KVCache`` (no device work).

The writer is the incremental form of the reference's whole-buffer cache build
(TASK/reference.py:318-321 with quantize_fp8 :65-80 and quantize_mxfp4
:88-113).  Pins: whole-buffer equivalence, torch's own bf16 divide + fp8 cast
at a fixed scale, saturation and exact-grid closed forms, permutation.
"""
import numpy as np
import pytest
import torch

from oracle import mla_oracle as O


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _kv(n, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return _bits((torch.randn((n, O.QK_DIM), generator=g) * scale).to(torch.bfloat16))


def test_identity_slots_reproduce_whole_buffer_quantizers():
    x = _kv(40, 1)
    codes, s = O.quantize_fp8_per_tensor(x)
    packed, e8 = O.pack_mxfp4(x)
    f8 = np.zeros((40, 1, O.QK_DIM), np.uint8)
    f4 = np.zeros((40, 1, O.QK_DIM // 2), np.uint8)
    sc = np.zeros((40, 18), np.uint8)
    amax = O.append_kv(x, None, f8, s, f4, sc)
    assert np.array_equal(f8.reshape(40, -1), codes)
    assert np.array_equal(f4.reshape(40, -1), packed)
    assert np.array_equal(sc, e8)
    assert amax == int((x & 0x7FFF).max())


def test_chunked_permuted_appends_equal_a_row_permutation():
    x = _kv(50, 2)
    codes, s = O.quantize_fp8_per_tensor(x)
    packed, e8 = O.pack_mxfp4(x)
    rng = np.random.default_rng(3)
    slots = rng.permutation(80)[:50]
    f8 = np.full((80, O.QK_DIM), 0xAB, np.uint8)
    f4 = np.full((80, O.QK_DIM // 2), 0xCD, np.uint8)
    sc = np.full((80, 24), 0xEE, np.uint8)  # padded scale stride: columns 18.. untouched
    for lo, hi in ((0, 7), (7, 8), (8, 33), (33, 50)):  # ragged chunks, one of a single token
        O.append_kv(x[lo:hi], slots[lo:hi], f8, s, f4, sc)
    assert np.array_equal(f8[slots], codes)
    assert np.array_equal(f4[slots], packed)
    assert np.array_equal(sc[slots, :18], e8)
    assert (sc[:, 18:] == 0xEE).all()
    untouched = np.setdiff1d(np.arange(80), slots)
    assert (f8[untouched] == 0xAB).all() and (f4[untouched] == 0xCD).all() and (sc[untouched] == 0xEE).all()


def test_negative_slots_skip_tokens():
    x = _kv(6, 4)
    slots = np.array([3, -1, 0, -5, 5, 1])
    f8 = np.full((6, O.QK_DIM), 0x11, np.uint8)
    amax = O.append_kv(x, slots, f8, 0.01)
    for i, s in enumerate(slots):
        if s >= 0:
            assert np.array_equal(f8[s], O.quantize_fp8_with_scale(x[i], 0.01))
    assert (f8[[2, 4]] == 0x11).all()
    assert amax == int((x[slots >= 0] & 0x7FFF).max())
    assert O.append_kv(x[:0], slots[:0], f8, 0.01) == 0


@pytest.mark.parametrize("scale_bits", [0x3C23, 0x3A80, 0x3F80, 0x4100])
def test_fixed_scale_matches_torch(scale_bits):
    """quantize_fp8's element step at a bf16 scale, evaluated by torch itself
    (bf16 / bf16 -> bf16, clamp, float8_e4m3fn cast)."""
    x = _kv(64, 5, scale=3.0)
    s = float(O.bf16_to_f32(np.array([scale_bits], np.uint16))[0])
    xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
    ref = (xt / torch.tensor(s, dtype=torch.bfloat16)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    got = O.quantize_fp8_with_scale(x, s)
    assert np.array_equal(got, ref.view(torch.uint8).numpy())


def test_saturation_and_exact_grid_closed_forms():
    s = 2.0 ** -6
    big = O.f32_to_bf16(np.array([1000 * s, -1000 * s, 448 * s, -448 * s, 0.0], np.float32))
    assert list(O.quantize_fp8_with_scale(big, s)) == [0x7E, 0xFE, 0x7E, 0xFE, 0x00]
    # every finite e4m3 value k, times a power-of-two scale, is exact in bf16
    # and must come back as its own code
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    k = O.e4m3fn_to_f32(codes)
    xb = O.f32_to_bf16((k * np.float32(s)).astype(np.float32))
    got = O.quantize_fp8_with_scale(xb, s)
    want = np.where(codes == 0x80, 0x80, codes)  # -0 stays -0
    assert np.array_equal(got, want)


# ---- KVCache host logic (CPU tensors, no device calls) -------------------------

def test_kvcache_allocator_and_indices_on_host():
    from amd_optimization_challenge_amd.kv_cache import KVCache

    c = KVCache(8, device="cpu", scale_cols=24)
    assert c.free_slots == 8 and c.fp4_scales.shape == (8, 24)
    a = c.allocate(3)
    assert a == [0, 1, 2] and c.free_slots == 5
    c._seqs["s0"] = a
    c._seqs["s1"] = c.allocate(2)
    indptr, indices = c.indices(["s1", "s0", "missing"])
    assert indptr.tolist() == [0, 2, 5, 5]
    assert indices.tolist() == [3, 4, 0, 1, 2]
    c.release("s0")
    assert c.free_slots == 6
    assert c.allocate(3) == [0, 1, 2]  # released slots are reused lowest first
    with pytest.raises(MemoryError):
        c.allocate(4)
    kv = c.kv_data()
    assert kv["fp8"][0].dtype == torch.float8_e4m3fn and kv["mxfp4"][0].shape == (8, 1, 288)


def test_kvcache_refuses_host_tensors_and_keeps_its_slots():
    from amd_optimization_challenge_amd.kv_cache import KVCache

    c = KVCache(4, formats=("mxfp4",), device="cpu")
    with pytest.raises(ValueError):
        c.append("s", torch.zeros((2, 576), dtype=torch.bfloat16))
    assert c.free_slots == 4 and c.seq_len("s") == 0
    with pytest.raises(ValueError):
        KVCache(4, formats=("bf16",), device="cpu")
    with pytest.raises(ValueError):
        KVCache(4, device="cpu", scale_cols=17)
