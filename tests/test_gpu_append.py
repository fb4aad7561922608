"""KV-cache append writer (mla_append_kv) on the device: bit-exact against the
oracle writer and against the whole-buffer quantizers, and a decode through an
incrementally built cache (KVCache) against the oracle."""
import math

import numpy as np
import pytest
import torch

from amd_optimization_challenge_amd import custom_kernel, inputs, ops
from amd_optimization_challenge_amd.kv_cache import KVCache
from oracle import mla_oracle as O

from mla_cases import assert_close

pytestmark = pytest.mark.gpu


def to_dev_bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def rand_bits(n, seed, mult=1.0):
    rng = np.random.default_rng(seed)
    return O.f32_to_bf16((rng.standard_normal((n, 576)) * mult).astype(np.float32))


def u8(t):
    return t.view(torch.uint8).cpu().numpy()


@pytest.mark.parametrize("scale_cols", [18, 24])
def test_append_matches_oracle_writer(cuda, scale_cols):
    """Ragged chunks, permuted and skipped slots, a scale that saturates some
    tokens, padded e8m0 rows: every byte and the running max equal the oracle's."""
    print(f"append vs oracle scale_cols={scale_cols}", flush=True)
    n, cap = 300, 420
    x = rand_bits(n, 11, mult=4.0)
    scale = np.float32(O.bf16_to_f32(np.array([0x3C00], np.uint16))[0])  # 2^-7: |x| > 3.5 saturates
    rng = np.random.default_rng(12)
    slots = rng.permutation(cap)[:n].astype(np.int32)
    slots[[5, 77, 299]] = -1
    f8_ref = np.full((cap, 576), 0xAB, np.uint8)
    f4_ref = np.full((cap, 288), 0xCD, np.uint8)
    sc_ref = np.full((cap, scale_cols), 0xEE, np.uint8)
    f8 = torch.from_numpy(f8_ref.copy()).cuda().view(torch.float8_e4m3fn).reshape(cap, 1, 576)
    f4 = torch.from_numpy(f4_ref.copy()).cuda().reshape(cap, 1, 288)
    sc = torch.from_numpy(sc_ref.copy()).cuda()
    sc_t = torch.tensor([scale], dtype=torch.float32, device=cuda)
    amax = torch.zeros(1, dtype=torch.int32, device=cuda)
    xd = to_dev_bf16(x)
    sd = torch.from_numpy(slots).cuda()
    want_amax = 0
    for lo, hi in ((0, 1), (1, 64), (64, 65), (65, 200), (200, 300)):
        ops.append_kv(xd[lo:hi], sd[lo:hi], fp8=(f8, sc_t), mxfp4=(f4, sc), amax=amax)
        want_amax = max(want_amax, O.append_kv(x[lo:hi], slots[lo:hi], f8_ref, scale, f4_ref, sc_ref))
    torch.cuda.synchronize()
    assert np.array_equal(u8(f8).reshape(cap, 576), f8_ref)
    assert np.array_equal(u8(f4).reshape(cap, 288), f4_ref)
    assert np.array_equal(sc.cpu().numpy(), sc_ref)
    assert int(amax.item()) == want_amax
    assert (f8_ref == 0x7E).any() and (f8_ref == 0xFE).any()  # the case does saturate


@pytest.mark.parametrize("n", [1, 17, 4096, 131072])
def test_append_equals_whole_buffer_build(cuda, n):
    """Appending every row with the whole buffer's scale writes the bytes of the
    whole-buffer quantizers (size-independent property, up to 151 MB of input)."""
    print(f"append vs whole build n={n}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(n)
    x = torch.randn((n, 1, 576), generator=g, dtype=torch.bfloat16).cuda()
    whole8, s = ops.quant_fp8_per_tensor(x)
    whole4, e8 = ops.pack_mxfp4(x.reshape(n, 576))
    perm = torch.randperm(n, generator=g).to(torch.int32).cuda()
    f8 = torch.zeros_like(whole8)
    f4 = torch.zeros((n, 1, 288), dtype=torch.uint8, device=cuda)
    sc = torch.zeros((n, 18), dtype=torch.uint8, device=cuda)
    ops.append_kv(x, perm, fp8=(f8, s), mxfp4=(f4, sc))
    torch.cuda.synchronize()
    assert torch.equal(f8.view(torch.uint8)[perm.long()], whole8.view(torch.uint8))
    assert torch.equal(f4.reshape(n, 288)[perm.long()], whole4)
    assert torch.equal(sc[perm.long()], e8)


def test_append_edge_cases(cuda):
    x = torch.zeros((0, 576), dtype=torch.bfloat16, device=cuda)
    f4 = torch.zeros((4, 1, 288), dtype=torch.uint8, device=cuda)
    sc = torch.zeros((4, 18), dtype=torch.uint8, device=cuda)
    ops.append_kv(x, None, mxfp4=(f4, sc))  # n = 0 is a no-op
    with pytest.raises(ValueError):
        ops.append_kv(x, None)
    # all-zero and single-token rows: e8m0 127-127 rule for zero blocks
    z = torch.zeros((1, 576), dtype=torch.bfloat16, device=cuda)
    ops.append_kv(z, torch.tensor([2], dtype=torch.int32, device=cuda), mxfp4=(f4, sc))
    torch.cuda.synchronize()
    _, e8_ref = O.pack_mxfp4(np.zeros((1, 576), np.uint16))
    assert np.array_equal(sc[2].cpu().numpy(), e8_ref[0])
    assert not f4.any()


@pytest.mark.parametrize("kv_mode", ["fp8", "mxfp4", "mxfp4k_fp8v"])
def test_decode_through_incrementally_built_cache(cuda, kv_mode):
    """Prefill + three decode steps appended per sequence (slots interleave across
    sequences), then the decode over kv_indices from the cache equals both the
    decode over the whole-buffer caches (bit for bit) and the oracle (2e-2)."""
    print(f"KVCache decode kv_mode={kv_mode}", flush=True)
    lens = [37, 1, 300, 64, 129, 513]
    steps = 3
    heads = 16
    sm = 1 / math.sqrt(192)
    g = torch.Generator().manual_seed(21)
    per_seq = [torch.randn((L, 576), generator=g, dtype=torch.bfloat16) for L in lens]
    q = torch.randn((len(lens), heads, 576), generator=g, dtype=torch.bfloat16)
    kv_all = torch.cat(per_seq)  # sequence-major, the whole-buffer order
    _, s_whole = O.quantize_fp8_per_tensor(O.bf16_tensor_bits(kv_all))

    cache = KVCache(sum(lens) + 50, device=cuda, scale_cols=20, fp8_scale=float(s_whole))
    for b, L in enumerate(lens):
        pre = max(L - steps, 0)
        if pre:
            cache.append(b, per_seq[b][:pre].cuda())
    for t in range(steps):
        for b, L in enumerate(lens):
            i = max(L - steps, 0) + t
            if i < L:
                cache.append(b, per_seq[b][i:i + 1].cuda())
    assert [cache.seq_len(b) for b in range(len(lens))] == lens
    assert not cache.fp8_saturated()
    kv_indptr, kv_indices = cache.indices(range(len(lens)))
    cfg = inputs.make_config(len(lens), heads, sum(lens), kv_mode, sm, kv_indices, max(lens))
    qd = q.cuda()
    qo = torch.arange(len(lens) + 1, dtype=torch.int32, device=cuda)
    out_inc = custom_kernel((qd, cache.kv_data(), qo, kv_indptr, cfg)).clone()

    whole = inputs.build_kv_data(kv_all.reshape(-1, 1, 576).cuda(), kv_mode)
    cfg_w = dict(cfg, kv_indices=None)
    out_whole = custom_kernel((qd, whole, qo, kv_indptr, cfg_w))
    torch.cuda.synchronize()
    assert torch.equal(out_inc, out_whole)

    kvb = O.bf16_tensor_bits(kv_all).reshape(-1, 576)
    caches = {}
    if kv_mode in ("fp8", "mxfp4k_fp8v"):
        c, s = O.quantize_fp8_per_tensor(kvb)
        caches.update(fp8_codes=c, fp8_scale=s)
    if kv_mode in ("mxfp4", "mxfp4k_fp8v"):
        p, e = O.pack_mxfp4(kvb)
        caches.update(fp4_packed=p, fp4_scales=e)
    _, ref = O.reference_path(O.bf16_tensor_bits(q), kv_mode, caches, kv_indptr.cpu().numpy(),
                              np.arange(sum(lens), dtype=np.int32), sm)
    assert_close(out_inc.float().cpu().numpy(), ref)


def test_kvcache_calibrates_on_first_append_and_reports_saturation(cuda):
    g = torch.Generator().manual_seed(5)
    pre = torch.randn((64, 576), generator=g, dtype=torch.bfloat16)
    cache = KVCache(80, formats=("fp8",), device=cuda)
    cache.append("a", pre.cuda())
    _, s = O.quantize_fp8_per_tensor(O.bf16_tensor_bits(pre))
    assert float(cache.fp8_scale.item()) == float(s)
    assert not cache.fp8_saturated()
    cache.append("a", (pre[:1] * 4).cuda())  # 4x the prefill's max: clamped
    assert cache.fp8_saturated()
    assert cache.seq_len("a") == 65 and cache.free_slots == 15


def test_fp8_fixed_scale_exhaustive(cuda):
    """Every finite bf16 value (and +-inf) through the fp8 writer at ~600
    scales -- random f32 mantissas over 2^-40..2^20, bf16 scales, and the
    edges where the kernel's reciprocal shortcut is switched off (|s| outside
    [2^-125, 2^125], subnormal s) -- against the oracle's x / s."""
    allb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    bits = allb[~(((allb & 0x7F80) == 0x7F80) & ((allb & 0x7F) != 0))]
    n_tok = -(-bits.size // 576)
    rows = np.zeros(n_tok * 576, np.uint16)
    rows[:bits.size] = bits
    x = to_dev_bf16(rows.reshape(n_tok, 576))
    rng = np.random.default_rng(77)
    scales = list((rng.uniform(1, 2, 500) * np.exp2(rng.integers(-40, 21, 500))).astype(np.float32))
    scales += list(O.bf16_to_f32(rng.integers(0x2000, 0x4A00, 80).astype(np.uint16)))
    scales += [np.float32(v) for v in (2.0 ** -125, 2.0 ** -125 * 0.99, 2.0 ** -126, 1e-40, 2.0 ** 125,
                                       2.0 ** 125 * 1.01, 3e38, 1.0, 448.0, 1 / 448.0)]
    f8 = torch.zeros((n_tok, 1, 576), dtype=torch.float8_e4m3fn, device=cuda)
    st = torch.tensor(np.array(scales, np.float32), device=cuda)
    outs = []
    for i in range(len(scales)):
        ops.append_kv(x, None, fp8=(f8, st[i:i + 1]))
        outs.append(f8.view(torch.uint8).reshape(-1)[:bits.size].clone())
    got = torch.stack(outs).cpu().numpy()
    for i, s in enumerate(scales):
        want = O.quantize_fp8_with_scale(bits, s)
        bad = np.nonzero(got[i] != want)[0]
        assert bad.size == 0, (float(s), [(hex(int(bits[j])), int(got[i][j]), int(want[j])) for j in bad[:8]])
