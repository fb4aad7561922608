"""The a16w8 route (bf16 Q, fp8 cache, no per-tensor Q scale;
mla_decode_fwd_a16w8) against the oracle with Q unquantized (TASK/reference.py
:55-58 Q_DTYPE = bf16), at the decode tolerance, plus a precision pin: with
head rows of very different magnitude, per-tensor fp8 Q (a8w8) loses the small
rows and this route does not."""
import math

import numpy as np
import pytest
import torch

from amd_optimization_challenge_amd import _lib, custom_kernel
from mla_cases import assert_close, device_data, host_case
from oracle import mla_oracle as O

pytestmark = pytest.mark.gpu


def _run(case, sm, q_dtype, q_seq_len=1, return_lse=False):
    q, kv, indptr, idx, qb, caches = case
    data = device_data(q, kv, indptr, idx, caches, "fp8", sm)
    cfg = dict(data[4], q_dtype=q_dtype, q_seq_len=q_seq_len, return_lse=return_lse)
    res = custom_kernel(data[:4] + (cfg,))
    torch.cuda.synchronize()
    return res


@pytest.mark.parametrize("lens", [[1], [63, 64, 65], [0, 200, 7], [3000, 10, 129], [1024] * 5])
def test_a16w8_matches_bf16_q_oracle(cuda, lens):
    print(f"a16w8 lens={lens[:4]}", flush=True)
    case = host_case(lens, 16, "fp8", seed=len(lens) * 7 + 3)
    sm = 1 / math.sqrt(576)
    got = _run(case, sm, "bf16").float().cpu().numpy()
    _, _, indptr, idx, qb, caches = case
    _, ref = O.reference_path(qb, "fp8", caches, indptr.numpy(), idx.numpy(), sm, q_dtype="bf16")
    assert np.all(np.isfinite(got))
    assert_close(got, ref)
    for b, L in enumerate(lens):
        if L == 0:
            assert np.all(got[b] == 0)


def test_a16w8_keeps_small_head_rows(cuda):
    """Heads scaled by 2^-12 .. 2^3: one tensor-wide fp8 scale flushes the small
    rows' q towards zero (their scores collapse); per-row scales keep them."""
    print("a16w8 row-scale pin", flush=True)
    case = host_case([500, 300, 77], 16, "fp8", seed=11)
    q, kv, indptr, idx, qb, caches = case
    g = torch.Generator().manual_seed(3)
    scale = torch.pow(2.0, torch.linspace(-12, 3, 16))
    q2 = (q.float() * 6.0 * scale[None, :, None] + 0.0 * torch.randn(q.shape, generator=g)).to(torch.bfloat16)
    case2 = (q2, kv, indptr, idx, O.bf16_tensor_bits(q2), caches)
    sm = 1 / math.sqrt(576)
    _, ref = O.reference_path(case2[4], "fp8", caches, indptr.numpy(), idx.numpy(), sm, q_dtype="bf16")
    a16 = _run(case2, sm, "bf16").float().cpu().numpy()
    a8 = _run(case2, sm, "fp8").float().cpu().numpy()
    e16 = np.linalg.norm(a16 - ref) / np.linalg.norm(ref)
    e8 = np.linalg.norm(a8 - ref) / np.linalg.norm(ref)
    print(f"rel L2 vs bf16-Q oracle: a16w8 {e16:.2e}, a8w8 {e8:.2e}", flush=True)
    assert_close(a16, ref)
    assert e16 < 0.25 * e8


def test_a16w8_multi_token_rows_and_lse(cuda):
    print("a16w8 q_seq_len 2 + lse", flush=True)
    lens = [300, 64, 9]
    qlen = 2
    case = host_case(lens, 16, "fp8", seed=5)
    q, kv, indptr, idx, qb, caches = case
    g = torch.Generator().manual_seed(9)
    q2 = torch.randn(len(lens) * qlen, 16, 576, generator=g).to(torch.bfloat16)
    case2 = (q2, kv, indptr, idx, O.bf16_tensor_bits(q2), caches)
    sm = 1 / math.sqrt(576)
    data = device_data(q2, kv, indptr, idx, caches, "fp8", sm)
    cfg = dict(data[4], q_dtype="bf16", q_seq_len=qlen, return_lse=True)
    qo = torch.arange(len(lens) + 1, dtype=torch.int32, device="cuda") * qlen
    out, lse = custom_kernel((data[0], data[1], qo, data[3], cfg))
    torch.cuda.synchronize()
    _, ref, ref_lse = O.reference_path(case2[4], "fp8", caches, indptr.numpy(), idx.numpy(), sm, q_seq_len=qlen,
                                       return_lse=True, q_dtype="bf16")
    assert_close(out.float().cpu().numpy(), ref)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("heads,mode", [(128, "fp8"), (16, "mxfp4")])
def test_a16w8_unsupported_shapes_raise(cuda, heads, mode):
    case = host_case([64], heads, mode, seed=1)
    q, kv, indptr, idx, qb, caches = case
    data = device_data(q, kv, indptr, idx, caches, mode, 0.1)
    with pytest.raises(_lib.MlaLibraryError):
        custom_kernel(data[:4] + (dict(data[4], q_dtype="bf16"),))
