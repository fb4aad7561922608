"""The bf16 cache (a16w16: TASK/reference.py:55-58 KV_DTYPE = bf16, Q bf16)
against the oracle with nothing quantized, at the decode tolerance; multi-token
rows with lse; a paged bf16 cache; the shapes it refuses."""
import math

import numpy as np
import pytest
import torch

from amd_optimization_challenge_amd import _lib, custom_kernel, inputs
from mla_cases import assert_close
from oracle import mla_oracle as O

pytestmark = pytest.mark.gpu


def _case(lens, heads, seed, qlen=1):
    g = torch.Generator().manual_seed(seed)
    T = sum(lens)
    q = torch.randn(len(lens) * qlen, heads, 576, generator=g).to(torch.bfloat16)
    kv = torch.randn(T + 7, 1, 576, generator=g).to(torch.bfloat16)  # 7 rows no token uses
    idx = torch.randperm(T + 7, generator=g)[:T].to(torch.int32)
    indptr = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    return q, kv, indptr, idx


def _data(q, kv, indptr, idx, sm, **extra):
    dev = torch.device("cuda")
    B = indptr.numel() - 1
    cfg = inputs.make_config(B, q.shape[1], int(indptr[-1]), "bf16", sm, idx.to(dev), 0)
    cfg.update(extra)
    qlen = int(extra.get("q_seq_len", 1))
    qo = torch.arange(B + 1, dtype=torch.int32, device=dev) * qlen
    return (q.to(dev), {"bf16": kv.to(dev)}, qo, indptr.to(dev), cfg)


def _ref(q, kv, indptr, idx, sm, **kw):
    return O.reference_path(O.bf16_tensor_bits(q), "bf16", {"bf16_bits": O.bf16_tensor_bits(kv)}, indptr.numpy(),
                            idx.numpy(), sm, q_dtype="bf16", **kw)


@pytest.mark.parametrize("lens", [[1], [63, 64, 65], [0, 200, 7], [3000, 10, 129], [1024] * 5])
def test_bf16_cache_matches_oracle(cuda, lens):
    print(f"bf16 kv lens={lens[:4]}", flush=True)
    q, kv, indptr, idx = _case(lens, 16, seed=len(lens) * 13)
    sm = 1 / math.sqrt(576)
    got = custom_kernel(_data(q, kv, indptr, idx, sm))
    torch.cuda.synchronize()
    got = got.float().cpu().numpy()
    _, ref = _ref(q, kv, indptr, idx, sm)
    assert np.all(np.isfinite(got))
    assert_close(got, ref)
    for b, L in enumerate(lens):
        if L == 0:
            assert np.all(got[b] == 0)


def test_bf16_cache_wide_scores(cuda):
    """Scores spread far past one tile's offset range: the accumulator
    reference restarts, as for the fp8 caches."""
    print("bf16 kv wide scores", flush=True)
    q, kv, indptr, idx = _case([700, 130, 5], 16, seed=4)
    q = q.float()
    q[..., 7] = 40.0
    kv = kv.float()
    kv[:, 0, 7] = torch.linspace(-20, 60, kv.shape[0])
    q, kv = q.to(torch.bfloat16), kv.to(torch.bfloat16)
    sm = 1 / math.sqrt(576)
    got = custom_kernel(_data(q, kv, indptr, idx, sm))
    torch.cuda.synchronize()
    _, ref = _ref(q, kv, indptr, idx, sm)
    assert_close(got.float().cpu().numpy(), ref)


def test_bf16_cache_multi_token_rows_and_lse(cuda):
    print("bf16 kv q_seq_len 4 + lse", flush=True)
    q, kv, indptr, idx = _case([300, 64, 9], 16, seed=8, qlen=4)
    sm = 0.3
    out, lse = custom_kernel(_data(q, kv, indptr, idx, sm, q_seq_len=4, return_lse=True))
    torch.cuda.synchronize()
    _, ref, ref_lse = _ref(q, kv, indptr, idx, sm, q_seq_len=4, return_lse=True)
    assert_close(out.float().cpu().numpy(), ref)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=2e-3, atol=2e-3)


def test_bf16_cache_paged(cuda):
    print("bf16 kv paged", flush=True)
    lens, P = [100, 0, 33], 16
    npages = [(L + P - 1) // P for L in lens]
    ids = np.random.default_rng(0).permutation(sum(npages) + 3)
    starts = np.concatenate([[0], np.cumsum(npages)])
    pind, pids, last = O.page_table(lens, P, lambda b, n: ids[starts[b]:starts[b] + n])
    rows = (sum(npages) + 3) * P
    g = torch.Generator().manual_seed(2)
    q = torch.randn(len(lens), 16, 576, generator=g).to(torch.bfloat16)
    kv = torch.randn(rows, 1, 576, generator=g).to(torch.bfloat16)
    kvi, kvx = O.expand_pages(pind, pids, last, P)
    sm = 1 / math.sqrt(576)
    dev = torch.device("cuda")
    data = _data(q, kv, torch.from_numpy(kvi), torch.from_numpy(kvx), sm)
    cfg = dict(data[4], page_size=P, kv_indices=torch.from_numpy(pids).to(dev),
               kv_last_page_lens=torch.from_numpy(last).to(dev))
    out = custom_kernel((data[0], {"bf16": kv.to(dev).reshape(-1, P, 1, 576)}, data[2],
                         torch.from_numpy(pind).to(dev), cfg))
    torch.cuda.synchronize()
    _, ref = _ref(q, kv, torch.from_numpy(kvi), torch.from_numpy(kvx), sm)
    assert_close(out.float().cpu().numpy(), ref)


def test_bf16_cache_refuses_128_heads(cuda):
    q, kv, indptr, idx = _case([64], 128, seed=1)
    with pytest.raises(_lib.MlaLibraryError):
        custom_kernel(_data(q, kv, indptr, idx, 0.1))
