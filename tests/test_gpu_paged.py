"""Paged caches (AITER's page_size / kv_last_page_lens arguments,
mixed-mla/asm_dumps/aiter_mla.py:149-175): the device page-table expansion
(mla_expand_pages) against the oracle's, bit for bit, and whole decodes over a
paged cache against the oracle at the decode tolerance."""
import math

import numpy as np
import pytest
import torch

from amd_optimization_challenge_amd import custom_kernel, ops
from mla_cases import assert_close, case_from_tensors, device_data
from oracle import mla_oracle as O

pytestmark = pytest.mark.gpu


def _page_table(lens, P, spare, seed):
    rng = np.random.default_rng(seed)
    npages = [(L + P - 1) // P for L in lens]
    perm = rng.permutation(sum(npages) + spare).astype(np.int64)
    starts = np.concatenate([[0], np.cumsum(npages)])
    return O.page_table(lens, P, lambda b, n: perm[starts[b]:starts[b] + n]), sum(npages) + spare


@pytest.mark.parametrize("P", [2, 8, 16, 64])
def test_expand_pages_matches_oracle(cuda, P):
    lens = [0, 1, P, P + 1, 5 * P - 3, 2000, 0, 37, 1]
    print(f"expand pages P={P}", flush=True)
    (indptr, ids, last), _ = _page_table(lens, P, 7, P)
    last = last.copy()
    last[1] = 0  # clamped to 1
    last[3] = P + 5  # clamped to P
    want_indptr, want_idx = O.expand_pages(indptr, ids, last, P)
    dev = torch.device("cuda")
    kv_indptr, kv_indices = ops.expand_pages(torch.from_numpy(indptr).to(dev), torch.from_numpy(ids).to(dev),
                                             torch.from_numpy(last).to(dev), P)
    torch.cuda.synchronize()
    got_indptr = kv_indptr.cpu().numpy()
    assert np.array_equal(got_indptr, want_indptr)
    assert np.array_equal(kv_indices.cpu().numpy()[:got_indptr[-1]], want_idx)


def test_expand_pages_empty_batch_entries(cuda):
    dev = torch.device("cuda")
    indptr = torch.zeros(4, dtype=torch.int32, device=dev)
    ids = torch.zeros(0, dtype=torch.int32, device=dev)
    last = torch.ones(3, dtype=torch.int32, device=dev)
    kv_indptr, _ = ops.expand_pages(indptr, ids, last, 16)
    torch.cuda.synchronize()
    assert kv_indptr.cpu().tolist() == [0, 0, 0, 0]


MODES = [(16, "fp8"), (16, "mxfp4"), (16, "mxfp4k_fp8v"), (128, "fp8"), (128, "mxfp4k_fp8v")]


@pytest.mark.parametrize("P", [2, 8, 16])
@pytest.mark.parametrize("heads,mode", MODES)
def test_paged_decode_matches_oracle(cuda, heads, mode, P):
    lens = [63, 0, 300, 1024, 5]
    print(f"paged decode H={heads} mode={mode} P={P}", flush=True)
    (indptr, ids, last), npages = _page_table(lens, P, 5, 100 + P)
    rows = npages * P
    g = torch.Generator().manual_seed(P * 7 + heads)
    q = torch.randn(len(lens), heads, 576, generator=g).to(torch.bfloat16)
    kv = torch.randn(rows, 1, 576, generator=g).to(torch.bfloat16)  # the physical cache, every row
    _, kv_indices = O.expand_pages(indptr, ids, last, P)
    kv_indptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    case = case_from_tensors(q, kv, torch.from_numpy(kv_indptr), torch.from_numpy(kv_indices), mode)
    _, _, _, _, qb, caches = case
    sm = 1 / math.sqrt(576)
    q_d, kv_data, qo_indptr, _, cfg = device_data(q, kv, torch.from_numpy(kv_indptr),
                                                  torch.from_numpy(kv_indices), caches, mode, sm)
    dev = torch.device("cuda")
    paged = {}
    for key, val in kv_data.items():
        if key == "bf16":
            continue
        cache, extra = val
        cache = cache.reshape(npages, P, 1, cache.shape[-1])
        if key == "mxfp4":
            extra = extra.reshape(npages, P, extra.shape[-1])
        paged[key] = (cache, extra)
    cfg = dict(cfg, page_size=P, kv_indices=torch.from_numpy(ids).to(dev),
               kv_last_page_lens=torch.from_numpy(last).to(dev))
    out = custom_kernel((q_d, paged, qo_indptr, torch.from_numpy(indptr).to(dev), cfg))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    _, ref = O.reference_path(qb, mode, caches, kv_indptr, kv_indices, sm)
    assert np.all(np.isfinite(got))
    assert_close(got, ref)
    assert np.all(got[1] == 0)  # the empty sequence
