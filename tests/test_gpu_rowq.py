"""The per-row Q route (``mla_decode_fwd_rowq``): bf16 Q quantized per head
row inside the 16-head decode, which for up to 256 query rows also plans its
own work (decode + combine, two launches).  Parity against the oracle's
per-row path (atol = rtol = 2e-2 and rel-L2), indexed and contiguous, both
caches, short / ragged / empty rows, past 64 rows (the block plans in the
kernel), past 256 (the planner kernel runs first), causal rows with LSE; the
plan the decode's work-group 0 leaves in the workspace equals the planner
kernel's for the same target."""
import math

import numpy as np
import pytest
import torch

from amd_optimization_challenge_amd import custom_kernel, ops
from mla_cases import assert_close, device_data, host_case
from oracle import mla_oracle as O

pytestmark = pytest.mark.gpu
SM = 1 / math.sqrt(192)


@pytest.mark.parametrize("contig", [False, True])
@pytest.mark.parametrize("mode", ["fp8", "mxfp4"])
@pytest.mark.parametrize("lens", [[1, 63, 64, 65], [3000, 10, 129, 700, 1], [0, 200, 7], [1024] * 32,
                                  [(i * 37) % 700 + 1 for i in range(80)], [96] * 256,
                                  [0 if i % 11 == 0 else (i * 53) % 400 + 1 for i in range(200)],
                                  [(i * 13) % 90 + 1 for i in range(300)]])
def test_rowq_matches_oracle(cuda, mode, lens, contig):
    print(f"rowq mode={mode} B={len(lens)} contig={contig}", flush=True)
    q, kv, indptr, idx, qb, caches = host_case(lens, 16, mode, seed=len(lens) + 3, permute=not contig)
    qd, kv_data, _, kv_indptr, cfg = device_data(q, kv, indptr, idx, caches, mode, SM, pass_indices=not contig)
    out = ops.decode_fwd(qd, kv_data, kv_indptr, cfg["kv_indices"], SM, mode, q_dtype="fp8_row")
    torch.cuda.synchronize()
    _, ref = O.reference_path(qb, mode, caches, indptr.numpy(), idx.numpy(), SM, q_dtype="fp8_row")
    got = out.float().cpu().numpy()
    assert_close(got, ref)
    for b, L in enumerate(lens):
        if L == 0:
            assert np.all(got[b] == 0)


@pytest.mark.parametrize("mode", ["fp8", "mxfp4"])
@pytest.mark.parametrize("qlen,lens", [(2, [300, 7, 1, 64, 2000, 2]), (4, [300, 7, 1, 64, 2000, 2]),
                                       (4, [(i * 29) % 240 + 4 for i in range(40)])])
def test_rowq_causal_rows_and_lse(cuda, mode, qlen, lens):
    """Causal multi-token rows: 12 and 24 query rows (the wave plans) and 160
    (the block plans)."""
    print(f"rowq causal mode={mode} qlen={qlen} S={len(lens)}", flush=True)
    S = len(lens)
    g = torch.Generator().manual_seed(200 + qlen)
    q = torch.randn(S * qlen, 16, 576, generator=g).to(torch.bfloat16)
    _, kv, indptr, idx, _, caches = host_case(lens, 16, mode, seed=9 + qlen)
    qb = O.bf16_tensor_bits(q)
    dev = torch.device("cuda")
    _, kv_data, _, kv_indptr, cfg = device_data(q[:S], kv, indptr, idx, caches, mode, 0.08)
    out, lse = ops.decode_fwd(q.to(dev), kv_data, kv_indptr, cfg["kv_indices"], 0.08, mode, q_seq_len=qlen,
                              return_lse=True, q_dtype="fp8_row")
    torch.cuda.synchronize()
    _, ref, ref_lse = O.reference_path(qb, mode, caches, indptr.numpy(), idx.numpy(), 0.08, q_seq_len=qlen,
                                       return_lse=True, q_dtype="fp8_row")
    assert_close(out.float().cpu().numpy(), ref)
    inf_ref = np.isneginf(ref_lse)
    got_lse = lse.cpu().numpy()
    assert np.array_equal(np.isneginf(got_lse), inf_ref)
    assert np.all(np.abs(got_lse[~inf_ref] - ref_lse[~inf_ref]) <= 1e-2 + 1e-2 * np.abs(ref_lse[~inf_ref]))


@pytest.mark.parametrize("mode", ["fp8", "mxfp4"])
@pytest.mark.parametrize("lens", [[3000, 10, 129, 700, 1], [(i * 7919) % 9000 + 1 for i in range(64)], [5] * 3,
                                  [(i * 7919) % 3000 + 1 for i in range(200)], [512] * 256,
                                  [0 if i % 7 == 0 else (i * 31) % 1500 + 1 for i in range(130)]])
def test_in_kernel_plan_equals_planner_kernel(cuda, mode, lens):
    """Indexed rows: the in-kernel plan targets what mla_plan targets, so the
    rows' (first item, piece count) and the header the decode's work-group 0
    writes are the planner kernel's, word for word."""
    print(f"in-kernel plan mode={mode} B={len(lens)}", flush=True)
    q, kv, indptr, idx, qb, caches = host_case(lens, 16, mode, seed=5)
    qd, kv_data, _, kv_indptr, cfg = device_data(q, kv, indptr, idx, caches, mode, SM)
    B = len(lens)
    ws = ops.workspace(B, 16, mode, cuda)
    ws.fill_(0x5A)
    ops.decode_fwd(qd, kv_data, kv_indptr, cfg["kv_indices"], SM, mode, ws=ws, q_dtype="fp8_row")
    torch.cuda.synchronize()
    mine = ops.read_plan(ws, B, 16, mode)
    ws2 = ops.workspace(B, 16, mode, cuda).clone()
    ops.plan(kv_indptr, B, 16, mode, ws2)
    torch.cuda.synchronize()
    ref = ops.read_plan(ws2, B, 16, mode)
    for k in ("num_items", "chunk", "total", "batch", "max_items"):
        assert mine[k] == ref[k], k
    assert torch.equal(mine["batch_info"], ref["batch_info"])


def test_auto_route_small_batch_is_two_launches_and_in_tolerance(cuda):
    """kv_mode 'auto' at 16 heads runs this route: within 2e-2 of the oracle's
    per-row path on a contiguous batch (the task's shape)."""
    lens = [1024] * 4
    q, kv, indptr, idx, qb, caches = host_case(lens, 16, "mxfp4", seed=1, permute=False)
    data = device_data(q, kv, indptr, idx, caches, "mxfp4", SM, pass_indices=False)
    qd, kv_data, qo, kv_indptr, cfg = data
    got = custom_kernel((qd, kv_data, qo, kv_indptr, dict(cfg, kv_mode="auto"))).float().cpu().numpy()
    _, ref = O.reference_path(qb, "mxfp4", caches, indptr.numpy(), idx.numpy(), SM, q_dtype="fp8_row")
    assert_close(got, ref)
