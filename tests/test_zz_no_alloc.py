"""mla_decode_fwd_noalloc (workspace = the library's static device scratch)
against mla_decode_fwd with a caller workspace: bit-identical outputs and lse
on two calls in a row, the second smaller, and the clear error for a shape
whose workspace exceeds the scratch.  Both calls go through the C ABI."""
import numpy as np
import pytest
import torch

from amd_optimization_challenge_amd import _lib, ops
from mla_cases import assert_close, device_data, host_case
from oracle import mla_oracle as O

pytestmark = pytest.mark.gpu

CASES = [  # (lens, heads, kv_mode, q_seq_len); the second call of each pair is smaller
    (([900, 40, 3000, 7, 1], 16, "fp8", 1), ([300, 2], 16, "fp8", 1)),
    (([700, 1500, 64], 128, "fp8", 1), ([65, 1], 128, "fp8", 1)),
    (([2000, 333, 5, 70], 16, "mxfp4", 2), ([129, 40], 16, "mxfp4", 1)),
    (([1200, 9, 400], 128, "mxfp4k_fp8v", 1), ([100], 128, "mxfp4k_fp8v", 1)),
]


def _run_pair(lens, heads, mode, qlen, seed):
    case = host_case(lens, heads, mode, seed)
    q, kv, indptr, idx, qb, caches = case
    rows = len(lens) * qlen
    if qlen > 1:  # q_seq_len rows per sequence: draw the extra query rows
        g = torch.Generator().manual_seed(seed + 1)
        q = torch.randn((rows, heads, 576), generator=g).to(torch.bfloat16)
        qb = O.bf16_tensor_bits(q)
    data = device_data(q, kv, indptr, idx, caches, mode, 0.0721)
    qd, kv_data, _, indptr_d, cfg = data
    ref_out, ref_lse = ops.decode_fwd(qd, kv_data, indptr_d, cfg["kv_indices"], cfg["sm_scale"], mode,
                                      q_seq_len=qlen, return_lse=True)
    out = torch.full_like(ref_out, 7.0)
    got_out, got_lse = ops.decode_fwd_noalloc(qd, kv_data, indptr_d, cfg["kv_indices"], cfg["sm_scale"], mode,
                                              out=out, q_seq_len=qlen, return_lse=True)
    torch.cuda.synchronize()
    assert got_out.data_ptr() == out.data_ptr()
    assert torch.equal(got_out, ref_out), "no-alloc output differs from the workspace entry point"
    assert torch.equal(got_lse, ref_lse), "no-alloc lse differs from the workspace entry point"
    _, ref = O.reference_path(qb, mode, caches, indptr.numpy(), idx.numpy(), cfg["sm_scale"], q_seq_len=qlen)
    assert_close(got_out.float().cpu().numpy(), ref)


@pytest.mark.parametrize("pair", CASES, ids=lambda p: f"H{p[0][1]}-{p[0][2]}")
def test_noalloc_matches_workspace_entry(cuda, pair):
    for i, (lens, heads, mode, qlen) in enumerate(pair):
        print(f"noalloc H={heads} mode={mode} qlen={qlen} lens={lens} (call {i + 1})", flush=True)
        _run_pair(lens, heads, mode, qlen, seed=11 + 7 * i + heads)


def test_noalloc_rejects_oversized_shape(cuda):
    print("noalloc oversized shape", flush=True)
    lib = _lib.load()
    n = __import__("ctypes").c_int64(0)
    assert lib.mla_workspace_bytes(4096, 128, 0, __import__("ctypes").byref(n)) == 0
    assert n.value > lib.mla_noalloc_scratch_bytes()
    q = torch.zeros((4096, 128, 576), dtype=torch.bfloat16, device=cuda)
    indptr = torch.zeros(4097, dtype=torch.int32, device=cuda)
    fp8 = torch.zeros((1, 1, 576), dtype=torch.float8_e4m3fn, device=cuda)
    sc = torch.ones(1, dtype=torch.float32, device=cuda)
    with pytest.raises(_lib.MlaLibraryError, match="64|workspace"):
        ops.decode_fwd_noalloc(q, {"fp8": (fp8, sc)}, indptr, None, 0.1, "fp8")


@pytest.mark.parametrize("heads,mode", [(16, "fp8"), (128, "fp8"), (128, "mxfp4k_fp8v")])
def test_noalloc_replays_under_graph_capture(cuda, heads, mode):
    """The no-alloc entry point captured in a HIP graph (after one eager call
    on the device, which resolves the scratch address): every replay, with
    eager work between replays, equals the eager result bit for bit."""
    print(f"noalloc graph capture H={heads} mode={mode}", flush=True)
    q, kv, indptr, idx, qb, caches = host_case([900, 40, 333], heads, mode, seed=71)
    qd, kv_data, _, indptr_d, cfg = device_data(q, kv, indptr, idx, caches, mode, 0.0721)
    args = (qd, kv_data, indptr_d, cfg["kv_indices"], cfg["sm_scale"], mode)
    eager = ops.decode_fwd_noalloc(*args, out=torch.empty((3, heads, 512), dtype=torch.bfloat16, device=cuda))
    torch.cuda.synchronize()
    eager = eager.clone()
    out = torch.empty_like(eager)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.decode_fwd_noalloc(*args, out=out)
    for rep in range(3):
        out.fill_(rep + 1.0)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep} differs from the eager call"
    del g
