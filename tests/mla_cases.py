"""Shared helpers for the GPU parity tests: build a decode case on the host
with the oracle's caches, run the HIP path, and compute the oracle output."""
import math

import numpy as np
import torch

from amd_optimization_challenge_amd import custom_kernel, inputs
from oracle import mla_oracle as O

TOL = 2e-2  # north-star tolerance on the bf16 output: atol = rtol = 2e-2


def host_case(lens, heads, kv_mode, seed, permute=True):
    q, kv, indptr, idx = inputs.make_host_inputs(len(lens), heads, ("list", lens), seed, permute)
    return case_from_tensors(q, kv, indptr, idx, kv_mode)


def case_from_tensors(q, kv, indptr, idx, kv_mode):
    """Oracle caches (bit-exact quantizers) for given bf16 q [B,H,576] / kv [T,1,576]."""
    qb = O.bf16_tensor_bits(q)
    kvb = O.bf16_tensor_bits(kv).reshape(-1, 576)
    caches = {}
    if kv_mode in ("fp8", "mxfp4k_fp8v"):
        c, s = O.quantize_fp8_per_tensor(kvb)
        caches.update(fp8_codes=c, fp8_scale=s)
    if kv_mode in ("mxfp4", "mxfp4k_fp8v"):
        p, e = O.pack_mxfp4(kvb)
        caches.update(fp4_packed=p, fp4_scales=e)
    return q, kv, indptr, idx, qb, caches


def device_data(q, kv, indptr, idx, caches, kv_mode, sm_scale, pass_indices=True):
    dev = torch.device("cuda")
    T = kv.shape[0]
    kv_data = {"bf16": kv.to(dev)}
    if "fp8_codes" in caches:
        kv_data["fp8"] = (torch.from_numpy(caches["fp8_codes"].reshape(T, 1, 576)).to(dev)
                          .view(torch.float8_e4m3fn),
                          torch.tensor([caches["fp8_scale"]], dtype=torch.float32, device=dev))
    if "fp4_packed" in caches:
        kv_data["mxfp4"] = (torch.from_numpy(caches["fp4_packed"].reshape(T, 1, 288)).to(dev)
                            .view(torch.float4_e2m1fn_x2),
                            torch.from_numpy(caches["fp4_scales"]).to(dev).view(torch.float8_e8m0fnu))
    B = q.shape[0]
    cfg = inputs.make_config(B, q.shape[1], int(indptr[-1]), kv_mode, sm_scale,
                             idx.to(dev) if pass_indices else None, 0)
    return (q.to(dev), kv_data, torch.arange(B + 1, dtype=torch.int32, device=dev), indptr.to(dev), cfg)


def run_and_reference(lens, heads, kv_mode, seed=0, sm_scale=1 / math.sqrt(192), permute=True):
    return run_case(host_case(lens, heads, kv_mode, seed, permute), kv_mode, sm_scale)


def run_case(case, kv_mode, sm_scale):
    q, kv, indptr, idx, qb, caches = case
    data = device_data(q, kv, indptr, idx, caches, kv_mode, sm_scale)
    out = custom_kernel(data)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    _, ref = O.reference_path(qb, kv_mode, caches, indptr.numpy(), idx.numpy(), sm_scale)
    return got, ref, data


def assert_close(got, ref, tol=TOL, rel_l2=0.03):
    ref_b = O.bf16_to_f32(O.f32_to_bf16(ref))
    err = np.abs(got - ref_b)
    bad = err > tol + tol * np.abs(ref_b)
    nrm = np.linalg.norm(ref)
    rl2 = float(np.linalg.norm(got - ref) / nrm) if nrm > 0 else float(np.linalg.norm(got))
    assert not bad.any(), f"{int(bad.sum())} elements outside atol=rtol={tol}; max err {err.max():.3e}"
    assert rl2 < rel_l2, f"relative L2 error {rl2:.3e}"
    return rl2
