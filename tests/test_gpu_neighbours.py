"""The steps either side of the decode on the GPU: W_UK absorption, v_up_proj
(+ per-tensor FP8), and the three chained, against the CPU oracle."""
import math

import numpy as np
import pytest
import torch

from amd_optimization_challenge_amd import custom_kernel, neighbours as N
from mla_cases import assert_close, case_from_tensors, device_data
from oracle import mla_oracle as O

pytestmark = pytest.mark.gpu


def _close_bf16(got, ref):
    ref_b = O.bf16_to_f32(O.f32_to_bf16(ref))
    scale = float(np.abs(ref_b).max()) or 1.0
    err = np.abs(got - ref_b)
    # f32 accumulation in a different order, one bf16 rounding of the result
    assert np.all(err <= 2 ** -7 * np.abs(ref_b) + 2 ** -12 * scale), float(err.max())


@pytest.mark.parametrize("B,H", [(4, 16), (64, 128), (37, 16), (1, 128), (130, 16)])
def test_absorb_q_matches_oracle(cuda, B, H):
    print(f"absorb_q B={B} H={H}", flush=True)
    g = torch.Generator().manual_seed(B * 7 + H)
    qn = torch.randn(B, H, 128, generator=g).to(torch.bfloat16)
    qr = torch.randn(B, H, 64, generator=g).to(torch.bfloat16)
    w = (torch.randn(H, 128, 512, generator=g) / math.sqrt(128)).to(torch.bfloat16)
    got = N.absorb_q(qn.cuda(), qr.cuda(), w.cuda())
    torch.cuda.synchronize()
    ref = O.absorb_q(O.bf16_tensor_bits(qn), O.bf16_tensor_bits(qr), O.bf16_tensor_bits(w))
    _close_bf16(got.float().cpu().numpy(), ref)
    assert torch.equal(got[..., 512:].cpu(), qr)


@pytest.mark.parametrize("B,H", [(4, 16), (64, 128), (1, 16), (37, 128), (130, 16)])
def test_v_up_proj_and_fp8_match_oracle(cuda, B, H):
    print(f"v_up_proj B={B} H={H}", flush=True)
    g = torch.Generator().manual_seed(B + 3 * H)
    o = torch.randn(B, H, 512, generator=g).to(torch.bfloat16)
    w = (torch.randn(H, 512, 128, generator=g) / math.sqrt(512)).to(torch.bfloat16)
    y = N.v_up_proj(o.cuda(), w.cuda())
    q8, sc = N.v_up_proj(o.cuda(), w.cuda(), quant_fp8=True)
    torch.cuda.synchronize()
    ref = O.v_up_proj(O.bf16_tensor_bits(o), O.bf16_tensor_bits(w))
    _close_bf16(y.float().cpu().numpy(), ref)
    # the FP8 step is bit-exact on the GEMM's own bf16 output
    codes, s = O.quantize_fp8_per_tensor(O.bf16_tensor_bits(y.cpu()))
    assert np.array_equal(q8.view(torch.uint8).cpu().numpy(), codes.reshape(q8.shape))
    assert float(sc) == float(s)
    assert torch.equal(y, N.v_up_proj(o.cuda(), w.cuda()))  # deterministic: same bits again


def test_absorb_decode_up_chain(cuda):
    """q_nope/q_rope -> absorb -> decode (fp8 cache) -> v_up_proj, against the
    oracle chain fed the same bf16 intermediates."""
    print("absorb -> decode -> v_up chain", flush=True)
    g = torch.Generator().manual_seed(41)
    lens = [300, 65, 1]
    B, H, T = len(lens), 16, sum(lens)
    qn = torch.randn(B, H, 128, generator=g).to(torch.bfloat16)
    qr = torch.randn(B, H, 64, generator=g).to(torch.bfloat16)
    w_uk = (torch.randn(H, 128, 512, generator=g) / math.sqrt(128)).to(torch.bfloat16)
    w_uv = (torch.randn(H, 512, 128, generator=g) / math.sqrt(512)).to(torch.bfloat16)
    kv = torch.randn(T, 1, 576, generator=g).to(torch.bfloat16)
    indptr = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    idx = torch.randperm(T, generator=g).to(torch.int32)
    q = N.absorb_q(qn.cuda(), qr.cuda(), w_uk.cuda())
    case = case_from_tensors(q.cpu(), kv, indptr, idx, "fp8")
    data = device_data(*case[:4], case[5], "fp8", 1 / math.sqrt(192))
    o = custom_kernel(data)
    y = N.v_up_proj(o, w_uv.cuda())
    torch.cuda.synchronize()
    _, o_ref = O.reference_path(case[4], "fp8", case[5], indptr.numpy(), idx.numpy(), 1 / math.sqrt(192))
    assert_close(o.float().cpu().numpy(), o_ref)
    y_ref = O.v_up_proj(O.bf16_tensor_bits(o.cpu()), O.bf16_tensor_bits(w_uv))
    _close_bf16(y.float().cpu().numpy(), y_ref)
