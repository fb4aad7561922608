"""Bit-exactness of the device quantizers against the pinned CPU oracle."""
import os

import numpy as np
import pytest
import torch

from amd_optimization_challenge_amd import ops
from oracle import mla_oracle as O

pytestmark = pytest.mark.gpu
G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def to_dev_bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def gpu_fp8(bits):
    out, sc = ops.quant_fp8_per_tensor(to_dev_bf16(bits))
    torch.cuda.synchronize()
    return out.view(torch.uint8).cpu().numpy(), np.float32(sc.item())


@pytest.mark.parametrize("n,mult", [(1, 1.0), (7, 3.0), (8, 1.0), (9, 0.01), (1000, 100.0),
                                    (4 * 16 * 576, 1.0), (65536 + 3, 7.0), (3_000_005, 1.0)])
def test_fp8_quant_bit_exact(cuda, n, mult):
    print(f"fp8 quant n={n}", flush=True)
    rng = np.random.default_rng(n)
    bits = O.f32_to_bf16((rng.standard_normal(n) * mult).astype(np.float32))
    codes, scale = gpu_fp8(bits)
    ref_codes, ref_scale = O.quantize_fp8_per_tensor(bits)
    assert scale == np.float32(ref_scale)
    assert np.array_equal(codes, ref_codes)


def test_fp8_quant_exhaustive_and_zero(cuda):
    allb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = allb[(allb & 0x7F80) != 0x7F80]
    for bits in (finite, finite[(finite & 0x7FFF) < 0x3F80], np.zeros(4096, np.uint16)):
        codes, scale = gpu_fp8(bits)
        ref_codes, ref_scale = O.quantize_fp8_per_tensor(bits)
        assert scale == np.float32(ref_scale) and np.array_equal(codes, ref_codes)


def test_fp8_quant_golden(cuda):
    d = np.load(os.path.join(G, "fp8_quant.npz"))
    codes, scale = gpu_fp8(d["x"])
    assert scale == d["scale"] and np.array_equal(codes.reshape(d["codes"].shape), d["codes"])


def gpu_pack(bits, scale_cols=None):
    x = to_dev_bf16(bits)
    packed, scales = ops.pack_mxfp4(x, scale_cols=scale_cols)
    torch.cuda.synchronize()
    return packed.cpu().numpy(), scales.cpu().numpy()


@pytest.mark.parametrize("rows,cols,spread", [(1, 32, 0), (64, 576, 6), (1000, 576, 20), (3, 96, 2)])
def test_mxfp4_pack_bit_exact(cuda, rows, cols, spread):
    print(f"mxfp4 pack {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols)
    x = (rng.standard_normal((rows, cols)) * np.exp(rng.uniform(-spread, spread, (rows, 1)))).astype(np.float32)
    bits = O.f32_to_bf16(x)
    packed, scales = gpu_pack(bits)
    rp, rs = O.pack_mxfp4(bits)
    assert np.array_equal(scales, rs)
    assert np.array_equal(packed, rp)


def test_mxfp4_pack_every_bf16_value(cuda):
    allb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = allb[(allb & 0x7F80) != 0x7F80]
    rng = np.random.default_rng(1)
    for order in (np.sort(finite), rng.permutation(finite)):  # blocks of neighbours and random blocks
        n = (len(order) // 576) * 576
        bits = order[:n].reshape(-1, 576)
        packed, scales = gpu_pack(bits)
        rp, rs = O.pack_mxfp4(bits)
        assert np.array_equal(scales, rs) and np.array_equal(packed, rp)


def test_mxfp4_pack_golden_and_padded_scales(cuda):
    d = np.load(os.path.join(G, "mxfp4_pack.npz"))
    packed, scales = gpu_pack(d["x"], scale_cols=24)
    assert np.array_equal(packed, d["packed"])
    assert np.array_equal(scales[:, :18], d["scales"]) and np.all(scales[:, 18:] == 127)
