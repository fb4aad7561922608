"""Writes the small golden fixtures under tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py

The reference ships no golden vectors for this path (its only bit-exactness
test compares against a live AITER call on a GPU), so these fixtures are the
oracle's outputs on seeded inputs; the oracle itself is pinned by
tests/test_oracle_*.py.  Fixtures: fp8_quant.npz, mxfp4_pack.npz, decode_fp8.npz.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import mla_oracle as O  # noqa: E402


def main():
    rng = np.random.default_rng(20261201)
    # a2: one Q-shaped tensor (config 1: B=4, H=16)
    q = O.f32_to_bf16(rng.standard_normal((4, 16, 576)).astype(np.float32))
    codes, scale = O.quantize_fp8_per_tensor(q)
    np.savez_compressed(os.path.join(HERE, "fp8_quant.npz"), x=q, codes=codes, scale=np.float32(scale))

    # a4: 64 rows of 576 with special blocks
    x = (rng.standard_normal((64, 576)) * np.exp(rng.uniform(-6, 6, (64, 1)))).astype(np.float32)
    x[0, :32] = 0.0
    x[1, :32] = np.linspace(-7, 7, 32)                       # saturation region
    x[2, :32] = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0] * 4) * 0.25  # ties at e=-2
    x[3, :32] = 1.75                                         # scale round-up
    x[4, :32] = -0.0
    xb = O.f32_to_bf16(x)
    packed, e8 = O.pack_mxfp4(xb)
    np.savez_compressed(os.path.join(HERE, "mxfp4_pack.npz"), x=xb, packed=packed, scales=e8)

    # a7/a8: tiny fp8 decode, H = 16, lengths 5 and 70, permuted slots
    T = 75
    qd = O.f32_to_bf16(rng.standard_normal((2, 16, 576)).astype(np.float32))
    kv = O.f32_to_bf16(rng.standard_normal((T, 576)).astype(np.float32))
    kc, ks = O.quantize_fp8_per_tensor(kv)
    indptr = np.array([0, 5, 75], np.int32)
    idx = rng.permutation(T).astype(np.int32)
    sm = np.float32(1.0 / np.sqrt(192.0))
    bits, f = O.reference_path(qd, "fp8", dict(fp8_codes=kc, fp8_scale=ks), indptr, idx, sm)
    np.savez_compressed(os.path.join(HERE, "decode_fp8.npz"), q=qd, kv=kv, kv_codes=kc,
                        kv_scale=np.float32(ks), kv_indptr=indptr, kv_indices=idx, sm_scale=sm,
                        out_f32=f, out_bf16=bits)


if __name__ == "__main__":
    main()
