"""The committed fixtures still match the (pinned) oracle."""
import os

import numpy as np

from oracle import mla_oracle as O

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_fp8_fixture():
    d = np.load(os.path.join(G, "fp8_quant.npz"))
    codes, scale = O.quantize_fp8_per_tensor(d["x"])
    assert np.array_equal(codes, d["codes"]) and np.float32(scale) == d["scale"]


def test_mxfp4_fixture():
    d = np.load(os.path.join(G, "mxfp4_pack.npz"))
    packed, e8 = O.pack_mxfp4(d["x"])
    assert np.array_equal(packed, d["packed"]) and np.array_equal(e8, d["scales"])


def test_decode_fixture():
    d = np.load(os.path.join(G, "decode_fp8.npz"))
    bits, f = O.reference_path(d["q"], "fp8", dict(fp8_codes=d["kv_codes"], fp8_scale=d["kv_scale"]),
                               d["kv_indptr"], d["kv_indices"], float(d["sm_scale"]))
    np.testing.assert_allclose(f, d["out_f32"], rtol=1e-5, atol=1e-6)
