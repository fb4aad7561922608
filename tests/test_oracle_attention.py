"""Pins the oracle's attention (the dequantize-then-fp32 softmax(QK^T*sm_scale)V
that ref_kernel approximates, TASK/reference.py:349-369) with a float64
brute force and closed forms."""
import numpy as np
import pytest

from oracle import mla_oracle as O


def rand_case(rng, B, H, lens, T_extra=3):
    T = int(sum(lens)) + T_extra
    q = rng.standard_normal((B, H, 576)).astype(np.float32)
    k = rng.standard_normal((T, 576)).astype(np.float32)
    v = rng.standard_normal((T, 512)).astype(np.float32)
    indptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    idx = rng.permutation(T)[: indptr[-1]]
    return q, k, v, indptr, idx


@pytest.mark.parametrize("lens", [[5, 7], [1, 13, 2], [40]])
def test_matches_float64_brute_force(lens):
    rng = np.random.default_rng(len(lens))
    q, k, v, indptr, idx = rand_case(rng, len(lens), 3, lens)
    sm = 1.0 / np.sqrt(192.0)
    out = O.mla_decode(q, k, v, indptr, idx, sm)
    ref = O.mla_decode_f64(q, k, v, indptr, idx, sm)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)


def test_single_token_returns_its_value_row():
    rng = np.random.default_rng(7)
    q, k, v, indptr, idx = rand_case(rng, 3, 4, [1, 1, 1])
    out = O.mla_decode(q, k, v, indptr, idx, 0.1)
    for b in range(3):
        np.testing.assert_allclose(out[b], np.broadcast_to(v[idx[b]], (4, 512)), rtol=0, atol=1e-6)


def test_identical_keys_average_values():
    rng = np.random.default_rng(8)
    q, k, v, indptr, idx = rand_case(rng, 1, 2, [9])
    k[:] = k[0]
    out = O.mla_decode(q, k, v, indptr, idx, 0.5)
    np.testing.assert_allclose(out[0], np.broadcast_to(v[idx].mean(0), (2, 512)), rtol=1e-5, atol=1e-5)


def test_dominant_token_and_sm_scale_sign():
    # a key aligned with q and a large sm_scale pulls the output onto its value row
    rng = np.random.default_rng(9)
    q, k, v, indptr, idx = rand_case(rng, 1, 1, [6])
    k[idx[4]] = q[0, 0] * 3
    out = O.mla_decode(q, k, v, indptr, idx, 1.0)
    np.testing.assert_allclose(out[0, 0], v[idx[4]], rtol=1e-4, atol=1e-4)


def test_permutation_invariance_and_empty_sequence():
    rng = np.random.default_rng(10)
    q, k, v, indptr, idx = rand_case(rng, 3, 2, [4, 0, 6])
    out = O.mla_decode(q, k, v, indptr, idx, 0.3)
    assert np.all(out[1] == 0)
    perm = rng.permutation(k.shape[0])
    inv = np.argsort(perm)
    out2 = O.mla_decode(q, k[perm], v[perm], indptr, inv[idx], 0.3)
    np.testing.assert_allclose(out, out2, rtol=1e-6, atol=1e-6)


def test_reference_path_end_to_end_small():
    import torch

    rng = np.random.default_rng(11)
    T = 64
    qb = O.f32_to_bf16(rng.standard_normal((2, 16, 576)).astype(np.float32))
    kvb = O.f32_to_bf16(rng.standard_normal((T, 576)).astype(np.float32))
    codes, sc = O.quantize_fp8_per_tensor(kvb)
    packed, e8 = O.pack_mxfp4(kvb)
    caches = dict(fp8_codes=codes, fp8_scale=sc, fp4_packed=packed, fp4_scales=e8)
    indptr = np.array([0, 30, 64])
    idx = rng.permutation(T)
    for mode in ("fp8", "mxfp4", "mxfp4k_fp8v"):
        bits, f = O.reference_path(qb, mode, caches, indptr, idx, 1 / np.sqrt(192))
        assert bits.shape == (2, 16, 512) and np.all(np.isfinite(f))
        # against the unquantized bf16 attention: quantization error stays small
        qf = O.bf16_to_f32(qb)
        kf = O.bf16_to_f32(kvb)
        ref = O.mla_decode(qf, kf, kf[:, :512], indptr, idx, 1 / np.sqrt(192))
        err = np.linalg.norm(f - ref) / np.linalg.norm(ref)
        assert err < (0.06 if mode == "fp8" else 0.25), (mode, err)


# ---- q_seq_len > 1 (causal MTP rows) and the log-sum-exp output -------------
def test_lse_matches_float64_and_closed_form():
    rng = np.random.default_rng(11)
    q, k, v, indptr, idx = rand_case(rng, 3, 2, [6, 1, 0])
    sm = 0.2
    out, lse = O.mla_decode(q, k, v, indptr, idx, sm, return_lse=True)
    ref, ref_lse = O.mla_decode_f64(q, k, v, indptr, idx, sm, return_lse=True)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(lse[:2], ref_lse[:2], rtol=1e-5, atol=1e-4)
    # one key: lse = sm * q.k exactly; no key: -inf
    np.testing.assert_allclose(lse[1], sm * (q[1] @ k[idx[6]]), rtol=1e-5, atol=1e-4)
    assert np.all(np.isneginf(lse[2]))


@pytest.mark.parametrize("qlen", [2, 4])
def test_mtp_rows_are_causal_prefix_decodes(qlen):
    """Query i of a sequence with L keys equals a single-query decode over the
    first L - (qlen - 1 - i) keys (a separate call on a truncated indptr)."""
    rng = np.random.default_rng(20 + qlen)
    lens = [9, 3, 1, 17]
    S = len(lens)
    q, k, v, indptr, idx = rand_case(rng, S * qlen, 2, [0] * S * qlen, T_extra=sum(lens) + 3)
    indptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    idx = rng.permutation(k.shape[0])[: indptr[-1]]
    out, lse = O.mla_decode(q, k, v, indptr, idx, 0.15, q_seq_len=qlen, return_lse=True)
    ref, ref_lse = O.mla_decode_f64(q, k, v, indptr, idx, 0.15, q_seq_len=qlen, return_lse=True)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)
    for b in range(S):
        for i in range(qlen):
            n = max(lens[b] - (qlen - 1 - i), 0)
            one = O.mla_decode(q[b * qlen + i: b * qlen + i + 1], k, v, np.array([0, n]),
                               idx[indptr[b]: indptr[b] + n], 0.15)
            np.testing.assert_allclose(out[b * qlen + i], one[0], rtol=1e-6, atol=1e-6)
            if n == 0:
                assert np.all(out[b * qlen + i] == 0) and np.all(np.isneginf(lse[b * qlen + i]))
