"""The oracle's neighbouring products (W_UK absorption, v_up_proj) pinned on
the CPU: float64 brute force on tiny shapes, identity-block weights, and the
rope pass-through."""
import numpy as np

from oracle import mla_oracle as O


def _bits(x):
    return O.f32_to_bf16(np.asarray(x, np.float32))


def test_absorb_q_brute_force_and_rope_pass_through():
    rng = np.random.default_rng(3)
    B, H = 3, 2
    qn, qr, w = (_bits(rng.standard_normal(s)) for s in [(B, H, 128), (B, H, 64), (H, 128, 512)])
    got = O.absorb_q(qn, qr, w)
    assert got.shape == (B, H, 576) and got.dtype == np.float32
    qn64, w64 = O.bf16_to_f32(qn).astype(np.float64), O.bf16_to_f32(w).astype(np.float64)
    for b in range(B):
        for h in range(H):
            exp = np.array([sum(qn64[b, h, k] * w64[h, k, n] for k in range(128)) for n in range(0, 512, 37)])
            assert np.allclose(got[b, h, 0:512:37], exp, rtol=1e-5, atol=1e-4)
    assert np.array_equal(got[..., 512:], O.bf16_to_f32(qr))


def test_absorb_q_identity_block_reproduces_q_nope():
    rng = np.random.default_rng(4)
    qn, qr = _bits(rng.standard_normal((2, 3, 128))), _bits(rng.standard_normal((2, 3, 64)))
    w = np.zeros((3, 128, 512), np.float32)
    for h in range(3):
        w[h, :, 128 * h:128 * h + 128] = np.eye(128)  # head h copies q_nope into latent block h
    got = O.absorb_q(qn, qr, _bits(w))
    for h in range(3):
        assert np.array_equal(got[:, h, 128 * h:128 * h + 128], O.bf16_to_f32(qn)[:, h])
        rest = np.delete(got[:, h, :512], np.s_[128 * h:128 * h + 128], axis=-1)
        assert np.all(rest == 0)


def test_v_up_proj_brute_force_and_identity():
    rng = np.random.default_rng(5)
    o, w = _bits(rng.standard_normal((2, 2, 512))), _bits(rng.standard_normal((2, 512, 128)))
    got = O.v_up_proj(o, w)
    o64, w64 = O.bf16_to_f32(o).astype(np.float64), O.bf16_to_f32(w).astype(np.float64)
    exp = np.einsum("bhk,hkn->bhn", o64, w64)
    assert np.allclose(got, exp, rtol=1e-5, atol=1e-4)
    eye = np.zeros((2, 512, 128), np.float32)
    eye[:, 384:, :] = np.eye(128)
    assert np.array_equal(O.v_up_proj(o, _bits(eye)), O.bf16_to_f32(o)[..., 384:])
