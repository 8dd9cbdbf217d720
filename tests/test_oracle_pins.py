"""Independent pins of the oracle functions the attention closed form rests
on: the centred calibration covariance, the scalar dequantiser and scores,
and the block-VQ scores.  Each check is one a plausible slip fails -- an
uncentred or N-1 covariance, E where E_inv belongs (or the reverse), a
dropped norm or scale, a transposed operand, blocks taken in the wrong
order -- and none re-evaluates the oracle's own torch expression: the
expected values come from numpy float64, explicit bit/gather loops, closed
forms of diagonal and identity metrics, and the algebraic identity that ties
dequantisation back to the encoder's metric.  CPU only."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import smaq_ref as R
from tests.conftest import sample_keys, spectral_sigma


def _bit_loop_codes(packed: torch.Tensor, bits: int, d: int) -> np.ndarray:
    """Codes from packed bytes by an explicit per-field loop (low field first)."""
    vpb = max(1, 8 // bits)
    mask = (1 << bits) - 1
    pk = packed.reshape(-1, packed.shape[-1]).tolist()
    out = np.zeros((len(pk), d), dtype=np.int64)
    for r, row in enumerate(pk):
        for j in range(d):
            out[r, j] = (row[j // vpb] >> ((j % vpb) * bits)) & mask
    return out


# ----------------------------------------------------- fit_sigma_centered ---

def test_fit_sigma_centered_is_the_biased_covariance():
    """smaq/quantizer.py:121-129: centred, divided by N (numpy's biased
    covariance).  A mean offset makes the uncentred form clearly different."""
    g = torch.Generator().manual_seed(31)
    q = torch.randn(200, 16, generator=g) * torch.linspace(0.2, 3.0, 16) + torch.linspace(-4.0, 5.0, 16)
    got = R.fit_sigma_centered(q).double().numpy()
    want = np.cov(q.double().numpy(), rowvar=False, bias=True)
    scale = np.abs(want).max()
    np.testing.assert_allclose(got, want, atol=2e-6 * scale, rtol=0)
    # the checks above would catch either slip by a wide margin
    q64 = q.double().numpy()
    uncentred = q64.T @ q64 / q64.shape[0]
    assert np.abs(uncentred - want).max() > 100 * 2e-6 * scale
    unbiased = np.cov(q64, rowvar=False, bias=False)
    assert np.abs(unbiased - want).max() > 100 * 2e-6 * scale


def test_fit_sigma_centered_small_cases():
    one = torch.tensor([[1.5, -2.0, 7.0]])
    assert torch.equal(R.fit_sigma_centered(one), torch.zeros(3, 3))        # single row: zero spread
    two = torch.tensor([[1.0, 0.0], [3.0, 4.0]])                             # mean (2, 2), deviations +-(1, 2)
    np.testing.assert_array_equal(R.fit_sigma_centered(two).numpy(), np.array([[1.0, 2.0], [2.0, 4.0]]))
    # a constant shift of every query leaves the covariance unchanged
    g = torch.Generator().manual_seed(32)
    q = torch.randn(64, 8, generator=g)
    a = R.fit_sigma_centered(q).double()
    b = R.fit_sigma_centered(q + 10.0).double()
    assert float((a - b).abs().max()) < 1e-4


# ---------------------------------------------------------- smaq_dequantize ---

def _encoded(bits, n=300, seed=12, sigma_seed=4):
    sigma, _, _ = spectral_sigma(128, sigma_seed)
    E, Ei = R.build_metric(sigma)
    c, _, db = R.scalar_tables(bits)
    k = sample_keys(n, seed=seed)
    return E, Ei, c, R.scalar_encode(k, E, db, bits)


@pytest.mark.parametrize("bits", [3, 4])
def test_dequantize_inverts_the_encoder_metric(bits):
    """E (k_hat / n) = c[code]: dequantisation undoes the encoder's rotation
    (smaq/quantizer.py:138-152).  Using E where E_inv belongs fails this by
    orders of magnitude."""
    E, Ei, c, q = _encoded(bits)
    khat = R.smaq_dequantize(q, c, Ei, 128).double().numpy()
    n = q.norms.double().numpy()
    codes = _bit_loop_codes(q.indices, bits, 128)
    want = c.double().numpy()[codes]
    back = (khat / n[:, None]) @ E.double().numpy().T
    err = np.abs(back - want).max()
    assert err < 2e-3
    wrong = (R.smaq_dequantize(q, c, E, 128).double().numpy() / n[:, None]) @ E.double().numpy().T
    assert np.abs(wrong - want).max() > 100 * err


def test_dequantize_identity_metric_closed_form():
    """E = E_inv = I: k_hat = fp32(c[code] * n), bit for bit."""
    c, _, db = R.scalar_tables(3)
    k = sample_keys(64, seed=14)
    eye = torch.eye(128)
    q = R.scalar_encode(k, eye, db, 3)
    khat = R.smaq_dequantize(q, c, eye, 128).numpy()
    codes = _bit_loop_codes(q.indices, 3, 128)
    want = (c.numpy()[codes] * q.norms.numpy()[:, None]).astype(np.float32)
    assert np.array_equal(khat, want)


def test_dequantize_diagonal_metric_closed_form():
    """E = diag(e): k_hat_i = c[code_i] / e_i * n (two roundings at most)."""
    e = torch.linspace(0.25, 4.0, 128)
    E, Ei = torch.diag(e), torch.diag(1.0 / e)
    c, _, db = R.scalar_tables(4)
    k = sample_keys(80, seed=15)
    q = R.scalar_encode(k, E, db, 4)
    khat = R.smaq_dequantize(q, c, Ei, 128).double().numpy()
    codes = _bit_loop_codes(q.indices, 4, 128)
    want = c.double().numpy()[codes] / e.double().numpy()[None, :] * q.norms.double().numpy()[:, None]
    np.testing.assert_allclose(khat, want, rtol=3e-7, atol=0)


# -------------------------------------------------------------- smaq_scores ---

def test_scores_diagonal_metric_closed_form():
    """s[t, n] = scale * n_n * sum_i q_ti / e_i * c[code_ni] (float64 loops);
    E in place of E_inv, a missing norm or a missing scale all fail."""
    e = torch.linspace(0.3, 3.0, 128)
    E, Ei = torch.diag(e), torch.diag(1.0 / e)
    c, _, db = R.scalar_tables(3)
    k = sample_keys(50, seed=16)
    q = R.scalar_encode(k, E, db, 3)
    query = sample_keys(3, seed=17)
    got = R.smaq_scores(query, q, c, Ei, 128, scale=0.125).double().numpy()
    codes = _bit_loop_codes(q.indices, 3, 128)
    c64, e64, q64 = c.double().numpy(), e.double().numpy(), query.double().numpy()
    n64 = q.norms.double().numpy()
    want = np.zeros((3, 50))
    for t in range(3):
        for j in range(50):
            want[t, j] = 0.125 * n64[j] * sum(q64[t, i] / e64[i] * c64[codes[j, i]] for i in range(128))
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6 * np.abs(want).max())
    swapped = R.smaq_scores(query, q, c, E, 128, scale=0.125).double().numpy()
    assert np.abs(swapped - want).max() > 0.1 * np.abs(want).max()


def test_scores_equal_query_dot_reconstructed_key():
    """With a calibrated (symmetric) metric the scores equal q . k_hat * scale
    where k_hat = n * E^-1 c[code] is rebuilt from the encoder metric E by a
    float64 solve, independent of the oracle's E_inv and dequantiser."""
    E, Ei, c, q = _encoded(3, n=120, seed=18, sigma_seed=6)
    query = sample_keys(5, seed=19)
    got = R.smaq_scores(query, q, c, Ei, 128, scale=0.0884).double().numpy()
    codes = _bit_loop_codes(q.indices, 3, 128)
    y = c.double().numpy()[codes]                                   # [N, D]
    khat = np.linalg.solve(E.double().numpy(), y.T).T * q.norms.double().numpy()[:, None]
    want = query.double().numpy() @ khat.T * 0.0884
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-3 * np.abs(want).max())


def test_scores_output_dtype_is_the_query_dtype():
    E, Ei, c, q = _encoded(3, n=40)
    query = sample_keys(2, seed=20)
    s32 = R.smaq_scores(query, q, c, Ei, 128, scale=0.5)
    s16 = R.smaq_scores(query.bfloat16(), q, c, Ei, 128, scale=0.5)
    assert s32.dtype == torch.float32 and s16.dtype == torch.bfloat16
    # bf16 query: fp32 arithmetic on the bf16-rounded query, one final rounding
    want = R.smaq_scores(query.bfloat16().float(), q, c, Ei, 128, scale=0.5).bfloat16()
    assert torch.equal(s16, want)


# ----------------------------------------------------------- blockvq_scores ---

@pytest.mark.parametrize("nb,nc,bd", [(16, 256, 8), (64, 256, 2), (4, 16, 32)])
def test_blockvq_scores_gather_loop(nb, nc, bd):
    """s[t, n] = scale * sum_b q[t, b*bd:(b+1)*bd] . decoded[b][idx[n, b]]
    (smaq/block_vq.py:246-297), from an explicit per-block gather in float64.
    Blocks in the wrong order, a transposed product or an index column
    mix-up all fail."""
    g = torch.Generator().manual_seed(nb * 7 + bd)
    dec = torch.randn(nb, nc, bd, generator=g)
    idx = torch.randint(0, nc, (40, nb), generator=g)
    query = torch.randn(6, nb * bd, generator=g)
    got = R.blockvq_scores(query, R.BlockQ(idx, nb, bd), dec, scale=0.3).double().numpy()
    d64, q64, ix = dec.double().numpy(), query.double().numpy(), idx.numpy()
    want = np.zeros((6, 40))
    for j in range(40):
        key = np.concatenate([d64[b, ix[j, b]] for b in range(nb)])
        want[:, j] = 0.3 * (q64 @ key)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())
    flipped = R.blockvq_scores(query, R.BlockQ(idx, nb, bd), dec.flip(0), scale=0.3).double().numpy()
    assert np.abs(flipped - want).max() > 0.05 * np.abs(want).max()


def test_blockvq_scores_keys_on_codewords():
    """Keys that sit exactly on decoded codewords score as the plain dot
    product q . k (no scale), and the output dtype follows the query."""
    g = torch.Generator().manual_seed(33)
    dec = torch.randn(4, 8, 4, generator=g)
    idx = torch.randint(0, 8, (10, 4), generator=g)
    keys = torch.cat([dec[b][idx[:, b]] for b in range(4)], dim=1)
    query = torch.randn(3, 16, generator=g)
    got = R.blockvq_scores(query, R.BlockQ(idx, 4, 4), dec)
    np.testing.assert_allclose(got.double().numpy(), query.double().numpy() @ keys.double().numpy().T,
                               rtol=1e-6, atol=1e-6)
    assert R.blockvq_scores(query.half(), R.BlockQ(idx, 4, 4), dec).dtype == torch.float16


# ------------------------------------------ rotation_dequantize / scores ---

def _rotation_encoded(bits, n, seed):
    """A random orthogonal (non-symmetric) rotation, non-uniform coordinate
    scales e^[-1.2, 1.2] in shuffled order, midpoint tables, encoded keys
    (smaq/weighted_scalar.py:347-355)."""
    g = torch.Generator().manual_seed(seed)
    rot, _ = torch.linalg.qr(torch.randn(128, 128, generator=g))
    s = torch.exp(torch.linspace(-1.2, 1.2, 128))[torch.randperm(128, generator=g)]
    c, _, db = R.midpoint_tables(bits)
    k = sample_keys(n, seed=seed + 1)
    return rot, s, c, R.scalar_encode(k, rot, db, bits, coord_scales=s)


@pytest.mark.parametrize("bits", [3, 4])
def test_rotation_dequantize_inverts_the_encoder(bits):
    """(k_hat / n) R^T * s = c[code]: dequantisation undoes the encoder's
    rotate-then-scale (smaq/weighted_scalar.py:347-363).  Passing the scales
    where the inverse scales belong, or R^T for R, fails by a wide margin."""
    rot, s, c, q = _rotation_encoded(bits, 200, 40)
    n = q.norms.double().numpy()
    r64, s64 = rot.double().numpy(), s.double().numpy()
    want = c.double().numpy()[_bit_loop_codes(q.indices, bits, 128)]

    def back(khat):
        return (khat.double().numpy() / n[:, None]) @ r64.T * s64[None, :]

    err = np.abs(back(R.rotation_dequantize(q, c, 1.0 / s, rot, 128)) - want).max()
    assert err < 1e-4
    assert np.abs(back(R.rotation_dequantize(q, c, s, rot, 128)) - want).max() > 1000 * err
    assert np.abs(back(R.rotation_dequantize(q, c, 1.0 / s, rot.T.contiguous(), 128)) - want).max() > 1000 * err


def test_rotation_scores_closed_form():
    """dim 8, R a signed permutation (row i holds sign_i at column perm_i, so
    (q R^T)_i = sign_i q_perm_i), scales powers of two:
    s[t, j] = scale * n_j * sum_i sign_i q[t, perm_i] / s_i * c[code_ji],
    codes packed by an explicit loop (smaq/weighted_scalar.py:342-345,
    365-379).  Scales for inverse scales, R^T for R, a dropped norm or
    scale all fail."""
    perm, sign = [3, 0, 6, 1, 7, 2, 5, 4], [1, -1, 1, 1, -1, 1, -1, 1]
    rot = torch.zeros(8, 8)
    for i in range(8):
        rot[i, perm[i]] = sign[i]
    s = torch.tensor([0.25, 0.5, 1.0, 2.0, 4.0, 0.5, 2.0, 1.0])
    c, _, _ = R.midpoint_tables(3)
    g = torch.Generator().manual_seed(44)
    codes = torch.randint(0, 8, (12, 8), generator=g)
    packed = torch.zeros(12, 4, dtype=torch.uint8)
    for j in range(12):
        for p in range(4):
            packed[j, p] = int(codes[j, 2 * p]) | (int(codes[j, 2 * p + 1]) << 3)
    norms = torch.rand(12, generator=g) + 0.5
    query = torch.randn(2, 8, generator=g)
    q = R.ScalarQ(packed, norms, 3)
    got = R.rotation_scores(query, q, c, 1.0 / s, rot, 8, scale=0.7).double().numpy()
    c64, q64, n64, s64 = c.double().numpy(), query.double().numpy(), norms.double().numpy(), s.double().numpy()
    want = np.zeros((2, 12))
    for t in range(2):
        for j in range(12):
            want[t, j] = 0.7 * n64[j] * sum(sign[i] * q64[t, perm[i]] / s64[i] * c64[int(codes[j, i])]
                                            for i in range(8))
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6 * np.abs(want).max())
    big = 0.1 * np.abs(want).max()
    assert np.abs(R.rotation_scores(query, q, c, s, rot, 8, scale=0.7).double().numpy() - want).max() > big
    assert np.abs(R.rotation_scores(query, q, c, 1.0 / s, rot.T.contiguous(), 8, scale=0.7).double().numpy()
                  - want).max() > big
    assert np.abs(R.rotation_scores(query, q, c, 1.0 / s, rot, 8).double().numpy() - want).max() > big


def test_rotation_scores_equal_query_dot_reconstructed_key():
    """The scores equal q . k_hat * scale with k_hat = n u, u solving the
    encoder's map u R^T * s = c[code] by a float64 linear solve -- neither the
    oracle's dequantiser nor R's orthogonality is assumed."""
    rot, s, c, q = _rotation_encoded(4, 100, 41)
    query = sample_keys(4, seed=43)
    got = R.rotation_scores(query, q, c, 1.0 / s, rot, 128, scale=0.0884).double().numpy()
    y = c.double().numpy()[_bit_loop_codes(q.indices, 4, 128)]
    u = np.linalg.solve(rot.double().numpy(), (y / s.double().numpy()[None, :]).T).T
    want = query.double().numpy() @ (u * q.norms.double().numpy()[:, None]).T * 0.0884
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-5 * np.abs(want).max())
    assert got.shape == (4, 100)
