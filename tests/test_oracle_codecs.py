"""Pins the CPU oracle's codec functions with checks that do not restate it:
brute-force bit loops, scipy closed forms, float64 recomputation, invariants
of the metric, hand-computed known answers.  CPU only."""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest
import torch
from scipy.stats import norm as scipy_norm

from oracle import smaq_ref as R
from tests.bf16ref import bf16_round
from tests.conftest import sample_keys, spectral_sigma


# ---------------------------------------------------------------- packing ---

@pytest.mark.parametrize("bits", range(1, 9))
@pytest.mark.parametrize("d", [1, 7, 8, 64, 128, 130])
def test_pack_codes_bit_loop(bits, d):
    g = torch.Generator().manual_seed(bits * 1000 + d)
    codes = torch.randint(0, 2 ** bits, (5, d), generator=g)
    packed = R.pack_codes(codes, bits)
    vpb = max(1, 8 // bits)
    assert packed.dtype == torch.uint8
    assert packed.shape == (5, (d + vpb - 1) // vpb)
    pk = packed.tolist()
    cd = codes.tolist()
    for r in range(5):
        for byte_i, byte in enumerate(pk[r]):
            for slot in range(vpb):
                j = byte_i * vpb + slot
                field = (byte >> (slot * bits)) & ((1 << bits) - 1)
                assert field == (cd[r][j] if j < d else 0)
            if vpb * bits < 8:
                assert byte >> (vpb * bits) == 0          # unused high bits stay zero
    assert torch.equal(R.unpack_codes(packed, bits, d), codes)


# ----------------------------------------------------------------- tables ---

@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5])
def test_scalar_tables_closed_form(bits):
    c, b, db = R.scalar_tables(bits)
    n = 2 ** bits
    want_c = scipy_norm.ppf(np.arange(1, n + 1) / (n + 1))
    want_b = scipy_norm.ppf(np.clip(np.arange(1, n) / n, 1e-6, 1 - 1e-6))
    np.testing.assert_allclose(c.numpy(), want_c, atol=2e-6, rtol=2e-6)
    np.testing.assert_allclose(db.numpy(), want_b, atol=2e-6, rtol=2e-6)
    assert b[0] == -math.inf and b[-1] == math.inf and torch.equal(b[1:-1], db)
    # centroid j lies inside cell j
    assert torch.all(db > c[:-1]) and torch.all(db < c[1:])


def test_scalar_tables_known_values():
    # 4-bit: centroids span +-1.5647, outer decision boundaries +-1.5341
    c, _, db = R.scalar_tables(4)
    assert abs(c[-1].item() - 1.5647) < 1e-4 and abs(c[0].item() + 1.5647) < 1e-4
    assert abs(db[-1].item() - 1.5341) < 1e-4 and abs(db[0].item() + 1.5341) < 1e-4
    # odd number of cuts: the middle one is ppf(0.5) = 0 exactly
    assert db[7].item() == 0.0


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_midpoint_tables(bits):
    c, b, db = R.midpoint_tables(bits)
    left = (db - c[:-1]).numpy()
    right = (c[1:] - db).numpy()
    np.testing.assert_allclose(left, right, rtol=1e-6, atol=1e-7)
    assert b[0] == -math.inf and b[-1] == math.inf


# ----------------------------------------------------------------- metric ---

def test_metric_invariants_full():
    sigma, _, _ = spectral_sigma(128, seed=3)
    E, Ei = R.build_metric(sigma)
    E64, Ei64 = E.double(), Ei.double()
    np.testing.assert_allclose((E64 @ Ei64).numpy(), np.eye(128), atol=2e-4)
    np.testing.assert_allclose(E64.numpy(), E64.T.numpy(), atol=1e-5)
    # volume normalised: det(E) = prod(sqrt(s)) = 1
    sign, logdet = np.linalg.slogdet(E64.numpy())
    assert sign > 0 and abs(logdet) < 1e-3
    # E shares Sigma's eigenvectors, so they commute
    np.testing.assert_allclose((E64 @ sigma.double()).numpy(), (sigma.double() @ E64).numpy(), atol=1e-5)


def test_metric_diagonal_closed_form():
    lam = np.array([4.0, 1.0, 0.25, 0.0, 1e-9, 9.0], dtype=np.float64)
    E, Ei = R.build_metric(torch.tensor(np.diag(lam), dtype=torch.float32))
    l = np.log(np.maximum(np.log1p(5.0 * np.maximum(lam, 0)), 1e-8))
    s = np.exp(l - l.mean())
    np.testing.assert_allclose(np.abs(E.numpy()), np.diag(np.sqrt(s)), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(np.abs(Ei.numpy()), np.diag(1 / np.sqrt(s)), rtol=1e-5, atol=1e-4)


def test_rotated_diag_scales_identity_rotation():
    lam = np.array([3.0, 1.0, 0.5, 0.1], dtype=np.float64)
    s = R.diag_metric_scales(torch.tensor(np.diag(lam), dtype=torch.float32), torch.eye(4)).numpy()
    l = np.log(np.log1p(5.0 * lam))
    shaped = np.exp(l - l.mean())
    want = np.sqrt(shaped)
    want = np.exp(np.log(want) - np.log(want).mean())
    np.testing.assert_allclose(s, want, rtol=1e-5)
    assert abs(np.log(s).mean()) < 1e-6


# ----------------------------------------------------------- scalar codec ---

def _np_searchsorted_ties(y64, bounds):
    codes = np.searchsorted(bounds, y64, side="left")
    near = np.zeros_like(y64, dtype=bool)
    for b in bounds:
        near |= np.abs(y64 - b) <= 1e-6 * np.maximum(np.maximum(abs(b), np.abs(y64)), 1e-6)
    return codes, near


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_scalar_encode_vs_float64(bits):
    sigma, _, _ = spectral_sigma(128, seed=0)
    queries = sample_keys(64, seed=7)
    E, _ = R.build_metric(R.fit_sigma_centered(queries))
    _, _, db = R.scalar_tables(bits)
    k = sample_keys(3000, seed=11)
    q = R.scalar_encode(k, E, db, bits)
    k64 = k.double().numpy()
    n64 = np.sqrt((k64 ** 2).sum(-1))
    y64 = (k64 / n64[:, None]) @ E.double().numpy().T
    want, near = _np_searchsorted_ties(y64, db.double().numpy())
    got = R.unpack_codes(q.indices, bits, 128).numpy()
    assert ((got != want) & ~near).sum() == 0
    # norms: fp32 summation of 128 squares stays within 2 ulp of float64
    ulp = np.spacing(np.float32(n64)).astype(np.float64)
    assert np.all(np.abs(q.norms.double().numpy() - n64) <= 2 * ulp)


def test_scalar_encode_special_cases():
    _, _, db = R.scalar_tables(4)
    eye = torch.eye(128)
    zero = R.scalar_encode(torch.zeros(2, 128), eye, db, 4)
    assert torch.all(R.unpack_codes(zero.indices, 4, 128) == 7)       # 7 cuts below 0
    assert torch.all(zero.norms == 0)
    basis = torch.eye(128)[:5] * 3.0
    q = R.scalar_encode(basis, eye, db, 4)
    codes = R.unpack_codes(q.indices, 4, 128)
    n_below_one = int((db < 1.0).sum())
    for i in range(5):
        assert codes[i, i] == n_below_one
        assert torch.all(codes[i, torch.arange(128) != i] == 7)
    signs = torch.sign(torch.randn(4, 128, generator=torch.Generator().manual_seed(3)))
    sat = R.scalar_encode(signs, 1000 * eye, db, 4)      # |y| = 1000 / sqrt(128) everywhere
    c = R.unpack_codes(sat.indices, 4, 128)
    assert torch.all((c == 0) | (c == 15))


def test_scalar_encode_bf16_per_op_rounding():
    """bf16 keys: norm, +1e-10 and the division each round to bf16 (numpy model)."""
    _, _, db = R.scalar_tables(3)
    E, _ = R.build_metric(spectral_sigma(128, 2)[0])
    k = sample_keys(512, seed=5).bfloat16()
    q = R.scalar_encode(k, E, db, 3)
    kf = k.float().numpy()
    n = bf16_round(np.sqrt((kf.astype(np.float64) ** 2).sum(-1)).astype(np.float32))
    assert np.array_equal(q.norms.float().numpy(), n)
    u = bf16_round(kf / bf16_round(n + np.float32(1e-10))[:, None])
    y64 = u.astype(np.float64) @ E.double().numpy().T
    want, near = _np_searchsorted_ties(y64, db.double().numpy())
    got = R.unpack_codes(q.indices, 3, 128).numpy()
    assert ((got != want) & ~near).sum() == 0


def test_rotation_encode_identity_reduces_to_plain_scalar():
    c, _, db = R.midpoint_tables(3)
    k = sample_keys(200, seed=9)
    a = R.scalar_encode(k, torch.eye(128), db, 3, coord_scales=torch.ones(128))
    k64 = k.double().numpy()
    y64 = k64 / np.sqrt((k64 ** 2).sum(-1))[:, None]
    want, near = _np_searchsorted_ties(y64, db.double().numpy())
    got = R.unpack_codes(a.indices, 3, 128).numpy()
    assert ((got != want) & ~near).sum() == 0


def test_dequantize_score_consistency():
    """scores from codes == q . dequantize(k) (a8 vs a9 invariant)."""
    sigma, _, _ = spectral_sigma(128, 4)
    E, Ei = R.build_metric(sigma)
    c, _, db = R.scalar_tables(3)
    k = sample_keys(300, seed=12)
    q = R.scalar_encode(k, E, db, 3)
    khat = R.smaq_dequantize(q, c, Ei, 128)
    query = sample_keys(4, seed=13)
    s = R.smaq_scores(query, q, c, Ei, 128, scale=0.1)
    np.testing.assert_allclose(s.numpy(), (query.double() @ khat.double().T * 0.1).numpy(), rtol=2e-4, atol=2e-4)


# --------------------------------------------------------------- block VQ ---

def test_blockvq_encode_brute_force():
    g = torch.Generator().manual_seed(21)
    nb, nc, bd = 4, 64, 8
    E_blocks = torch.stack([torch.linalg.qr(torch.randn(bd, bd, generator=g))[0] * 1.3 for _ in range(nb)])
    cents = torch.randn(nb, nc, bd, generator=g)
    k = torch.randn(700, nb * bd, generator=g)
    got = R.blockvq_encode(k, E_blocks, cents).indices.numpy()
    k64, E64, C64 = k.double().numpy(), E_blocks.double().numpy(), cents.double().numpy()
    ties = 0
    for b in range(nb):
        x = k64[:, b * bd:(b + 1) * bd] @ E64[b].T
        d = np.sqrt(((x[:, None, :] - C64[b][None]) ** 2).sum(-1))
        srt = np.sort(d, axis=1)
        near = srt[:, 1] <= srt[:, 0] * (1 + 1e-6)
        ties += near.sum()
        assert ((d.argmin(1) != got[:, b]) & ~near).sum() == 0
    assert ties < 5


def test_blockvq_identity_metric_is_plain_vq():
    g = torch.Generator().manual_seed(22)
    cents = torch.randn(2, 16, 2, generator=g)
    pick = torch.randint(0, 16, (50, 2), generator=g)
    k = torch.cat([cents[0][pick[:, 0]], cents[1][pick[:, 1]]], dim=1)   # keys sit on codewords
    got = R.blockvq_encode(k, torch.eye(2).expand(2, 2, 2), cents).indices
    assert torch.equal(got, pick)


def test_blockvq_dequantize_lut():
    g = torch.Generator().manual_seed(23)
    dec = torch.randn(3, 10, 4, generator=g)
    idx = torch.randint(0, 10, (6, 3), generator=g)
    out = R.blockvq_dequantize(R.BlockQ(idx, 3, 4), dec)
    for r in range(6):
        for b in range(3):
            assert torch.equal(out[r, b * 4:(b + 1) * 4], dec[b, idx[r, b]])


# ----------------------------------------------------------------- values ---

def _fraction_codes(vals, bits):
    lo, hi = min(vals), max(vals)
    levels = 2 ** bits - 1
    scale = Fraction(hi - lo) / levels
    out = []
    for v in vals:
        x = Fraction(v - lo) / scale
        fl = math.floor(x)
        frac = x - fl
        r = fl + (1 if frac > Fraction(1, 2) or (frac == Fraction(1, 2) and fl % 2 == 1) else 0)
        out.append(max(0, min(levels, r)))
    return out


def test_quantize_values_known_answer():
    vals = list(range(32)) + [(-1) ** i * i / 4 for i in range(32)]
    v = torch.tensor(vals, dtype=torch.float32).reshape(1, 64)
    q = R.quantize_values(v, bits=2, group_size=32)
    codes = _fraction_codes(vals[:32], 2) + _fraction_codes([Fraction(x).limit_denominator(8) for x in vals[32:]], 2)
    want = [codes[4 * i] | codes[4 * i + 1] << 2 | codes[4 * i + 2] << 4 | codes[4 * i + 3] << 6 for i in range(16)]
    assert q.data.tolist() == [want]
    assert q.zeros.tolist() == [[0.0, min(vals[32:])]]
    assert abs(q.scales[0, 0].item() - 31 / 3) < 1e-5


@pytest.mark.parametrize("bits", [2, 4, 3, 8])
def test_quantize_values_bounds(bits):
    g = torch.Generator().manual_seed(30 + bits)
    v = torch.randn(40, 8, 128, generator=g) * 3
    q = R.quantize_values(v, bits=bits, group_size=32)
    vhat = R.dequantize_values(q, 32)
    err = (v - vhat).abs().reshape(40, 8, 4, 32)
    sc = q.scales.unsqueeze(-1)
    assert torch.all(err <= sc * 0.5 * (1 + 1e-5) + 1e-6)
    codes = R.unpack_values(q).reshape(40, 8, 4, 32).long()
    vg = v.reshape(40, 8, 4, 32)
    assert torch.all(codes.gather(-1, vg.argmin(-1, keepdim=True)) == 0)
    assert torch.all(codes.gather(-1, vg.argmax(-1, keepdim=True)) == 2 ** bits - 1)


def test_quantize_values_constant_groups():
    for dt, want_scale in ((torch.float32, np.float32(1e-10)), (torch.bfloat16, bf16_round(np.float32(1e-10))),
                           (torch.float16, 0.0)):
        v = torch.full((3, 64), 0.75, dtype=dt)
        q = R.quantize_values(v, bits=2, group_size=32)
        assert torch.all(q.data == 0)
        assert np.allclose(q.scales.float().numpy(), want_scale, rtol=0, atol=0)
        assert torch.all(q.zeros.float() == 0.75)


def test_quantize_values_bf16_per_op_rounding():
    g = torch.Generator().manual_seed(40)
    v = (torch.randn(300, 128, generator=g) * 2).bfloat16()
    q = R.quantize_values(v, bits=2, group_size=32)
    x = v.float().numpy().reshape(300, 4, 32)
    lo, hi = x.min(-1, keepdims=True), x.max(-1, keepdims=True)
    sc = bf16_round(bf16_round(hi - lo) / np.float32(3))
    sc = np.maximum(sc, bf16_round(np.float32(1e-10)))
    codes = np.clip(np.rint(bf16_round(bf16_round(x - lo) / sc)), 0, 3).astype(np.uint8).reshape(300, 32, 4)
    packed = codes[..., 0] | codes[..., 1] << 2 | codes[..., 2] << 4 | codes[..., 3] << 6
    assert np.array_equal(q.data.numpy(), packed)
    assert np.array_equal(q.scales.float().numpy(), sc[..., 0])
    assert np.array_equal(q.zeros.float().numpy(), lo[..., 0])


# ------------------------------------------- scalar encoder's error margin ---

def _split_bf16_np(x: np.ndarray):
    """The encoder's truncated bf16 split of fp32 values (x = p0 + p1 + p2)."""
    x = x.astype(np.float32)
    b0 = (x.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    r1 = (x - b0).astype(np.float32)
    b1 = (r1.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    r2 = (r1 - b1).astype(np.float32)
    b2 = (r2.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    return b0, b1, b2


def test_bf16_split_bounds_used_by_the_encoder_margin():
    """x = p0 + p1 + p2 exactly, |p1| < 2^-7 |x|, |p2| < 2^-14 |x| (normal
    range): the skipped cross products are below 2^-21 relative."""
    g = np.random.default_rng(5)
    x = (g.standard_normal(200000) * np.exp2(g.integers(-20, 20, 200000))).astype(np.float32)
    p0, p1, p2 = _split_bf16_np(x)
    assert np.array_equal(p0.astype(np.float64) + p1 + p2, x.astype(np.float64))
    ax = np.abs(x.astype(np.float64))
    assert np.all(np.abs(p1) < ax * 2.0 ** -7) and np.all(np.abs(p2) < ax * 2.0 ** -14)


def test_reference_chain_error_within_128_roundings():
    """The reference's y = u @ M^T (torch-CPU, one sequential FMA chain per
    output) stays within 128 * 2^-24 * S of the exact sum, S = sum |u_d m_d|,
    on inputs built for heavy cancellation (partial sums far above |y|), the
    bound the matrix-core encoder's decision margin uses."""
    g = torch.Generator().manual_seed(6)
    D, N = 128, 4096
    sign = torch.cat([torch.ones(64), -torch.ones(64)])
    M = (sign * 20.0) * (1.0 + 0.01 * torch.randn(D, D, generator=g))       # rows: +A then -A
    u = (1.0 + 0.1 * torch.randn(N, D, generator=g)) / D ** 0.5
    y = (u @ M.T).double()
    y64 = u.double() @ M.double().T
    S = u.double().abs() @ M.double().abs().T
    err = (y - y64).abs() / S
    assert float(err.max()) <= 128 * 2.0 ** -24
    # the construction does cancel: |y| is far below S
    assert float((y64.abs() / S).median()) < 0.05
