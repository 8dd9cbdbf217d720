"""GPU parity of the codec kernels against the CPU oracle on identical seeded
inputs.  Integer outputs (packed codes, block-VQ indices, packed values) must
be bit-exact; the only tolerated code differences are boundary/argmin ties
within 1e-6 relative, which are counted and printed.  Floating outputs
(norms, scales, zeros) are bit-exact except where noted."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import smaq_amd as S
from smaq_amd import _native
from oracle import smaq_ref as R
from tests.conftest import sample_keys, spectral_sigma

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _store_view(x: torch.Tensor) -> torch.Tensor:
    """[T, Hkv, D] -> [1, Hkv, T, D] transpose view, as the store passes it."""
    return x.transpose(0, 1).unsqueeze(0)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("bits", [2, 4, 3, 8])
@pytest.mark.parametrize("T", [1, 7, 129])
def test_pack_values_bit_exact(dev, dtype, bits, T):
    g = torch.Generator().manual_seed(bits * 100 + T)
    v = (torch.randn(T, 8, 128, generator=g) * 2).to(dtype)
    v[:, 0, :32] = 0.5                              # a constant group
    v[0, 1, 32:64] = torch.linspace(-1, 1, 32).to(dtype)
    ref = R.quantize_values(_store_view(v), bits=bits, group_size=32)
    got = S.quantize_values(_store_view(v.to(dev)), bits=bits, group_size=32)
    assert torch.equal(got.data.cpu(), ref.data)
    assert torch.equal(got.scales.cpu(), ref.scales)
    assert torch.equal(got.zeros.cpu(), ref.zeros)
    back = S.dequantize_values(got, 32).cpu()
    assert torch.equal(back, R.dequantize_values(ref, 32))


@pytest.mark.parametrize("bits", [2, 4])
def test_pack_values_bf16_wide_range(dev, bits):
    """The bf16 group-32 packer divides by multiplying with RN(1 / scale);
    the codes must still equal the true division's on every row: 65536 rows
    at magnitudes 1e-35..1e35, constant rows, two-level rows, exact multiples
    of the step, subnormal and non-finite values."""
    g = torch.Generator().manual_seed(140 + bits)
    n = 65536
    mag = torch.pow(10.0, torch.empty(n, 1).uniform_(-35, 35, generator=g))
    v = torch.randn(n, 128, generator=g) * mag
    v[:512] = 3.25                                                   # constant groups
    v[512:1024] = torch.where(torch.rand(512, 128, generator=g) < 0.5, -1.0, 2.0)   # two levels
    step = torch.pow(2.0, torch.randint(-10, 10, (1024, 1), generator=g).float())
    lev = (1 << bits) - 1
    v[1024:2048] = torch.randint(0, 4 * lev + 1, (1024, 128), generator=g).float() * step / 4   # multiples
    v[2048:2560] = torch.randn(512, 128, generator=g) * 1e-39        # subnormal in bf16
    v[2560, 5] = float("nan")
    v[2561, 40] = float("inf")
    v[2562, 70] = -float("inf")
    vb = v.bfloat16()
    ref = R.quantize_values(vb, bits=bits, group_size=32)
    got = S.quantize_values(vb.to(dev), bits=bits, group_size=32)
    bad = (got.data.cpu() != ref.data).any(1)
    assert not bad.any(), f"{int(bad.sum())} rows differ, first {int(bad.nonzero()[0])}"
    # scales / zeros bit for bit, a NaN matching any NaN: the NaN group's
    # payload comes from the host CPU's vector min (0x7fc0 on one machine,
    # 0xffff on another), the kernel writes the canonical 0x7fc0
    for name in ("scales", "zeros"):
        a, b = getattr(got, name).cpu(), getattr(ref, name)
        an, bn = a.isnan(), b.isnan()
        assert torch.equal(an, bn) and int(an.sum()) == 1, name
        assert torch.equal(a[~an].view(torch.int16), b[~bn].view(torch.int16)), name


@pytest.mark.parametrize("group", [16, 64, 128])
def test_pack_values_groups(dev, group):
    v = torch.randn(3, 50, 128, generator=torch.Generator().manual_seed(group)).bfloat16()
    ref = R.quantize_values(v, bits=2, group_size=group)
    got = S.quantize_values(v.to(dev), bits=2, group_size=group)
    assert torch.equal(got.data.cpu(), ref.data) and torch.equal(got.scales.cpu(), ref.scales)


def test_pack_values_errors(dev):
    with pytest.raises(ValueError):
        S.quantize_values(torch.randn(2, 100, device=dev), bits=2, group_size=32)


def _calibrated(bits, seed=0):
    q = sample_keys(64, seed=seed + 70)
    E, Ei = R.build_metric(R.fit_sigma_centered(q))
    return q, E, Ei


def _ties_ok(got_codes, ref_codes, y_ref, bounds):
    mism = got_codes != ref_codes
    if not mism.any():
        return 0
    yv = y_ref[mism]
    b = bounds.double()
    near = ((yv.double()[:, None] - b[None]).abs() <= 1e-6 * torch.maximum(b.abs()[None], yv.double().abs()[:, None]).clamp_min(1e-6)).any(1)
    assert bool(near.all()), f"{int((~near).sum())} code mismatches away from any boundary"
    return int(mism.sum())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_scalar_encode_parity(dev, dtype, bits):
    q, E, Ei = _calibrated(bits)
    qz = S.SMAQQuantizer(128, bits=bits, device=dev)
    qz.fit(q)
    assert torch.equal(qz.E.cpu(), E) and torch.equal(qz.E_inv.cpu(), Ei)
    keys = sample_keys(37 * 8, seed=bits).reshape(37, 8, 128).to(dtype)
    _, _, db = R.scalar_tables(bits)
    ref = R.scalar_encode(_store_view(keys), E, db, bits)
    qz.tie_counter = _native.TieCounter(dev)
    got = qz.quantize(_store_view(keys.to(dev)))
    ties = qz.tie_counter.value()
    y = R.scalar_y(_store_view(keys), E)
    ref_codes = R.unpack_codes(ref.indices, bits, 128)
    got_codes = R.unpack_codes(got.indices.cpu(), bits, 128)
    n_mis = _ties_ok(got_codes, ref_codes, y, db)
    print(f"\n[scalar {dtype} {bits}b] code mismatches={n_mis} boundary-ties(gpu)={ties}")
    assert n_mis == 0                 # same FMA order as MKL: exact
    assert got.norms.dtype == dtype
    assert torch.equal(got.norms.cpu(), ref.norms)


def test_scalar_encode_contiguous_and_small_row_counts(dev):
    q, E, Ei = _calibrated(3)
    qz = S.SMAQQuantizer(128, bits=3, device=dev).fit(q)
    _, _, db = R.scalar_tables(3)
    for n in (1, 5, 6, 1000):
        k = sample_keys(n, seed=n)
        got = qz.quantize(k.to(dev))
        ref = R.scalar_encode(k, E, db, 3)
        y = R.scalar_y(k, E)
        n_mis = _ties_ok(R.unpack_codes(got.indices.cpu(), 3, 128), R.unpack_codes(ref.indices, 3, 128), y, db)
        # MKL uses a different summation order below 6 rows; codes may then
        # differ only at boundary ties
        if n >= 6:
            assert n_mis == 0
        assert torch.equal(got.norms.cpu(), ref.norms)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_rotation_adapter_parity(dev, bits):
    sigma, u, _ = spectral_sigma(128, 5)
    rot = torch.linalg.qr(torch.randn(128, 128, generator=torch.Generator().manual_seed(9)))[0]
    ad = S.RotationAdapter(128, bits=bits, Sigma_q=sigma, rotation=rot, device=dev)
    cs = ad.coord_scales.cpu()
    assert torch.equal(cs, R.diag_metric_scales(sigma, rot))
    keys = sample_keys(300, seed=31)
    c, _, db = R.midpoint_tables(bits)
    ref = R.scalar_encode(keys, rot, db, bits, coord_scales=cs)
    got = ad.quantize(keys.to(dev))
    y = R.scalar_y(keys, rot, cs)
    assert _ties_ok(R.unpack_codes(got.indices.cpu(), bits, 128), R.unpack_codes(ref.indices, bits, 128), y, db) == 0
    inv = 1.0 / cs.clamp(min=1e-6)
    ref_hat = R.rotation_dequantize(ref, c, inv, rot, 128)
    torch.testing.assert_close(ad.dequantize(got).cpu(), ref_hat, atol=1e-5, rtol=1e-5)
    query = sample_keys(6, seed=32)
    s_ref = R.rotation_scores(query, ref, c, inv, rot, 128, scale=0.09)
    torch.testing.assert_close(ad.attention_score(query.to(dev), got, scale=0.09).cpu(), s_ref, atol=1e-4, rtol=1e-4)


def test_scalar_dequant_scores_rotate(dev):
    q, E, Ei = _calibrated(4)
    qz = S.SMAQQuantizer(128, bits=4, device=dev).fit(q)
    c, _, db = R.scalar_tables(4)
    keys = sample_keys(257, seed=41)
    ref = R.scalar_encode(keys, E, db, 4)
    got = qz.quantize(keys.to(dev))
    torch.testing.assert_close(qz.dequantize(got).cpu(), R.smaq_dequantize(ref, c, Ei, 128), atol=1e-5, rtol=1e-5)
    query = sample_keys(12, seed=42).reshape(3, 4, 128)
    torch.testing.assert_close(qz.rotate_query(query.to(dev)).cpu(), query @ Ei.T, atol=1e-5, rtol=1e-5)
    s_ref = R.smaq_scores(query, ref, c, Ei, 128, scale=0.088)
    for uk in (False, True):
        s = qz.attention_score(query.to(dev), got, scale=0.088, use_kernel=uk)
        torch.testing.assert_close(s.cpu(), s_ref, atol=2e-4, rtol=1e-4)
    from smaq_amd.kernels import smaq_attention_scores
    raw = smaq_attention_scores(qz, query[0].to(dev), got)
    torch.testing.assert_close(raw.cpu(), R.smaq_scores(query[0], ref, c, Ei, 128), atol=2e-3, rtol=1e-4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("scaled", [False, True])
def test_rotate_rows_128_chunking_and_accuracy(dev, dtype, scaled):
    """smaq_rotate_rows at head_dim 128 (the decode query rotation): each
    output is eight 16-term fmaf chains summed in a fixed tree, an order set
    by the row alone, so 5001 rows in one call (8-row blocks, the last one
    partial) equal the same rows in calls of 301 (4-row blocks), 2499 and
    2201 rows, and rows read from a buffer that is not 16-byte aligned
    (element loads instead of 16-byte loads), bit for bit, and match the
    float64 product within the rounding bound of a 20-step fp32 evaluation
    (16 chained products, 3 tree levels, the scale)."""
    g = torch.Generator().manual_seed(130)
    M = torch.linalg.qr(torch.randn(128, 128, generator=g, dtype=torch.float64))[0].float()
    cs = (torch.rand(128, generator=g) + 0.5) if scaled else None
    x = torch.randn(5001, 128, generator=g).to(dtype)
    Mt, csd = M.T.contiguous().to(dev), None if cs is None else cs.to(dev)
    xd = x.to(dev)
    whole = torch.empty(5001, 128, device=dev)
    _native.rotate_rows_into(xd, Mt, csd, whole)
    parts = torch.empty(5001, 128, device=dev)
    _native.rotate_rows_into(xd[:301], Mt, csd, parts[:301])
    _native.rotate_rows_into(xd[301:2800], Mt, csd, parts[301:2800])
    _native.rotate_rows_into(xd[2800:], Mt, csd, parts[2800:])
    assert torch.equal(whole, parts)
    buf = torch.empty(5001 * 128 + 1, dtype=dtype, device=dev)
    xm = buf[1:].view(5001, 128)
    xm.copy_(xd)
    assert xm.data_ptr() % 16 != 0
    odd = torch.empty(5001, 128, device=dev)
    _native.rotate_rows_into(xm, Mt, csd, odd)
    assert torch.equal(whole, odd)
    ref = x.double() @ M.T.double()
    if cs is not None:
        ref = ref * cs.double()
    bound = 21 * 2.0 ** -24 * (x.double().abs() @ M.T.double().abs()) * (1.0 if cs is None else cs.double() * 2)
    assert bool(((whole.cpu().double() - ref).abs() <= bound + 1e-30).all())


def _vq_setup(nb=16, bd=8, nc=256, seed=0, n_fit=4096):
    keys = sample_keys(n_fit, seed=seed + 80)
    queries = sample_keys(n_fit, seed=seed + 81)
    Eb, Eib, C, Dc = R.blockvq_fit(keys, queries, block_dim=bd, n_centroids=nc, iters=5, seed=42)
    return Eb, Eib, C, Dc


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("bd", [8, 2])
def test_blockvq_encode_parity(dev, dtype, bd):
    Eb, Eib, C, Dc = _vq_setup(nb=128 // bd, bd=bd)
    vq = S.SMAQBlockVQ(128, block_dim=bd, device=dev)
    vq.E_blocks, vq.E_inv_blocks = Eb.to(dev), Eib.to(dev)
    vq.centroids, vq.decoded_centroids = C.to(dev), Dc.to(dev)
    keys = sample_keys(3000, seed=51).to(dtype)
    ref = R.blockvq_encode(keys, Eb, C).indices
    vq.tie_counter = _native.TieCounter(dev)
    got = vq.quantize(keys.to(dev)).indices.cpu().long()
    ties = vq.tie_counter.value()
    mism = got != ref
    n_mis = int(mism.sum())
    if n_mis:
        d = R.blockvq_distances(keys, Eb, C)
        r_idx = mism.nonzero()
        dg = d[r_idx[:, 0], r_idx[:, 1], got[mism]]
        dr = d[r_idx[:, 0], r_idx[:, 1], ref[mism]]
        assert bool(((dg - dr).abs() <= 1e-6 * dr.clamp_min(1e-30)).all()), "index mismatch beyond a tie"
    print(f"\n[blockvq {dtype} bd={bd}] index mismatches={n_mis} argmin-ties(gpu)={ties}")
    assert n_mis <= ties
    k_hat = vq.dequantize(S.BlockVQQuantized(got.to(dev).to(torch.uint8), 128 // bd, bd)).cpu()
    assert torch.equal(k_hat, R.blockvq_dequantize(R.BlockQ(got, 128 // bd, bd), Dc))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_blockvq_encode_eight_blocks(dev, dtype):
    """head_dim 64 (eight 8-dim blocks): the matrix-core encoder's rows hold
    fewer than 16 indices, so each token's indices leave byte by byte; odd
    row counts leave a partly filled last 64-token set."""
    d, bd = 64, 8
    Eb, Eib, C, Dc = R.blockvq_fit(sample_keys(4096, d=d, seed=90), sample_keys(4096, d=d, seed=91),
                                   block_dim=bd, n_centroids=256, iters=5, seed=42)
    vq = S.SMAQBlockVQ(d, block_dim=bd, device=dev)
    vq.E_blocks, vq.E_inv_blocks = Eb.to(dev), Eib.to(dev)
    vq.centroids, vq.decoded_centroids = C.to(dev), Dc.to(dev)
    keys = sample_keys(2999, d=d, seed=92).to(dtype)
    ref = R.blockvq_encode(keys, Eb, C).indices
    vq.tie_counter = _native.TieCounter(dev)
    got = vq.quantize(keys.to(dev)).indices.cpu().long()
    assert got.shape == ref.shape == (2999, d // bd)
    _check_vq_against_oracle(got, ref, keys, Eb, C, vq.tie_counter.value(), f"head_dim 64 {dtype}")


def _check_vq_against_oracle(idx_gpu, ref, keys, Eb, C, ties, what):
    """Indices equal the oracle's except at counted argmin ties (distances
    within 1e-6 relative of each other)."""
    mism = idx_gpu != ref
    n_mis = int(mism.sum())
    if n_mis:
        d = R.blockvq_distances(keys, Eb, C)
        r_idx = mism.nonzero()
        dg = d[r_idx[:, 0], r_idx[:, 1], idx_gpu[mism]]
        dr = d[r_idx[:, 0], r_idx[:, 1], ref[mism]]
        assert bool(((dg - dr).abs() <= 1e-6 * dr.clamp_min(1e-30)).all()), f"{what}: mismatch beyond a tie"
    print(f"\n[{what}] index mismatches={n_mis} argmin-ties(gpu)={ties}")
    assert n_mis <= ties


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_blockvq_encode_matrix_core_large(dev, dtype):
    """The matrix-core encoder (8-dim blocks, 256 centroids) on 40,000 rows:
    about 1e-3 of the (row, block) pairs take its exact recount, so this
    covers both paths against the oracle; the rows also go through the
    store's [T, Hkv, D] transpose view (strided row map)."""
    Eb, Eib, C, Dc = _vq_setup(seed=3)
    vq = S.SMAQBlockVQ(128, block_dim=8, device=dev)
    vq.E_blocks, vq.E_inv_blocks = Eb.to(dev), Eib.to(dev)
    vq.centroids, vq.decoded_centroids = C.to(dev), Dc.to(dev)
    keys = sample_keys(40000, seed=57).to(dtype)
    ref = R.blockvq_encode(keys, Eb, C).indices
    vq.tie_counter = _native.TieCounter(dev)
    got = vq.quantize(keys.to(dev)).indices.cpu().long()
    _check_vq_against_oracle(got, ref, keys, Eb, C, vq.tie_counter.value(), f"blockvq mfma {dtype}")
    kv = keys.reshape(10000, 4, 128)
    vq.tie_counter = _native.TieCounter(dev)
    got_v = vq.quantize(_store_view(kv.to(dev))).indices.cpu().long()   # [1, 4, T, 16]
    assert torch.equal(got_v[0].transpose(0, 1).reshape(40000, 16), got)


@pytest.mark.parametrize("scale", [1e-6, 1.0, 1e6])
def test_blockvq_encode_matrix_core_ranges(dev, scale):
    """The matrix-core encoder on 8 blocks (head_dim 64), a codebook far from
    unit scale (the per-block power-of-two rescaling) and keys whose shaped
    components exceed the f16 operand range (|x| > 2^13 / sigma: those pairs
    take the exact recount): indices as the oracle's up to counted ties."""
    D, nb = 64, 8
    keys0 = sample_keys(4096, seed=150)[:, :D] * scale
    Eb, Eib, C, Dc = R.blockvq_fit(keys0, sample_keys(4096, seed=151)[:, :D] * scale, block_dim=8,
                                   n_centroids=256, iters=3, seed=42)
    vq = S.SMAQBlockVQ(D, block_dim=8, device=dev)
    vq.E_blocks, vq.E_inv_blocks = Eb.to(dev), Eib.to(dev)
    vq.centroids, vq.decoded_centroids = C.to(dev), Dc.to(dev)
    keys = sample_keys(6000, seed=152)[:, :D] * scale
    keys[::7] *= 3.0e4          # shaped components far beyond the codebook's range
    keys[3, :8] = 0.0           # an all-zero block
    ref = R.blockvq_encode(keys, Eb, C).indices
    vq.tie_counter = _native.TieCounter(dev)
    got = vq.quantize(keys.to(dev)).indices.cpu().long()
    _check_vq_against_oracle(got, ref, keys, Eb, C, vq.tie_counter.value(), f"blockvq nb=8 scale {scale:g}")


def test_blockvq_encode_nonfinite_codebook(dev):
    """A NaN or infinite centroid component: the reference's cdist gives NaN
    distances and its argmin returns the first NaN's index (every key of the
    NaN block; the keys whose shaped component meets the infinity with the
    opposite sign); the matrix-core encoder sends such blocks to its exact
    recount and must return the same indices."""
    Eb, Eib, C, Dc = _vq_setup(seed=6)
    C = C.clone()
    C[3, 17, 2] = float("nan")
    C[5, 40, 0] = float("inf")
    vq = S.SMAQBlockVQ(128, block_dim=8, device=dev)
    vq.E_blocks, vq.E_inv_blocks = Eb.to(dev), Eib.to(dev)
    vq.centroids, vq.decoded_centroids = C.to(dev), Dc.to(dev)
    keys = sample_keys(2000, seed=92)
    ref = R.blockvq_encode(keys, Eb, C).indices
    got = vq.quantize(keys.to(dev)).indices.cpu().long()
    assert bool((ref[:, 3] == 17).all()) and bool((ref[:, 5] == 40).any())
    assert torch.equal(got[:, 3], ref[:, 3]) and torch.equal(got[:, 5], ref[:, 5])
    _check_vq_against_oracle(got, ref, keys, Eb, C, 2 ** 31, "blockvq non-finite codebook")


def test_blockvq_encode_exact_ties(dev):
    """Constructed ties: duplicated centroids (exactly equal distances, the
    first index wins), keys shaped onto midpoints of two centroids (distances
    equal up to rounding: the exact recount decides as the reference does and
    counts the tie) and a row with a NaN (the first index wins, not counted)."""
    Eb, Eib, C, Dc = _vq_setup(seed=4)
    C = C.clone()
    C[:, 200] = C[:, 7]          # exact duplicates: index 7 must win over 200
    C[:, 201] = C[:, 90]
    nb = C.shape[0]
    g = torch.Generator().manual_seed(91)
    rows = 600
    x = torch.empty(rows, nb, 8)
    for b in range(nb):
        a = torch.randint(0, 256, (rows,), generator=g)
        c2 = torch.randint(0, 256, (rows,), generator=g)
        mid = 0.5 * (C[b, a] + C[b, c2])
        x[:, b] = torch.where((torch.arange(rows) % 3 == 0)[:, None], C[b, 7] + 1e-3 * torch.randn(rows, 8, generator=g), mid)
    # keys whose shaped blocks are x: k_b = x_b E_b^-T
    keys = torch.cat([x[:, b] @ torch.linalg.inv(Eb[b]).T for b in range(nb)], dim=1).float()
    keys[5, 17] = float("nan")
    vq = S.SMAQBlockVQ(128, block_dim=8, device=dev)
    vq.E_blocks, vq.E_inv_blocks = Eb.to(dev), Eib.to(dev)
    vq.centroids, vq.decoded_centroids = C.to(dev), Dc.to(dev)
    ref = R.blockvq_encode(keys, Eb, C).indices
    vq.tie_counter = _native.TieCounter(dev)
    got = vq.quantize(keys.to(dev)).indices.cpu().long()
    ties = vq.tie_counter.value()
    fin = torch.isfinite(keys).all(dim=1)
    # These distances tie up to rounding, and the reference's own rounding is
    # host dependent: torch's CPU matmul for the cdist form sums its 10 terms
    # in an order that depends on the CPU's SIMD kernels (this build's oracle
    # host and the GPU host differ), shifting d2 by a few ulps of |x|^2 + |c|^2
    # -- many ulps of d2 itself.  A differing index must be a tie under that
    # bound, computed in float64 from the oracle's shaped keys.
    kf, gf, rf = keys[fin], got[fin], ref[fin]
    mism = (gf != rf).nonzero()
    for r, b in mism.tolist():
        xb = (kf[r:r + 1, 8 * b:8 * b + 8] @ Eb[b].T)[0].double()
        cg, cr = C[b, gf[r, b]].double(), C[b, rf[r, b]].double()
        d2g, d2r = ((xb - cg) ** 2).sum(), ((xb - cr) ** 2).sum()
        bound = 32 * 2.0 ** -24 * (2 * (xb * xb).sum() + (cg * cg).sum() + (cr * cr).sum())
        assert abs(float(d2g - d2r)) <= float(bound), f"row {r} block {b}: {float(d2g)} vs {float(d2r)}"
    print(f"\n[blockvq constructed ties] index differences={len(mism)} (all within the rounding bound) "
          f"argmin-ties(gpu)={ties}")
    assert torch.equal(got[~fin][:, 2], ref[~fin][:, 2])      # NaN block: first index (0)
    assert int(got[~fin][0, 2]) == 0
    assert ties > 0


def test_blockvq_fit_matches_oracle(dev):
    keys = sample_keys(2048, seed=90)
    queries = sample_keys(2048, seed=91)
    vq = S.SMAQBlockVQ(128, block_dim=8, n_centroids=64, device=dev).fit(keys, queries, kmeans_iters=3)
    Eb, Eib, C, Dc = R.blockvq_fit(keys, queries, block_dim=8, n_centroids=64, iters=3)
    assert torch.equal(vq.E_blocks.cpu(), Eb) and torch.equal(vq.centroids.cpu(), C)
    assert torch.equal(vq.decoded_centroids.cpu(), Dc)


@pytest.mark.parametrize("bits", [3, 4])
def test_scalar_encode_near_boundaries(dev, bits):
    """Keys constructed so that many y = u E^T land on or within 1e-7..1e-4 of
    a decision boundary: the matrix-core encoder must recount those from the
    exact chain (codes equal the oracle's; the tie counter equals the number
    of elements within 1e-6 relative of a boundary)."""
    q, E, Ei = _calibrated(bits)
    qz = S.SMAQQuantizer(128, bits=bits, device=dev).fit(q)
    _, _, db = R.scalar_tables(bits)
    g = torch.Generator().manual_seed(77 + bits)
    rows = 512
    # random unit u; in each row the 32 coordinates of y = u E^T closest to a
    # boundary are moved onto it (+ offsets 0 .. 1e-4), re-solving u = y E^-T
    # and its normalisation a few times so the targets survive ||u|| = 1
    E64, Ei64 = E.double(), Ei.double()
    u = torch.randn(rows, 128, generator=g, dtype=torch.float64)
    u = u / u.norm(dim=1, keepdim=True)
    y0 = u @ E64.T
    bd = db.double()
    dist = (y0[..., None] - bd).abs()
    near_b = bd[dist.argmin(-1)]
    sel = dist.min(-1).values.argsort(dim=1)[:, :32]
    offs = torch.tensor([0.0, 1e-7, -1e-7, 1e-6, -1e-6, 1e-5, -1e-5, 1e-4], dtype=torch.float64)
    tgt = near_b.gather(1, sel) + offs[torch.randint(0, offs.numel(), sel.shape, generator=g)]
    y = y0.clone()
    scale = torch.ones(rows, 1, dtype=torch.float64)
    for _ in range(8):
        y.scatter_(1, sel, tgt * scale)
        u = y @ Ei64.T
        scale = u.norm(dim=1, keepdim=True)
    keys = (u / scale * 3.0).float()
    ref = R.scalar_encode(keys, E, db, bits)
    qz.tie_counter = _native.TieCounter(dev)
    got = qz.quantize(keys.to(dev))
    yr = R.scalar_y(keys, E)
    gc, rc = R.unpack_codes(got.indices.cpu(), bits, 128), R.unpack_codes(ref.indices, bits, 128)
    assert torch.equal(gc, rc)
    bd = db.double()
    tol = 1e-6 * torch.maximum(bd.abs()[None, None], yr.double().abs()[..., None]).clamp_min(1e-6)
    n_ties = int(((yr.double()[..., None] - bd[None, None]).abs() <= tol).any(-1).sum())
    print(f"\n[near-boundary {bits}b] ties={n_ties} gpu={qz.tie_counter.value()}")
    assert qz.tie_counter.value() == n_ties
    assert torch.equal(got.norms.cpu(), ref.norms)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_scalar_encode_cancellation_matches_the_chain(dev, dtype):
    """Keys and a metric built for heavy cancellation: every y_j is a sum of
    128 terms whose partial sums reach ~100x |y_j|, so the reference chain's
    own rounding (up to a few 2^-24 S) decides codes near decision
    boundaries.  The encoder must reproduce the chain exactly: codes equal the
    oracle's everywhere, ties included (every undecided coordinate is
    recounted with the chain)."""
    g = torch.Generator().manual_seed(7)
    D, N = 128, 65536
    sign = torch.cat([torch.ones(64), -torch.ones(64)])
    M = (sign * 20.0) * (1.0 + 0.01 * torch.randn(D, D, generator=g))
    k = ((1.0 + 0.1 * torch.randn(N, D, generator=g)) * 3.0).to(dtype)
    qz = S.SMAQQuantizer(D, bits=4, device=dev, E=M, E_inv=torch.linalg.inv(M))
    got = qz.quantize(k.to(dev))
    _, _, db = R.scalar_tables(4)
    ref = R.scalar_encode(k, M, db, 4)
    y = R.scalar_y(k, M).double()
    S_ = (k.float() / (k.float().norm(dim=-1, keepdim=True))).double().abs() @ M.double().abs().T
    near = ((y[..., None] - db.double()).abs() < 128 * 2.0 ** -24 * S_[..., None]).any(-1)
    print(f"\n[cancellation {dtype}] coordinates within the chain-error band of a boundary: {int(near.sum())}")
    assert int(near.sum()) > 100          # the construction exercises the recount
    assert torch.equal(got.indices.cpu(), ref.indices)
    assert torch.equal(got.norms.cpu(), ref.norms)
