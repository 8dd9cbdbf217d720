"""Block-VQ calibration on the device (SMAQBlockVQ.fit(on_device=True)).

The reference fits with torch ops on the calibration data's device
(smaq/block_vq.py:37-79, 160-210); its CPU random stream cannot be reproduced
on the GPU, so the device fit is checked in two ways:

* each kernel against a float64 restatement of its step: shaped keys within
  the rounding bound of an 8-term fp32 chain (the GPU host's CPU sgemm may
  sum in another order, so it is not the comparison), k-means++ distances and
  Lloyd means within 1e-5 relative, empty clusters kept, the update
  deterministic;
* the fitted codebook's quality: held-out logit MSE (smaq/block_vq.py:303-311,
  the reference's own metric) within 10% of the host fit's for the same data
  and seed, and identical per-block metrics.
"""

from __future__ import annotations

import pytest
import torch

import smaq_amd as S
from smaq_amd import _native
from oracle import smaq_ref as R
from tests.conftest import sample_keys

pytestmark = pytest.mark.gpu


def _metrics(queries, nb=16, bd=8):
    Es = []
    for b in range(nb):
        qb = queries[:, b * bd:(b + 1) * bd].float()
        Es.append(R.build_metric((qb.T @ qb) / queries.shape[0]))
    return torch.stack([e[0] for e in Es]), torch.stack([e[1] for e in Es])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_shape_within_fp32_chain_bound(dev, dtype):
    keys = sample_keys(1000, seed=120).to(dtype)
    E, _ = _metrics(sample_keys(512, seed=121))
    x = _native.blockvq_shape(keys.to(dev), E.to(dev)).cpu()
    for b in range(16):
        kb = keys[:, 8 * b:8 * b + 8].double()
        ref = kb @ E[b].double().T
        # an 8-term fp32 chain: within a few units of 2^-24 of sum |k| |E|
        bound = 8 * 2.0 ** -24 * (kb.abs() @ E[b].double().abs().T)
        assert bool(((x[b].double() - ref).abs() <= bound).all()), f"block {b}"


def test_kmeanspp_distances(dev):
    g = torch.Generator().manual_seed(122)
    x = torch.randn(3, 777, 8, generator=g)
    picks = [torch.tensor([5, 0, 776]), torch.tensor([100, 3, 3]), torch.tensor([-4, 900, 7])]
    dmin = torch.empty(3, 777, device=dev)
    ref = None
    for i, p in enumerate(picks):
        _native.kmeanspp_update(x.to(dev), p.to(dev), dmin, first=(i == 0))
        pc = p.clamp(0, 776)  # out-of-range picks are clamped to a row
        d = ((x.double() - x.double()[torch.arange(3), pc][:, None, :]) ** 2).sum(-1)
        ref = d if ref is None else torch.minimum(ref, d)
    torch.testing.assert_close(dmin.cpu().double(), ref, rtol=1e-5, atol=1e-6)


def test_kmeans_update_means_empty_and_deterministic(dev):
    g = torch.Generator().manual_seed(123)
    nb, n, bd, nc = 4, 5000, 8, 256
    x = torch.randn(nb, n, bd, generator=g)
    idx = torch.randint(0, nc - 1, (n, nb), generator=g, dtype=torch.int64)   # centroid nc-1 stays empty
    idx[:, 2] = 7                                                            # block 2: one cluster only
    cents0 = torch.randn(nb, nc, bd, generator=g)
    got = cents0.clone().to(dev)
    _native.kmeans_update(x.to(dev), idx.to(torch.uint8).to(dev), got)
    again = cents0.clone().to(dev)
    _native.kmeans_update(x.to(dev), idx.to(torch.uint8).to(dev), again)
    assert torch.equal(got, again)
    got = got.cpu()
    for b in range(nb):
        for j in range(nc):
            m = idx[:, b] == j
            if m.any():
                torch.testing.assert_close(got[b, j].double(), x[b][m].double().mean(0), rtol=1e-5, atol=1e-6)
            else:
                assert torch.equal(got[b, j], cents0[b, j])


def test_device_fit_quality(dev):
    keys = sample_keys(8192, seed=124)
    queries = sample_keys(8192, seed=125)
    hold_k = sample_keys(4096, seed=126).to(dev)
    hold_q = sample_keys(4096, seed=127).to(dev)
    host = S.SMAQBlockVQ(128, device=dev).fit(keys, queries, kmeans_iters=8, seed=42)
    gpu = S.SMAQBlockVQ(128, device=dev).fit(keys.to(dev), queries.to(dev), kmeans_iters=8, seed=42,
                                             on_device=True)
    assert torch.equal(host.E_blocks.cpu(), gpu.E_blocks.cpu())
    assert torch.isfinite(gpu.centroids).all()
    torch.testing.assert_close(gpu.decoded_centroids.cpu(),
                               gpu.centroids.cpu() @ gpu.E_inv_blocks.cpu().transpose(1, 2),
                               rtol=1e-5, atol=1e-6)
    mse_host = host.logit_mse(hold_q, hold_k)
    mse_gpu = gpu.logit_mse(hold_q, hold_k)
    print(f"\nheld-out logit MSE: host fit {mse_host:.5e}, device fit {mse_gpu:.5e}")
    assert mse_gpu <= 1.10 * mse_host
    # the codebook is used: most centroids of most blocks own a point
    idx = gpu.quantize(keys.to(dev)).indices.long().cpu()
    used = torch.tensor([idx[:, b].unique().numel() for b in range(16)])
    assert int(used.min()) >= 200


def test_device_fit_small_calibration(dev):
    keys = sample_keys(100, seed=128)
    vq = S.SMAQBlockVQ(128, device=dev).fit(keys.to(dev), keys.to(dev), kmeans_iters=3, on_device=True)
    x = _native.blockvq_shape(keys.to(dev), vq.E_blocks).cpu()
    assert torch.equal(vq.centroids[:, :100].cpu(), x)
    assert not vq.centroids[:, 100:].any()
