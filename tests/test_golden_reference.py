"""Checks against tests/golden/reference_calibration.npz, written from the
reference itself by tests/golden/make_golden.py.  These pin the functions no
closed form pins: the k-means++ / Lloyd codebook RNG stream
(smaq/block_vq.py:37-79), the per-block calibration (smaq/block_vq.py:160-210)
and the RotationAdapter sweep (smaq/weighted_scalar.py:228-340)."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import smaq_amd as S
from oracle import smaq_ref as R

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_calibration.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture()
def one_thread():
    # the fixture was written single-threaded; torch-CPU reductions inside
    # cdist / multinomial follow the thread split
    n = torch.get_num_threads()
    torch.set_num_threads(1)
    yield
    torch.set_num_threads(n)


def test_kmeans_codebook_stream(gold, one_thread):
    data = torch.from_numpy(gold["kmeans_data"])
    assert np.array_equal(R.kmeans(data, 16, n_iters=5, seed=42).numpy(), gold["kmeans_c16_i5_s42"])
    assert np.array_equal(R.kmeans(data, 16, n_iters=0, seed=3).numpy(), gold["kmeans_c16_i0_s3"])
    small = torch.from_numpy(gold["kmeans_small_data"])
    assert np.array_equal(R.kmeans(small, 16, n_iters=5, seed=42).numpy(), gold["kmeans_small_c16"])


def test_blockvq_fit_oracle_and_host(gold, one_thread):
    keys, queries = torch.from_numpy(gold["bvq_keys"]), torch.from_numpy(gold["bvq_queries"])
    E, Ei, C, Dc = R.blockvq_fit(keys, queries, block_dim=8, n_centroids=16, iters=4, seed=42)
    for got, name in ((E, "bvq_E_blocks"), (Ei, "bvq_E_inv_blocks"), (C, "bvq_centroids"),
                      (Dc, "bvq_decoded_centroids")):
        assert np.array_equal(got.numpy(), gold[name]), name
    # the library's host-side calibration is the same computation
    vq = S.SMAQBlockVQ(16, block_dim=8, n_centroids=16, device="cpu").fit(keys, queries, kmeans_iters=4, seed=42)
    assert np.array_equal(vq.E_blocks.numpy(), gold["bvq_E_blocks"])
    assert np.array_equal(vq.centroids.numpy(), gold["bvq_centroids"])
    assert np.array_equal(vq.decoded_centroids.numpy(), gold["bvq_decoded_centroids"])


@pytest.mark.gpu
def test_rotation_adapter_sweep(gold, dev, one_thread):
    """The library's sweep (GPU encode/decode of each candidate) picks the
    reference's winner; per-candidate held-out logit MSE within 1e-4 rel."""
    rot = torch.from_numpy(gold["ra_rotation"])
    rq, rk = torch.from_numpy(gold["ra_queries"]), torch.from_numpy(gold["ra_keys"])
    best, res = S.RotationAdapter.fit(16, 3, rq.to(dev), rk.to(dev), rotation=rot, device=dev)
    assert res["best_c"] == float(gold["ra_best_c"])
    assert bool(res["best_use_rotation"]) == bool(gold["ra_best_use_rotation"])
    lm = np.array([e["lmse"] for e in res["all_results"]])
    np.testing.assert_allclose(lm, gold["ra_lmse"], rtol=1e-4)
    # coord scales come from host LAPACK eigh + MKL matmuls; the GPU box's CPU
    # takes other vector code paths than the machine that wrote the fixture
    np.testing.assert_allclose(best.coord_scales.float().cpu().numpy(), gold["ra_best_coord_scales"], rtol=2e-5)
