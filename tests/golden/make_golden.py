"""Writes tests/golden/reference_calibration.npz from the reference itself.

Run in the build container only (the reference tree is not on the GPU box):

    python tests/golden/make_golden.py

The reference is imported from /root/reference for the functions whose
output no closed form or invariant pins: the k-means++ / Lloyd codebook
(RNG stream: ``smaq/block_vq.py:37-79``), the per-block calibration that
feeds it (``smaq/block_vq.py:160-210``) and the RotationAdapter tuning sweep
(``smaq/weighted_scalar.py:228-340``).  Inputs are seeded here and stored
next to the outputs; the fixture holds numbers only.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference"


def main() -> None:
    sys.path.insert(0, REF)
    from smaq.block_vq import SMAQBlockVQ, _kmeans  # noqa: E402  (reference)
    from smaq.weighted_scalar import RotationAdapter  # noqa: E402  (reference)

    torch.set_num_threads(1)
    out = {}
    g = torch.Generator().manual_seed(7)
    # k-means on a small 8-dim cloud, and the n <= k early return
    data = torch.randn(600, 8, generator=g) * torch.linspace(0.2, 2.0, 8)
    out["kmeans_data"] = data.numpy()
    out["kmeans_c16_i5_s42"] = _kmeans(data, 16, n_iters=5, seed=42).numpy()
    out["kmeans_c16_i0_s3"] = _kmeans(data, 16, n_iters=0, seed=3).numpy()
    out["kmeans_small_data"] = data[:10].numpy()
    out["kmeans_small_c16"] = _kmeans(data[:10], 16, n_iters=5, seed=42).numpy()

    # block-VQ calibration: 2 blocks of 8 dims, 16 centroids
    keys = torch.randn(512, 16, generator=g) * torch.linspace(0.3, 1.5, 16)
    queries = torch.randn(512, 16, generator=g) * torch.linspace(1.5, 0.3, 16)
    vq = SMAQBlockVQ(head_dim=16, block_dim=8, n_centroids=16).fit(keys, queries, kmeans_iters=4, seed=42)
    out["bvq_keys"] = keys.numpy()
    out["bvq_queries"] = queries.numpy()
    out["bvq_E_blocks"] = vq.E_blocks.numpy()
    out["bvq_E_inv_blocks"] = vq.E_inv_blocks.numpy()
    out["bvq_centroids"] = vq.centroids.numpy()
    out["bvq_decoded_centroids"] = vq.decoded_centroids.numpy()

    # RotationAdapter sweep (dim 16, 3 bits, random orthogonal rotation)
    a = torch.randn(16, 16, generator=g)
    rot, r = torch.linalg.qr(a)
    rot = rot * torch.sign(torch.diagonal(r)).unsqueeze(0)
    rq = torch.randn(256, 16, generator=g) * torch.linspace(2.0, 0.2, 16)
    rk = torch.randn(256, 16, generator=g)
    best, res = RotationAdapter.fit(16, 3, rq, rk, rotation=rot, device=torch.device("cpu"))
    out["ra_rotation"] = rot.numpy()
    out["ra_queries"] = rq.numpy()
    out["ra_keys"] = rk.numpy()
    out["ra_best_c"] = np.array(res["best_c"], dtype=np.float64)
    out["ra_best_use_rotation"] = np.array(bool(res["best_use_rotation"]))
    out["ra_lmse"] = np.array([e["lmse"] for e in res["all_results"]], dtype=np.float64)
    out["ra_c"] = np.array([e["c"] for e in res["all_results"]], dtype=np.float64)
    out["ra_use_rotation"] = np.array([e["use_rotation"] for e in res["all_results"]])
    out["ra_best_coord_scales"] = best.coord_scales.numpy()

    path = os.path.join(HERE, "reference_calibration.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
