"""Rotation + per-coordinate-scale scalar quantizer (drop-in for
smaq/weighted_scalar.py).

``x_unit -> (x_unit R^T) * s -> scalar codes`` with midpoint decision
boundaries.  The encoder, dequantiser and scores share the scalar-codec HIP
kernels of ``smaq_amd.quantizer``; codebook and scale construction and the
``fit`` sweep run on the host.
"""

from __future__ import annotations

import torch

from smaq_amd import _native
from smaq_amd.quantizer import (SMAQQuantized, _normal_ppf, _pack_indices,  # noqa: F401
                                _unpack_indices, default_device, scores_from_codes)
from smaq_amd.ssf import ssf_log


def build_codebook(bits: int, device: torch.device, dtype: torch.dtype,
                   centroids: torch.Tensor | None = None, boundaries: torch.Tensor | None = None):
    """Gaussian-quantile centroids with midpoint boundaries, or the caller's
    own tables (smaq/weighted_scalar.py:22-51)."""
    if centroids is None:
        probs = torch.linspace(0.0, 1.0, (2 ** bits) + 2, dtype=torch.float32)[1:-1]
        centroids = _normal_ppf(probs).to(dtype=dtype)
    else:
        centroids = centroids.detach().to("cpu", dtype)
    if boundaries is None:
        full = torch.empty(centroids.shape[0] + 1, dtype=dtype)
        full[0] = -float("inf")
        full[-1] = float("inf")
        full[1:-1] = 0.5 * (centroids[:-1] + centroids[1:])
        boundaries = full
    else:
        boundaries = boundaries.detach().to("cpu", dtype)
    return centroids.to(device), boundaries.to(device)


def build_rotated_diagonal_metric_scales(Sigma_q: torch.Tensor, rotation: torch.Tensor | None = None,
                                         c: float = 5.0, min_scale: float = 1e-6) -> torch.Tensor:
    """sqrt(diag(R M R^T)), volume-normalised, with M the shaped metric
    (smaq/weighted_scalar.py:54-87).  Host computation in fp32."""
    dev = Sigma_q.device
    sig = Sigma_q.detach().to("cpu", torch.float32)
    evals, evecs = torch.linalg.eigh(sig)
    metric = evecs @ torch.diag(ssf_log(evals, c=c)) @ evecs.T
    if rotation is not None:
        if callable(rotation):
            rotation = rotation(torch.eye(sig.shape[0], dtype=torch.float32))
        rot = rotation.detach().to("cpu", torch.float32)
        metric = rot @ metric @ rot.T
    diag = metric.diagonal(dim1=-2, dim2=-1).clamp(min=min_scale)
    logs = torch.log(diag.sqrt())
    return torch.exp(logs - logs.mean()).to(dev)


def build_block_diagonal_metric_scales(Sigma_q: torch.Tensor, block_size: int = 2, c: float = 5.0,
                                       min_scale: float = 1e-6) -> torch.Tensor:
    """Per-coordinate scales for block-diagonal rotations, one metric per
    block (smaq/weighted_scalar.py:90-136)."""
    dev = Sigma_q.device
    sig = Sigma_q.detach().to("cpu", torch.float32)
    dim = sig.shape[0]
    n_blocks = dim // block_size
    parts = []
    for i in range(n_blocks):
        sl = slice(i * block_size, (i + 1) * block_size)
        evals, evecs = torch.linalg.eigh(sig[sl, sl])
        mb = evecs @ torch.diag(ssf_log(evals, c=c)) @ evecs.T
        logs = torch.log(mb.diagonal().clamp(min=min_scale).sqrt())
        parts.append(torch.exp(logs - logs.mean()))
    if dim % block_size:
        parts.append(torch.ones(dim - n_blocks * block_size, dtype=torch.float32))
    return torch.cat(parts).to(dev)


class RotationAdapter(torch.nn.Module):
    """Rotation-based scalar quantizer with per-dimension scaling
    (smaq/weighted_scalar.py:139-384)."""

    def __init__(
        self,
        dim: int,
        bits: int = 3,
        Sigma_q: torch.Tensor | None = None,
        rotation: torch.Tensor | None = None,
        coord_scales: torch.Tensor | None = None,
        c: float = 5.0,
        device: torch.device | None = None,
        dtype: torch.dtype = torch.float32,
        centroids: torch.Tensor | None = None,
        boundaries: torch.Tensor | None = None,
    ):
        super().__init__()
        self.dim = dim
        self.bits = bits
        self.device = torch.device(device) if device is not None else default_device()
        if rotation is None:
            rotation = torch.eye(dim, dtype=torch.float32)
        rotation = rotation.to(device=self.device, dtype=dtype)
        if coord_scales is None:
            if Sigma_q is None:
                Sigma_q = torch.eye(dim, dtype=torch.float32)
            coord_scales = build_rotated_diagonal_metric_scales(Sigma_q.to(torch.float32).cpu(),
                                                                rotation=rotation.to(torch.float32).cpu(), c=c)
        coord_scales = coord_scales.detach().to("cpu", dtype)
        inv_coord_scales = 1.0 / coord_scales.clamp(min=1e-6)  # host table, CPU rounding
        codebook, full = build_codebook(bits, self.device, dtype, centroids, boundaries)
        self.register_buffer("rotation", rotation)
        self.register_buffer("coord_scales", coord_scales.to(self.device))
        self.register_buffer("inv_coord_scales", inv_coord_scales.to(self.device))
        self.register_buffer("centroids", codebook)
        self.register_buffer("boundaries", full)
        self.register_buffer("decision_boundaries", full[1:-1].contiguous())
        self._c = c
        self._Sigma_q = Sigma_q
        self.tie_counter = None

    @classmethod
    def fit(cls, dim: int, bits: int, calibration_queries: torch.Tensor, calibration_keys: torch.Tensor,
            rotation: torch.Tensor | None = None, c_values: list[float] | None = None,
            use_rotation_values: list[bool] | None = None, device: torch.device | None = None,
            dtype: torch.dtype = torch.float32, centroids: torch.Tensor | None = None,
            boundaries: torch.Tensor | None = None):
        """Sweep c and rotation on/off, keep the lowest held-out logit MSE
        (smaq/weighted_scalar.py:228-340).  Each candidate encodes and decodes
        the validation keys with the GPU codec."""
        c_values = c_values or [0.5, 1.0, 2.0, 5.0, 10.0, 20.0, 50.0]
        use_rotation_values = use_rotation_values or [True, False]
        device = torch.device(device) if device is not None else default_device()
        n = calibration_queries.shape[0]
        mid = n // 2
        q_cal = calibration_queries[:mid]
        q_val, k_val = calibration_queries[mid:], calibration_keys[mid:]
        qc = q_cal.detach().to("cpu", torch.float32)
        sigma = (qc.T @ qc) / mid
        if rotation is None:
            rotation = torch.eye(dim, dtype=torch.float32)
        rotation = rotation.to(device=device, dtype=dtype)
        eye = torch.eye(dim, dtype=torch.float32, device=device)

        def logit_mse(q, k, k_hat):
            return (((q * (k - k_hat)).sum(dim=1)) ** 2).mean().item()

        best = (float("inf"), 5.0, True)
        results = []
        for use_rot in use_rotation_values:
            rot = rotation if use_rot else eye
            for c_val in c_values:
                ad = cls(dim=dim, bits=bits, Sigma_q=sigma, rotation=rot, c=c_val, device=device,
                         dtype=dtype, centroids=centroids, boundaries=boundaries)
                kv = k_val.to(device)
                k_hat = ad.dequantize(ad.quantize(kv))
                lm = logit_mse(q_val.to(device).float(), kv.float(), k_hat.float())
                results.append({"c": c_val, "use_rotation": use_rot, "lmse": lm})
                if lm < best[0]:
                    best = (lm, c_val, use_rot)
        best_lmse, best_c, best_rot = best
        adapter = cls(dim=dim, bits=bits, Sigma_q=sigma, rotation=rotation if best_rot else eye, c=best_c,
                      device=device, dtype=dtype, centroids=centroids, boundaries=boundaries)
        return adapter, {"best_c": best_c, "best_use_rotation": best_rot, "best_lmse": best_lmse,
                         "all_results": results}

    def rotate_query(self, query: torch.Tensor) -> torch.Tensor:
        """(q @ R^T) * (1 / s) in fp32 (smaq/weighted_scalar.py:342-345)."""
        return _native.rotate_rows(query, self.rotation.float().t().contiguous(), self.inv_coord_scales)

    def quantize(self, k: torch.Tensor) -> SMAQQuantized:
        """(smaq/weighted_scalar.py:347-355)"""
        codes, norms = _native.encode_scalar(k, self.rotation.float().t().contiguous(), self.decision_boundaries,
                                             self.bits, coord_scales=self.coord_scales, ties=self.tie_counter)
        return SMAQQuantized(indices=codes, norms=norms, bits=self.bits)

    def encode_into(self, k: torch.Tensor, codes: torch.Tensor, norms: torch.Tensor) -> None:
        """``quantize`` of k [lanes, T, dim] written into column views
        codes [lanes, T, P], norms [lanes, T] (append-only storage)."""
        _native.encode_scalar(k, self.rotation.float().t().contiguous(), self.decision_boundaries, self.bits,
                              coord_scales=self.coord_scales, ties=self.tie_counter, out=(codes, norms))

    def dequantize(self, q: SMAQQuantized) -> torch.Tensor:
        """(c[code] * (1/s)) @ R * norm (smaq/weighted_scalar.py:357-363)."""
        return _native.dequant_scalar(q.indices, q.norms, q.bits, self.dim, self.centroids,
                                      self.rotation.float().contiguous(), inv_scales=self.inv_coord_scales,
                                      out_dtype=self.rotation.dtype)

    def attention_score(self, query: torch.Tensor, quantized_key: SMAQQuantized,
                        scale: float | None = None) -> torch.Tensor:
        """(smaq/weighted_scalar.py:365-379)"""
        q_rot = self.rotate_query(query)
        return scores_from_codes(q_rot, quantized_key.indices, quantized_key.norms, quantized_key.bits,
                                 self.centroids, scale, query.dtype)

    def forward(self, k: torch.Tensor) -> torch.Tensor:
        return self.dequantize(self.quantize(k))


SMAQWeightedRotationQuantizer = RotationAdapter
