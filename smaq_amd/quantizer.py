"""SMAQ scalar key quantizer (drop-in for smaq/quantizer.py).

Keys are normalised, mapped by the calibrated metric ``E``, quantised per
coordinate against Gaussian-quantile boundaries and bit-packed; scores are
computed straight from the packed codes.  Table construction and ``fit`` run
on the host (they produce kernel inputs); ``quantize``, ``dequantize``,
``rotate_query`` and ``attention_score`` are HIP kernels in libsmaq_hip.so.
"""

from __future__ import annotations

import math
from typing import NamedTuple

import torch
import torch.nn.functional as F

from smaq_amd import _native
from smaq_amd.ssf import build_smaq_metric


def default_device() -> torch.device:
    return torch.device("cuda" if torch.cuda.is_available() else "cpu")


class SMAQQuantized(NamedTuple):
    """Bit-packed SMAQ key representation (smaq/quantizer.py:26-31)."""

    indices: torch.Tensor
    norms: torch.Tensor
    bits: int


def _pack_indices(indices: torch.Tensor, bits: int) -> torch.Tensor:
    """Pack codes max(1, 8 // bits) per byte, first code in the low bits, last
    dim zero-padded (format of smaq/quantizer.py:34-46).  Plain tensor bit ops,
    kept for callers of the reference helper; the encoders pack in-kernel."""
    vpb = max(1, 8 // bits)
    lead, d = indices.shape[:-1], indices.shape[-1]
    padded = ((d + vpb - 1) // vpb) * vpb
    codes = indices.to(torch.uint8)
    if padded > d:
        codes = F.pad(codes, (0, padded - d), value=0)
    codes = codes.reshape(*lead, -1, vpb)
    shifts = torch.arange(vpb, device=indices.device, dtype=torch.uint8) * bits
    return (codes << shifts).sum(dim=-1, dtype=torch.uint8)


def _unpack_indices(packed: torch.Tensor, bits: int, d: int) -> torch.Tensor:
    """Inverse of ``_pack_indices`` (smaq/quantizer.py:49-55), int64 codes."""
    vpb = max(1, 8 // bits)
    shifts = torch.arange(vpb, device=packed.device, dtype=torch.uint8) * bits
    out = ((packed.unsqueeze(-1) >> shifts) & ((1 << bits) - 1)).reshape(*packed.shape[:-1], -1)
    return out[..., :d].long()


def _normal_ppf(probs: torch.Tensor) -> torch.Tensor:
    """Inverse standard normal CDF via erfinv (smaq/quantizer.py:58-60)."""
    return math.sqrt(2.0) * torch.erfinv((2.0 * probs) - 1.0)


def gaussian_codebook(bits: int, dtype: torch.dtype = torch.float32):
    """Centroids c_j = ppf(j / (2^b + 1)), j = 1..2^b, and boundaries
    ppf(clamp(j / 2^b, 1e-6, 1 - 1e-6)) with +-inf ends (smaq/quantizer.py:96-119).
    Built on the CPU so every device gets identical tables."""
    probs = torch.linspace(0.0, 1.0, (2 ** bits) + 2, dtype=torch.float32)[1:-1]
    centroids = _normal_ppf(probs).to(dtype)
    bp = torch.linspace(0.0, 1.0, (2 ** bits) + 1, dtype=torch.float32)
    boundaries = _normal_ppf(bp.clamp(1e-6, 1.0 - 1e-6)).to(dtype)
    boundaries[0] = -float("inf")
    boundaries[-1] = float("inf")
    return centroids, boundaries


def scores_from_codes(query_rot: torch.Tensor, indices: torch.Tensor, norms: torch.Tensor, bits: int,
                      centroids: torch.Tensor, scale, out_dtype) -> torch.Tensor:
    """((query_rot . c[code]) * norm) [* scale] for query (..., n_q, D) against
    packed keys (..., n_k, P) with matmul-style broadcasting of batch dims."""
    qb, kb = query_rot.shape[:-2], indices.shape[:-2]
    nq, D = query_rot.shape[-2:]
    nk, P = indices.shape[-2:]
    batch = torch.broadcast_shapes(qb, kb)
    q = query_rot.expand(*batch, nq, D).reshape(-1, nq, D)
    codes = indices.expand(*batch, nk, P).reshape(-1, nk, P)
    nrm = norms.expand(*batch, nk).reshape(-1, nk)
    out = _native.scores_scalar(q.to(torch.float32), codes, nrm, bits, centroids, scale, out_dtype)
    return out.reshape(*batch, nq, nk)


class SMAQQuantizer(torch.nn.Module):
    """Spectral metric-aware scalar quantizer (smaq/quantizer.py:63-188).

    Buffers ``E``, ``E_inv``, ``centroids``, ``boundaries`` and
    ``decision_boundaries`` keep the reference's names, so ``state_dict``
    round-trips.  Set ``tie_counter`` to an ``_native.TieCounter`` to count
    coordinates that land within 1e-6 of a decision boundary.
    """

    def __init__(
        self,
        dim: int,
        Sigma_q: torch.Tensor | None = None,
        bits: int = 3,
        device: torch.device | None = None,
        dtype: torch.dtype = torch.float32,
        E: torch.Tensor | None = None,
        E_inv: torch.Tensor | None = None,
    ):
        super().__init__()
        self.dim = dim
        self.bits = bits
        self.device = torch.device(device) if device is not None else default_device()
        if E is None or E_inv is None:
            if Sigma_q is None:
                Sigma_q = torch.eye(dim, dtype=torch.float32)
            E, E_inv = build_smaq_metric(Sigma_q.to(torch.float32), c=5.0)
        self.register_buffer("E", E.to(self.device, dtype=dtype))
        self.register_buffer("E_inv", E_inv.to(self.device, dtype=dtype))
        centroids, boundaries = gaussian_codebook(bits, dtype)
        self.register_buffer("centroids", centroids.to(self.device))
        self.register_buffer("boundaries", boundaries.to(self.device))
        self.register_buffer("decision_boundaries", boundaries[1:-1].contiguous().to(self.device))
        self.tie_counter = None

    def fit(self, calibration_queries: torch.Tensor) -> "SMAQQuantizer":
        """Refit E from the centred query covariance (smaq/quantizer.py:121-129);
        host-side, in fp32 on the CPU."""
        q = calibration_queries.detach().to("cpu", torch.float32)
        centered = q - q.mean(dim=0, keepdim=True)
        sigma = (centered.T @ centered) / max(1, centered.shape[0])
        E, E_inv = build_smaq_metric(sigma, c=5.0)
        self.E.copy_(E.to(self.E.device, dtype=self.E.dtype))
        self.E_inv.copy_(E_inv.to(self.E_inv.device, dtype=self.E_inv.dtype))
        return self

    def rotate_query(self, query: torch.Tensor) -> torch.Tensor:
        """q @ E_inv^T in fp32 (smaq/quantizer.py:131-136)."""
        return _native.rotate_rows(query, self.E_inv.float().t().contiguous())

    def quantize(self, k: torch.Tensor) -> SMAQQuantized:
        """Compress keys (..., dim) (smaq/quantizer.py:138-145)."""
        codes, norms = _native.encode_scalar(k, self.E.float().t().contiguous(), self.decision_boundaries,
                                             self.bits, ties=self.tie_counter)
        return SMAQQuantized(indices=codes, norms=norms, bits=self.bits)

    def encode_into(self, k: torch.Tensor, codes: torch.Tensor, norms: torch.Tensor) -> None:
        """``quantize`` of k [lanes, T, dim] written into column views
        codes [lanes, T, P], norms [lanes, T] (append-only storage)."""
        _native.encode_scalar(k, self.E.float().t().contiguous(), self.decision_boundaries, self.bits,
                              ties=self.tie_counter, out=(codes, norms))

    def dequantize(self, q: SMAQQuantized) -> torch.Tensor:
        """((c[code] @ E_inv^T) * norm) as E.dtype (smaq/quantizer.py:147-152)."""
        return _native.dequant_scalar(q.indices, q.norms, q.bits, self.dim, self.centroids,
                                      self.E_inv.float().t().contiguous(), out_dtype=self.E.dtype)

    def attention_score(
        self,
        query: torch.Tensor,
        quantized_key: SMAQQuantized,
        scale: float | None = None,
        use_kernel: bool = False,
    ) -> torch.Tensor:
        """<query, key_hat> * scale from packed keys (smaq/quantizer.py:154-184).

        ``use_kernel`` is accepted for signature parity; both settings run the
        same HIP score kernel."""
        del use_kernel
        q_rot = self.rotate_query(query)
        return scores_from_codes(q_rot, quantized_key.indices, quantized_key.norms, quantized_key.bits,
                                 self.centroids, scale, query.dtype)

    def forward(self, k: torch.Tensor) -> torch.Tensor:
        return self.dequantize(self.quantize(k))
