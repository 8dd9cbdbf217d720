"""SMAQ block vector quantizer (drop-in for smaq/block_vq.py).

Keys are cut into ``block_dim``-dim blocks; each block is mapped by its own
metric ``E_b`` and replaced by the index of the nearest of ``n_centroids``
codewords; decoding is a table lookup of pre-decoded centroids.  Calibration
(``fit``: per-block metric + k-means++/Lloyd) runs on the host CPU with torch
(the reference's codebook for a seed), or with ``on_device=True`` on the GPU
through HIP kernels; ``quantize`` and ``dequantize`` are HIP kernels.

Indices are stored as uint8 (n_centroids <= 256) rather than the reference's
int64: the values are identical (decoders call ``.long()``), the cache is 8x
smaller, and ``memory_bytes`` reports the true 1 byte per index.
"""

from __future__ import annotations

import math
from typing import NamedTuple, Optional

import torch
import torch.nn as nn

from smaq_amd import _native
from smaq_amd.quantizer import default_device
from smaq_amd.ssf import build_smaq_metric


class BlockVQQuantized(NamedTuple):
    """Block-VQ indices (..., n_blocks) (smaq/block_vq.py:25-30)."""

    indices: torch.Tensor
    n_blocks: int
    block_dim: int


def _kmeans(data: torch.Tensor, n_centroids: int, n_iters: int = 20, seed: int = 42) -> torch.Tensor:
    """k-means++ seeding then Lloyd iterations with empty clusters kept
    (smaq/block_vq.py:37-79).  Host calibration on the CPU: the seeded
    generator's draws (one randint, then one multinomial per centroid) fix the
    codebook, so it matches the reference's CPU run for the same seed."""
    data = data.detach().to("cpu", torch.float32)
    n, d = data.shape
    gen = torch.Generator().manual_seed(seed)
    if n <= n_centroids:
        out = torch.zeros((n_centroids, d), dtype=data.dtype)
        out[:n] = data
        return out
    picks = [torch.randint(n, (1,), generator=gen).item()]
    for _ in range(n_centroids - 1):
        # full cdist against every pick, as the reference: MKL takes a different
        # summation path for a single column, so an incremental minimum would
        # not reproduce its distances bit for bit
        w = torch.cdist(data, data[picks]).min(dim=1).values.square()
        tot = w.sum()
        w = w / tot if tot > 0 else torch.full((n,), 1.0 / n, dtype=data.dtype)
        picks.append(torch.multinomial(w, 1, generator=gen).item())
    cents = data[picks].clone()
    ones = torch.ones(n)
    for _ in range(n_iters):
        assign = torch.cdist(data, cents).argmin(dim=1)
        acc = torch.zeros_like(cents)
        cnt = torch.zeros(n_centroids)
        acc.index_add_(0, assign, data)
        cnt.index_add_(0, assign, ones)
        live = cnt > 0
        acc[live] /= cnt[live].unsqueeze(1)
        acc[~live] = cents[~live]
        cents = acc
    return cents


class SMAQBlockVQ(nn.Module):
    """Block vector quantizer of the SMAQ paper (smaq/block_vq.py:86-315)."""

    def __init__(self, head_dim: int, block_dim: int = 8, n_centroids: int = 256, c: float = 5.0,
                 device: Optional[torch.device] = None, dtype: torch.dtype = torch.float32):
        super().__init__()
        if head_dim % block_dim != 0:
            raise ValueError(f"head_dim={head_dim} must be divisible by block_dim={block_dim}")
        if n_centroids > 256:
            raise ValueError("n_centroids must be <= 256 (uint8 indices)")
        self.head_dim = head_dim
        self.block_dim = block_dim
        self.n_blocks = head_dim // block_dim
        self.n_centroids = n_centroids
        self.c = c
        self._device = torch.device(device) if device is not None else default_device()
        self._dtype = dtype
        eye = torch.eye(block_dim, dtype=dtype)
        self.register_buffer("E_blocks", eye.expand(self.n_blocks, -1, -1).clone().to(self._device))
        self.register_buffer("E_inv_blocks", eye.expand(self.n_blocks, -1, -1).clone().to(self._device))
        self.register_buffer("centroids", torch.zeros(self.n_blocks, n_centroids, block_dim, dtype=dtype,
                                                      device=self._device))
        self.register_buffer("decoded_centroids", torch.zeros(self.n_blocks, n_centroids, block_dim,
                                                              dtype=dtype, device=self._device))
        self._fitted = False
        self.tie_counter = None

    @property
    def bits_per_dim(self) -> float:
        return math.log2(self.n_centroids) / self.block_dim

    def fit(self, calibration_keys: torch.Tensor, calibration_queries: torch.Tensor, kmeans_iters: int = 20,
            seed: int = 42, on_device: bool = False) -> "SMAQBlockVQ":
        """Per block: uncentred Sigma_q, metric, k-means in the shaped space,
        pre-decoded centroids (smaq/block_vq.py:160-210).

        Host CPU, fp32, by default: the codebook is the reference's for the
        same seed.  ``on_device=True`` (an extension) runs the k-means on the
        quantizer's GPU with the HIP kernels (all blocks at once, incremental
        k-means++ distances, the encoder as the assignment step); the device
        random stream differs from the CPU one, so that codebook is a
        different draw of the same algorithm (compare with ``logit_mse``)."""
        queries = calibration_queries.detach().to("cpu")
        n = queries.shape[0]
        metrics = []
        for bi in range(self.n_blocks):
            sl = slice(bi * self.block_dim, (bi + 1) * self.block_dim)
            qb = queries[:, sl].float()
            metrics.append(build_smaq_metric((qb.T @ qb) / n, c=self.c))
        if on_device:
            return self._fit_on_device(calibration_keys, metrics, kmeans_iters, seed)
        keys = calibration_keys.detach().to("cpu")
        Es, Eis, Cs, Ds = [], [], [], []
        for bi in range(self.n_blocks):
            sl = slice(bi * self.block_dim, (bi + 1) * self.block_dim)
            E, E_inv = metrics[bi]
            cents = _kmeans(keys[:, sl].float() @ E.T, self.n_centroids, kmeans_iters, seed + bi)
            Es.append(E)
            Eis.append(E_inv)
            Cs.append(cents)
            Ds.append(cents @ E_inv.T)
        self.E_blocks = torch.stack(Es).to(self._device, self._dtype)
        self.E_inv_blocks = torch.stack(Eis).to(self._device, self._dtype)
        self.centroids = torch.stack(Cs).to(self._device, self._dtype)
        self.decoded_centroids = torch.stack(Ds).to(self._device, self._dtype)
        self._fitted = True
        return self

    def _fit_on_device(self, calibration_keys, metrics, kmeans_iters: int, seed: int) -> "SMAQBlockVQ":
        dev = self._device
        keys = calibration_keys.detach().to(dev)
        if keys.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            keys = keys.float()
        keys = keys.contiguous()
        n, nb, bd, nc = keys.shape[0], self.n_blocks, self.block_dim, self.n_centroids
        E_blocks = torch.stack([m[0] for m in metrics]).to(dev, torch.float32)
        E_inv_blocks = torch.stack([m[1] for m in metrics]).to(dev, torch.float32)
        x = _native.blockvq_shape(keys, E_blocks)                   # [nb, n, bd]
        if n <= nc:
            cents = torch.zeros(nb, nc, bd, dtype=torch.float32, device=dev)
            cents[:, :n] = x
        else:
            gen = torch.Generator(device=dev).manual_seed(seed)
            pick = torch.randint(n, (nb,), generator=gen, device=dev)
            picks = [pick]
            dmin = torch.empty(nb, n, dtype=torch.float32, device=dev)
            _native.kmeanspp_update(x, pick, dmin, first=True)
            for _ in range(nc - 1):
                # draw with probability proportional to the squared distance to
                # the nearest pick; a block whose points all coincide with
                # picks draws uniformly (smaq/block_vq.py:56-61)
                w = torch.where(dmin.sum(dim=1, keepdim=True) > 0, dmin, torch.ones_like(dmin))
                pick = torch.multinomial(w, 1, generator=gen).squeeze(1)
                picks.append(pick)
                _native.kmeanspp_update(x, pick, dmin, first=False)
            sel = torch.stack(picks, dim=1)                          # [nb, nc]
            cents = torch.gather(x, 1, sel.unsqueeze(-1).expand(nb, nc, bd)).contiguous()
            for _ in range(kmeans_iters):
                idx = _native.encode_blockvq(keys, E_blocks, cents)   # [n, nb]
                _native.kmeans_update(x, idx, cents)
        self.E_blocks = E_blocks.to(self._dtype)
        self.E_inv_blocks = E_inv_blocks.to(self._dtype)
        self.centroids = cents.to(self._dtype)
        self.decoded_centroids = torch.bmm(cents, E_inv_blocks.transpose(1, 2).contiguous()).to(self._dtype)
        self._fitted = True
        return self

    def quantize(self, k: torch.Tensor) -> BlockVQQuantized:
        """Nearest codeword per block (smaq/block_vq.py:216-244)."""
        idx = _native.encode_blockvq(k, self.E_blocks, self.centroids, ties=self.tie_counter)
        return BlockVQQuantized(indices=idx, n_blocks=self.n_blocks, block_dim=self.block_dim)

    def encode_into(self, k: torch.Tensor, idx: torch.Tensor) -> None:
        """``quantize`` of k [lanes, T, head_dim] written into the index
        column view idx [lanes, T, n_blocks] (append-only storage)."""
        _native.encode_blockvq(k, self.E_blocks, self.centroids, ties=self.tie_counter, out=idx)

    def dequantize(self, q: BlockVQQuantized) -> torch.Tensor:
        """Pre-decoded centroid lookup (smaq/block_vq.py:246-267)."""
        return _native.dequant_blockvq(q.indices, self.decoded_centroids)

    def attention_score(self, query: torch.Tensor, quantized_key: BlockVQQuantized,
                        scale: Optional[float] = None) -> torch.Tensor:
        """q . k_hat [* scale] (smaq/block_vq.py:273-297): decoded keys from the
        LUT kernel, then a library GEMM."""
        k_hat = self.dequantize(quantized_key)
        scores = torch.matmul(query.float(), k_hat.float().transpose(-2, -1))
        if scale is not None:
            scores = scores * scale
        return scores.to(query.dtype)

    def logit_mse(self, queries: torch.Tensor, keys: torch.Tensor) -> float:
        """E[(q . (k - k_hat))^2] (smaq/block_vq.py:303-311)."""
        k_hat = self.dequantize(self.quantize(keys))
        delta = keys.float() - k_hat.float()
        return (queries.float() * delta).sum(dim=-1).square().mean().item()

    def forward(self, k: torch.Tensor) -> torch.Tensor:
        return self.dequantize(self.quantize(k))
