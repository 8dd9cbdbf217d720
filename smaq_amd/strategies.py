"""Concrete quantization strategies (drop-in for smaq/strategies.py).

The strategies are the boundary the kernels sit behind: a store calls
``quantize`` on append, and ``compute_hybrid_attention`` asks the strategy
for its ``fused_history`` description, which names the codec tables the
fused HIP attention kernel reads.  Strategies without one (the exact shadow
strategy, or user strategies) go through the generic per-head
``attention_score`` protocol instead.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, NamedTuple, Optional

import torch

from smaq_amd.block_vq import BlockVQQuantized, SMAQBlockVQ
from smaq_amd.core import CacheCapabilities, MetricStrategy, QuantizationStrategy
from smaq_amd.quantizer import SMAQQuantized, SMAQQuantizer, default_device
from smaq_amd.ssf import build_smaq_metric
from smaq_amd.weighted_scalar import RotationAdapter


class FusedHistory(NamedTuple):
    """What the fused attention kernel needs to score a strategy's keys.

    kind: "scalar" (packed codes + norms, scored with a rotated query) or
    "block_vq" (one uint8 index per block, scored through decoded centroids).
    The kernel dots the decoded key with q' = (q @ M^T) * s, where
    ``rot_t`` = M^T (None: M = I) and ``rot_scale`` = s (None: s = 1).
    """

    kind: str
    lut: torch.Tensor
    rot_t: Optional[torch.Tensor] = None
    rot_scale: Optional[torch.Tensor] = None
    bits: int = 0
    n_blocks: int = 0
    block_dim: int = 0
    n_centroids: int = 0


class IdentityMetricStrategy(MetricStrategy):
    name = "identity"

    def __init__(self, dim: int, device: torch.device | None = None):
        self.dim = dim
        self.device = torch.device(device) if device is not None else default_device()
        self.sigma_q = torch.eye(dim, dtype=torch.float32, device=self.device)

    def fit(self, calibration_queries: Any, calibration_keys: Any | None = None) -> "IdentityMetricStrategy":
        return self

    def export_state(self) -> dict[str, Any]:
        return {"Sigma_q": self.sigma_q}


class SMAQFullMetricStrategy(MetricStrategy):
    """Full shaped metric from Sigma_q (smaq/strategies.py:32-49)."""

    name = "smaq_full_metric"

    def __init__(self, dim: int, Sigma_q: torch.Tensor | None = None, device: torch.device | None = None):
        self.dim = dim
        self.device = torch.device(device) if device is not None else default_device()
        self.sigma_q = Sigma_q if Sigma_q is not None else torch.eye(dim, dtype=torch.float32, device=self.device)
        self.E, self.E_inv = build_smaq_metric(self.sigma_q.to(torch.float32), c=5.0)

    def fit(self, calibration_queries: Any, calibration_keys: Any | None = None) -> "SMAQFullMetricStrategy":
        q = calibration_queries.detach().to("cpu", torch.float32)
        centered = q - q.mean(dim=0, keepdim=True)
        self.sigma_q = ((centered.T @ centered) / max(1, centered.shape[0])).to(self.device)
        self.E, self.E_inv = build_smaq_metric(self.sigma_q.to(torch.float32), c=5.0)
        return self

    def export_state(self) -> dict[str, Any]:
        return {"Sigma_q": self.sigma_q, "E": self.E, "E_inv": self.E_inv}


class SMAQDiagonalMetricState(MetricStrategy):
    """Sigma_q holder for the diagonal metric (smaq/strategies.py:52-68)."""

    name = "smaq_diagonal_metric"

    def __init__(self, dim: int, Sigma_q: torch.Tensor | None = None, device: torch.device | None = None):
        self.dim = dim
        self.device = torch.device(device) if device is not None else default_device()
        self.sigma_q = Sigma_q if Sigma_q is not None else torch.eye(dim, dtype=torch.float32, device=self.device)

    def fit(self, calibration_queries: Any, calibration_keys: Any | None = None) -> "SMAQDiagonalMetricState":
        q = calibration_queries.detach().to("cpu", torch.float32)
        centered = q - q.mean(dim=0, keepdim=True)
        self.sigma_q = ((centered.T @ centered) / max(1, centered.shape[0])).to(self.device)
        return self

    def export_state(self) -> dict[str, Any]:
        return {"Sigma_q": self.sigma_q}


class ExactShadowQuantized(NamedTuple):
    values: torch.Tensor


@dataclass
class _StrategyMixin(QuantizationStrategy):
    """Strategies backed by a quantizer object (smaq/strategies.py:85-97)."""

    def flatten_quantized(self, quantized: Any) -> Any:
        raise NotImplementedError

    def concat_quantized(self, chunks: list[Any]) -> Any:
        raise NotImplementedError

    def select_head(self, quantized: Any, head_idx: int) -> Any:
        raise NotImplementedError

    def fused_history(self) -> Optional[FusedHistory]:
        return None


class IdentityScalarStrategy(_StrategyMixin):
    """Scalar codes with R = I, s = 1 (smaq/strategies.py:100-140)."""

    name = "identity_scalar"
    metric_name = "identity"
    quantization_name = "scalar"

    def __init__(self, dim: int, bits: int = 3, device: torch.device | None = None):
        self.quantizer = RotationAdapter(dim=dim, bits=bits, coord_scales=torch.ones(dim), device=device)
        self.bits = bits

    def quantize(self, keys: Any) -> Any:
        return self.quantizer.quantize(keys)

    def dequantize(self, quantized: Any) -> Any:
        return self.quantizer.dequantize(quantized)

    def attention_score(self, query: Any, quantized: Any, scale: float | None = None, **kwargs: Any) -> Any:
        return self.quantizer.attention_score(query, quantized, scale=scale)

    def flatten_quantized(self, quantized: SMAQQuantized) -> SMAQQuantized:
        ind = quantized.indices
        return SMAQQuantized(indices=ind.reshape(-1, ind.shape[-2], ind.shape[-1]).contiguous(),
                             norms=quantized.norms.reshape(-1, quantized.norms.shape[-1]).contiguous(),
                             bits=quantized.bits)

    def concat_quantized(self, chunks: list[SMAQQuantized]) -> SMAQQuantized:
        return SMAQQuantized(indices=torch.cat([c.indices for c in chunks], dim=-2),
                             norms=torch.cat([c.norms for c in chunks], dim=-1), bits=chunks[0].bits)

    def select_head(self, quantized: SMAQQuantized, head_idx: int) -> SMAQQuantized:
        return SMAQQuantized(indices=quantized.indices[head_idx], norms=quantized.norms[head_idx],
                             bits=quantized.bits)

    def memory_bytes(self, quantized: SMAQQuantized) -> int:
        return quantized.indices.nelement() + quantized.norms.nelement() * 2

    def fused_history(self) -> Optional[FusedHistory]:
        qz = self.quantizer
        if isinstance(qz, SMAQQuantizer):
            return FusedHistory("scalar", qz.centroids, rot_t=qz.E_inv.float().t().contiguous(), bits=qz.bits)
        if isinstance(qz, RotationAdapter):
            return FusedHistory("scalar", qz.centroids, rot_t=qz.rotation.float().t().contiguous(),
                                rot_scale=qz.inv_coord_scales.float().contiguous(), bits=qz.bits)
        return None


class SMAQFullMetricScalarStrategy(IdentityScalarStrategy):
    """Full SMAQ metric + scalar codes (smaq/strategies.py:143-168)."""

    name = "smaq_full_metric_scalar"
    metric_name = "smaq_full_metric"

    def __init__(self, dim: int, bits: int = 3, Sigma_q: torch.Tensor | None = None,
                 device: torch.device | None = None, dtype: torch.dtype = torch.float32):
        self.quantizer = SMAQQuantizer(dim=dim, bits=bits, Sigma_q=Sigma_q, device=device, dtype=dtype)
        self.bits = bits

    @property
    def supports_kernel(self) -> bool:
        return True

    def fit(self, calibration_queries: Any, calibration_keys: Any | None = None) -> "SMAQFullMetricScalarStrategy":
        self.quantizer.fit(calibration_queries)
        return self

    def attention_score(self, query: Any, quantized: Any, scale: float | None = None, **kwargs: Any) -> Any:
        return self.quantizer.attention_score(query, quantized, scale=scale,
                                              use_kernel=kwargs.get("use_kernel", False))


class SMAQDiagonalMetricStrategy(IdentityScalarStrategy):
    """Rotated diagonal metric + scalar codes (smaq/strategies.py:171-192)."""

    name = "smaq_diagonal_metric"
    metric_name = "smaq_diagonal_metric"

    def __init__(self, dim: int, bits: int = 3, Sigma_q: torch.Tensor | None = None,
                 rotation: torch.Tensor | None = None, device: torch.device | None = None,
                 dtype: torch.dtype = torch.float32):
        self.quantizer = RotationAdapter(dim=dim, bits=bits, Sigma_q=Sigma_q, rotation=rotation, device=device,
                                         dtype=dtype)
        self.bits = bits


class SMAQBlockVQStrategy(_StrategyMixin):
    """Block VQ keys (smaq/strategies.py:195-255)."""

    name = "smaq_block_vq"
    metric_name = "smaq_full_metric"
    quantization_name = "block_vq"

    def __init__(self, head_dim: int, block_dim: int = 8, n_centroids: int = 256, c: float = 5.0,
                 device: torch.device | None = None, dtype: torch.dtype = torch.float32):
        self.quantizer = SMAQBlockVQ(head_dim=head_dim, block_dim=block_dim, n_centroids=n_centroids, c=c,
                                     device=device, dtype=dtype)

    def fit(self, calibration_queries: Any, calibration_keys: Any | None = None) -> "SMAQBlockVQStrategy":
        if calibration_keys is None:
            calibration_keys = calibration_queries
        self.quantizer.fit(calibration_keys, calibration_queries)
        return self

    def quantize(self, keys: Any) -> Any:
        return self.quantizer.quantize(keys)

    def dequantize(self, quantized: Any) -> Any:
        return self.quantizer.dequantize(quantized)

    def attention_score(self, query: Any, quantized: Any, scale: float | None = None, **kwargs: Any) -> Any:
        return self.quantizer.attention_score(query, quantized, scale=scale)

    def flatten_quantized(self, quantized: BlockVQQuantized) -> BlockVQQuantized:
        ind = quantized.indices
        return BlockVQQuantized(indices=ind.reshape(-1, ind.shape[-2], ind.shape[-1]).contiguous(),
                                n_blocks=quantized.n_blocks, block_dim=quantized.block_dim)

    def concat_quantized(self, chunks: list[BlockVQQuantized]) -> BlockVQQuantized:
        return BlockVQQuantized(indices=torch.cat([c.indices for c in chunks], dim=-2),
                                n_blocks=chunks[0].n_blocks, block_dim=chunks[0].block_dim)

    def select_head(self, quantized: BlockVQQuantized, head_idx: int) -> BlockVQQuantized:
        return BlockVQQuantized(indices=quantized.indices[head_idx], n_blocks=quantized.n_blocks,
                                block_dim=quantized.block_dim)

    def memory_bytes(self, quantized: BlockVQQuantized) -> int:
        return quantized.indices.nelement() * quantized.indices.element_size()

    def fused_history(self) -> Optional[FusedHistory]:
        qz = self.quantizer
        return FusedHistory("block_vq", qz.decoded_centroids, n_blocks=qz.n_blocks, block_dim=qz.block_dim,
                            n_centroids=qz.n_centroids)


class ExactShadowStrategy(_StrategyMixin):
    """Uncompressed shadow copy of the keys (smaq/strategies.py:258-298).
    Not a codec: plain tensor copies and a library GEMM for scores."""

    name = "exact_shadow"
    metric_name = "identity"
    quantization_name = "shadow_exact"

    @property
    def capabilities(self) -> CacheCapabilities:
        return CacheCapabilities(strategy_name=self.name, metric_name=self.metric_name,
                                 quantization_name=self.quantization_name, compressed_history=False,
                                 compressed_history_shadow_only=True, values_compressed=False,
                                 decode_uses_compressed_keys=False, decode_uses_compressed_values=False)

    def quantize(self, keys: Any) -> Any:
        return ExactShadowQuantized(values=keys.detach().clone())

    def dequantize(self, quantized: Any) -> Any:
        return quantized.values

    def attention_score(self, query: Any, quantized: Any, scale: float | None = None, **kwargs: Any) -> Any:
        s = torch.matmul(query.float(), quantized.values.float().transpose(-2, -1))
        if scale is not None:
            s = s * scale
        return s.to(query.dtype)

    def flatten_quantized(self, quantized: ExactShadowQuantized) -> ExactShadowQuantized:
        v = quantized.values
        return ExactShadowQuantized(values=v.reshape(-1, v.shape[-2], v.shape[-1]).contiguous())

    def concat_quantized(self, chunks: list[ExactShadowQuantized]) -> ExactShadowQuantized:
        return ExactShadowQuantized(values=torch.cat([c.values for c in chunks], dim=-2))

    def select_head(self, quantized: ExactShadowQuantized, head_idx: int) -> ExactShadowQuantized:
        return ExactShadowQuantized(values=quantized.values[head_idx])

    def memory_bytes(self, quantized: ExactShadowQuantized) -> int:
        return quantized.values.nelement() * quantized.values.element_size()
