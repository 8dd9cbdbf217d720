"""Backend-agnostic contracts of the SMAQ cache (drop-in for smaq/core.py).

The quantization strategy ABC is the seam the HIP kernels sit behind: stores
and attention call ``quantize`` / ``attention_score`` on a strategy, and the
GPU strategies in ``smaq_amd.strategies`` route those calls to
libsmaq_hip.so.  Names, fields and defaults follow smaq/core.py:19-173 so
user code written against the reference keeps working.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from dataclasses import dataclass
from typing import Any, Optional


@dataclass(frozen=True)
class CacheCapabilities:
    """What a cache/backend actually does at runtime (smaq/core.py:19-30)."""

    strategy_name: str
    metric_name: str
    quantization_name: str
    compressed_history: bool
    compressed_history_shadow_only: bool
    values_compressed: bool
    decode_uses_compressed_keys: bool
    decode_uses_compressed_values: bool


@dataclass(frozen=True)
class LayoutInfo:
    """Normalised view of a model's KV layout (smaq/core.py:33-41)."""

    adapter_name: str
    effective_head_dim: int
    observed_key_dim: int
    observed_value_dim: int
    unified_kv: bool = False


class CalibrationProvider(ABC):
    """Source of per-layer query covariance (smaq/core.py:44-54)."""

    @abstractmethod
    def get_sigma_q(self, layer_idx: int, head_dim: int, device: Any | None = None) -> Any | None:
        raise NotImplementedError


class MetricStrategy(ABC):
    """Query-aware transform plus its calibration state (smaq/core.py:57-68)."""

    name: str = "metric"

    @abstractmethod
    def fit(self, calibration_queries: Any, calibration_keys: Any | None = None) -> "MetricStrategy":
        raise NotImplementedError

    @abstractmethod
    def export_state(self) -> dict[str, Any]:
        raise NotImplementedError


class QuantizationStrategy(ABC):
    """Encode/decode layout and score-time reconstruction (smaq/core.py:71-124)."""

    name: str = "quantization"
    metric_name: str = "metric"
    quantization_name: str = "quantization"

    @property
    def capabilities(self) -> CacheCapabilities:
        return CacheCapabilities(
            strategy_name=self.name,
            metric_name=self.metric_name,
            quantization_name=self.quantization_name,
            compressed_history=True,
            compressed_history_shadow_only=False,
            values_compressed=True,
            decode_uses_compressed_keys=True,
            decode_uses_compressed_values=False,
        )

    def fit(self, calibration_queries: Any, calibration_keys: Any | None = None) -> "QuantizationStrategy":
        return self

    @property
    def supports_kernel(self) -> bool:
        return False

    @abstractmethod
    def quantize(self, keys: Any) -> Any:
        raise NotImplementedError

    @abstractmethod
    def dequantize(self, quantized: Any) -> Any:
        raise NotImplementedError

    @abstractmethod
    def attention_score(self, query: Any, quantized: Any, scale: float | None = None, **kwargs: Any) -> Any:
        raise NotImplementedError

    @abstractmethod
    def flatten_quantized(self, quantized: Any) -> Any:
        raise NotImplementedError

    @abstractmethod
    def concat_quantized(self, chunks: list[Any]) -> Any:
        raise NotImplementedError

    @abstractmethod
    def select_head(self, quantized: Any, head_idx: int) -> Any:
        raise NotImplementedError

    @abstractmethod
    def memory_bytes(self, quantized: Any) -> int:
        raise NotImplementedError


class AttentionBackend(ABC):
    """Scores/outputs over compressed history plus an exact tail (smaq/core.py:127-140)."""

    @abstractmethod
    def compute(self, query: Any, store: Any, recent_k: Any | None, recent_v: Any | None,
                num_query_heads: int, scale: Optional[float] = None) -> Any:
        raise NotImplementedError


class CacheBackend(ABC):
    """Owns prefill/decode append, flush and historical storage (smaq/core.py:143-149)."""

    @property
    @abstractmethod
    def capabilities(self) -> CacheCapabilities:
        raise NotImplementedError


class ModelLayoutAdapter(ABC):
    """Normalises KV layout differences across model families (smaq/core.py:152-173)."""

    name: str = "generic"

    def resolve_head_dim(self, model: Any, layer_idx: int) -> int:
        attn = getattr(model.layers[layer_idx], "self_attn", None)
        if attn is not None and hasattr(attn, "head_dim"):
            return int(attn.head_dim)
        if attn is not None and hasattr(attn, "hidden_size") and hasattr(attn, "num_heads"):
            return int(attn.hidden_size // attn.num_heads)
        return 128

    @abstractmethod
    def normalize_kv(self, keys: Any, values: Any, expected_head_dim: int | None = None) -> LayoutInfo:
        raise NotImplementedError
