"""Model-layout adapters (drop-in for smaq/layout.py).

They report how a model family's observed K/V widths relate to the head_dim a
cache was configured for; the quantised path itself only sees [.., D] rows.
"""

from __future__ import annotations

from typing import Any

from smaq_amd.core import LayoutInfo, ModelLayoutAdapter


class GenericModelLayoutAdapter(ModelLayoutAdapter):
    """The observed key width is the effective head dim; a width other than
    the expected one marks a unified KV layout (smaq/layout.py:10-26)."""

    name = "generic"

    def normalize_kv(self, keys: Any, values: Any, expected_head_dim: int | None = None) -> LayoutInfo:
        kd, vd = int(keys.shape[-1]), int(values.shape[-1])
        return LayoutInfo(adapter_name=self.name, effective_head_dim=kd, observed_key_dim=kd, observed_value_dim=vd,
                          unified_kv=expected_head_dim is not None and kd != expected_head_dim)


class QwenModelLayoutAdapter(GenericModelLayoutAdapter):
    """Standard K/V shapes under the Qwen name (smaq/layout.py:29-32)."""

    name = "qwen"


class GemmaModelLayoutAdapter(GenericModelLayoutAdapter):
    """Gemma: widened or unified K/V widths are accepted as observed
    (smaq/layout.py:35-48)."""

    name = "gemma"


def infer_model_layout_adapter(model: Any) -> ModelLayoutAdapter:
    """Pick an adapter from the model's class and module names
    (smaq/layout.py:51-60)."""
    joined = f"{type(model).__module__.lower()} {type(model).__name__.lower()}"
    if "gemma" in joined:
        return GemmaModelLayoutAdapter()
    if "qwen" in joined:
        return QwenModelLayoutAdapter()
    return GenericModelLayoutAdapter()
