"""Calibration providers (drop-in for smaq/calibration.py:10-27).

A dictionary lookup of per-layer query covariance; the store asks it for
``Sigma_q`` when none is passed explicitly.
"""

from __future__ import annotations

from typing import Any, Mapping

from smaq_amd.core import CalibrationProvider


class IdentityCalibrationProvider(CalibrationProvider):
    """No explicit calibration: callers fall back to the identity metric."""

    def get_sigma_q(self, layer_idx: int, head_dim: int, device: Any | None = None) -> Any | None:
        return None


class StaticCalibrationProvider(CalibrationProvider):
    """Precomputed Sigma_q keyed by layer index or by ``"layer_{i}"``."""

    def __init__(self, per_layer: Mapping[Any, Any]):
        self.per_layer = dict(per_layer)

    def get_sigma_q(self, layer_idx: int, head_dim: int, device: Any | None = None) -> Any | None:
        if layer_idx in self.per_layer:
            return self.per_layer[layer_idx]
        return self.per_layer.get(f"layer_{layer_idx}")
