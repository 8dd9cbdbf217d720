"""Value codec and the standalone SMAQ KV cache (drop-in for smaq/kv_cache.py).

``quantize_values`` is the value bit-packer (HIP kernel): per group of
``group_size`` elements, asymmetric min/max quantisation to ``bits`` bits,
2-bit codes packed four per byte and 4-bit codes two per byte.
``dequantize_values`` is its HIP inverse.
"""

from __future__ import annotations

import math
from typing import Any, NamedTuple, Optional

import torch

from smaq_amd import _native
from smaq_amd.calibration import IdentityCalibrationProvider
from smaq_amd.core import CacheCapabilities, CalibrationProvider
from smaq_amd.quantizer import default_device
from smaq_amd.strategies import SMAQFullMetricScalarStrategy


class ValueQuantized(NamedTuple):
    """Bit-packed values (smaq/kv_cache.py:20-26)."""

    data: torch.Tensor
    scales: torch.Tensor
    zeros: torch.Tensor
    bits: int = 2


def unpack_values(vq: ValueQuantized) -> torch.Tensor:
    """Per-element uint8 codes from packed bytes (smaq/kv_cache.py:29-47)."""
    bits = vq.bits if len(vq) > 3 else 2
    p = vq.data
    if bits == 2:
        return torch.stack([p & 0x03, (p >> 2) & 0x03, (p >> 4) & 0x03, (p >> 6) & 0x03],
                           dim=-1).reshape(*p.shape[:-1], p.shape[-1] * 4)
    if bits == 4:
        return torch.stack([p & 0x0F, (p >> 4) & 0x0F], dim=-1).reshape(*p.shape[:-1], p.shape[-1] * 2)
    return p


def quantize_values(v: torch.Tensor, bits: int = 2, group_size: int = 32) -> ValueQuantized:
    """Groupwise asymmetric quantisation (smaq/kv_cache.py:50-91), HIP kernel."""
    data, scales, zeros = _native.pack_values(v, bits, group_size)
    return ValueQuantized(data=data, scales=scales, zeros=zeros, bits=bits)


def dequantize_values(vq: ValueQuantized, group_size: int = 32) -> torch.Tensor:
    """fp32 code * scale + zero (smaq/kv_cache.py:94-103), HIP kernel."""
    bits = vq.bits if len(vq) > 3 else 2
    return _native.dequant_values(vq.data, vq.scales, vq.zeros, bits, group_size)


def _cat_value_q(a: ValueQuantized, b: ValueQuantized, bits: int) -> ValueQuantized:
    return ValueQuantized(data=torch.cat([a.data, b.data], dim=-2),
                          scales=torch.cat([a.scales, b.scales], dim=-2),
                          zeros=torch.cat([a.zeros, b.zeros], dim=-2), bits=bits)


class SMAQKVCache:
    """Compressed history plus an exact recent buffer, layout [B, H, T, D]
    (smaq/kv_cache.py:106-290)."""

    def __init__(
        self,
        head_dim: int,
        Sigma_q: torch.Tensor | None = None,
        key_bits: int = 3,
        value_bits: int = 2,
        value_group_size: int = 32,
        buffer_size: int = 128,
        device: torch.device | None = None,
        dtype: torch.dtype = torch.float16,
        layer_idx: int = 0,
        key_strategy: Any | None = None,
        calibration_provider: CalibrationProvider | None = None,
    ):
        self.head_dim = head_dim
        self.key_bits = key_bits
        self.value_bits = value_bits
        self.value_group_size = value_group_size
        self.buffer_size = buffer_size
        self.device = torch.device(device) if device is not None else default_device()
        self.dtype = dtype
        self.layer_idx = layer_idx
        self.calibration_provider = calibration_provider or IdentityCalibrationProvider()
        sigma = Sigma_q
        if sigma is None:
            sigma = self.calibration_provider.get_sigma_q(layer_idx, head_dim, device=self.device)
        self.key_quantizer = key_strategy or SMAQFullMetricScalarStrategy(
            dim=head_dim, Sigma_q=sigma, bits=key_bits, device=self.device, dtype=torch.float32)
        self.seq_len = 0
        self.key_quantized: Optional[Any] = None
        self.value_quantized: Optional[ValueQuantized] = None
        self.key_buffer: Optional[torch.Tensor] = None
        self.value_buffer: Optional[torch.Tensor] = None

    @property
    def capabilities(self) -> CacheCapabilities:
        return self.key_quantizer.capabilities

    def prefill(self, keys: torch.Tensor, values: torch.Tensor):
        """Keep the last ``buffer_size`` tokens exact, compress the rest
        (smaq/kv_cache.py:154-174)."""
        seq_len = keys.shape[-2]
        self.seq_len = seq_len
        if seq_len <= self.buffer_size:
            self.key_buffer, self.value_buffer = keys, values
            return
        nq = seq_len - self.buffer_size
        self.key_buffer, self.value_buffer = keys[..., nq:, :], values[..., nq:, :]
        self.key_quantized = self.key_quantizer.quantize(keys[..., :nq, :])
        self.value_quantized = quantize_values(values[..., :nq, :], bits=self.value_bits,
                                               group_size=self.value_group_size)

    def append(self, key: torch.Tensor, value: torch.Tensor):
        """(smaq/kv_cache.py:176-188)"""
        self.seq_len += key.shape[-2]
        if self.key_buffer is not None:
            self.key_buffer = torch.cat([self.key_buffer, key], dim=-2)
            self.value_buffer = torch.cat([self.value_buffer, value], dim=-2)
        else:
            self.key_buffer, self.value_buffer = key, value
        if self.key_buffer.shape[-2] > self.buffer_size:
            self._flush_buffer()

    def _flush_buffer(self):
        """(smaq/kv_cache.py:190-216)"""
        nf = self.key_buffer.shape[-2] - self.buffer_size
        kf, vf = self.key_buffer[..., :nf, :], self.value_buffer[..., :nf, :]
        self.key_buffer, self.value_buffer = self.key_buffer[..., nf:, :], self.value_buffer[..., nf:, :]
        new_k = self.key_quantizer.quantize(kf)
        new_v = quantize_values(vf, bits=self.value_bits, group_size=self.value_group_size)
        if self.key_quantized is None:
            self.key_quantized, self.value_quantized = new_k, new_v
            return
        self.key_quantized = self.key_quantizer.concat_quantized([self.key_quantized, new_k])
        self.value_quantized = _cat_value_q(self.value_quantized, new_v, self.value_bits)

    def attention_scores(self, query: torch.Tensor, scale: float | None = None) -> torch.Tensor:
        """[compressed scores, exact scores] along the key axis, no softmax
        (smaq/kv_cache.py:218-241)."""
        if scale is None:
            scale = 1.0 / math.sqrt(self.head_dim)
        parts = []
        if self.key_quantized is not None:
            if getattr(self.key_quantizer, "supports_kernel", False):
                parts.append(self.key_quantizer.attention_score(query, self.key_quantized, scale=scale,
                                                                use_kernel=True))
            else:
                parts.append(self.key_quantizer.attention_score(query, self.key_quantized, scale=scale))
        if self.key_buffer is not None:
            # (a contiguous right operand: batched bf16 products of a transposed view are avoided)
            parts.append(torch.matmul(query, self.key_buffer.transpose(-2, -1).contiguous()) * scale)
        if not parts:
            return torch.empty(*query.shape[:-2], query.shape[-2], 0, device=query.device, dtype=query.dtype)
        return torch.cat(parts, dim=-1)

    def attend(self, attn_weights: torch.Tensor) -> torch.Tensor:
        """Weights over [compressed, exact] applied to the values
        (smaq/kv_cache.py:243-267)."""
        outs = []
        col = 0
        if self.value_quantized is not None:
            nq = self.value_quantized.data.shape[-2]
            v_hat = dequantize_values(self.value_quantized, self.value_group_size)
            outs.append(torch.matmul(attn_weights[..., col:col + nq], v_hat))
            col += nq
        if self.value_buffer is not None:
            nb = self.value_buffer.shape[-2]
            outs.append(torch.matmul(attn_weights[..., col:col + nb], self.value_buffer))
        if not outs:
            return torch.zeros(*attn_weights.shape[:-1], self.head_dim, device=attn_weights.device,
                               dtype=attn_weights.dtype)
        return sum(outs)

    def memory_bytes(self) -> dict[str, int]:
        """Byte accounting with 16-bit metadata (smaq/kv_cache.py:269-287)."""
        info = {"quantized_keys": 0, "quantized_values": 0, "buffer": 0, "total": 0}
        if self.key_quantized is not None:
            info["quantized_keys"] += self.key_quantizer.memory_bytes(self.key_quantized)
        if self.value_quantized is not None:
            vq = self.value_quantized
            info["quantized_values"] += vq.data.nelement() + vq.scales.nelement() * 2 + vq.zeros.nelement() * 2
        if self.key_buffer is not None:
            info["buffer"] += self.key_buffer.nelement() * 2
        if self.value_buffer is not None:
            info["buffer"] += self.value_buffer.nelement() * 2
        info["total"] = info["quantized_keys"] + info["quantized_values"] + info["buffer"]
        return info

    def get_seq_length(self) -> int:
        return self.seq_len
