"""Compressed KV store (drop-in for smaq/store.py).

History is exposed as a head-major ``FlatCache``: per KV head, key codes
[N, P], norms [N], value bytes [N, D/vpb], scales and zeros [N, D/group] --
the layout the fused attention kernel streams.  For the GPU codecs (scalar
SMAQ / rotation scalar / block-VQ keys) the fields are append-only columns
(``smaq_amd.columns.ColumnHistory``): an appended chunk is encoded by the HIP
kernels straight into the columns' next rows and ``get_flat_cache`` returns
views of the filled rows, so an append costs the encode of that chunk only.
(The reference quantises each chunk into its own tensors and concatenates
all of them on the first read after every append, smaq/store.py:83-114.)
Other strategies keep the reference's list of quantised chunks.
"""

from __future__ import annotations

from typing import Any, NamedTuple, Optional, Sequence

import torch

from smaq_amd.calibration import IdentityCalibrationProvider
from smaq_amd.columns import ColumnHistory, codec_kind
from smaq_amd.core import CacheCapabilities, CalibrationProvider
from smaq_amd.quantizer import default_device
from smaq_amd.strategies import SMAQFullMetricScalarStrategy
from smaq_amd.value_codec import ValueQuantized, quantize_values


class FlatCache(NamedTuple):
    """Flattened view for fast read access (smaq/store.py:20-25)."""

    key_q: Any
    value_q: ValueQuantized
    num_tokens: int


class CompressedKVStore:
    """Chunked SMAQ KV store (smaq/store.py:28-130)."""

    def __init__(
        self,
        head_dim: int,
        num_kv_heads: int,
        Sigma_q: torch.Tensor | None = None,
        key_bits: int = 3,
        value_bits: int = 2,
        value_group_size: int = 32,
        device: torch.device | None = None,
        layer_idx: int = 0,
        key_strategy: Any | None = None,
        calibration_provider: CalibrationProvider | None = None,
    ):
        self.head_dim = head_dim
        self.num_kv_heads = num_kv_heads
        self.key_bits = key_bits
        self.value_bits = value_bits
        self.value_group_size = min(value_group_size, head_dim)
        self.device = torch.device(device) if device is not None else default_device()
        self.layer_idx = layer_idx
        self.calibration_provider = calibration_provider or IdentityCalibrationProvider()
        if key_strategy is None:
            sigma = Sigma_q if Sigma_q is not None else self.calibration_provider.get_sigma_q(
                layer_idx, head_dim, device=self.device)
            key_strategy = SMAQFullMetricScalarStrategy(dim=head_dim, Sigma_q=sigma, bits=key_bits,
                                                        device=self.device, dtype=torch.float32)
        self.key_strategy = key_strategy
        self.quantizer = self.key_strategy
        self._lengths: list[int] = []
        self._hist: Optional[ColumnHistory] = None
        self._chunks: list[tuple[Any, ValueQuantized]] = []
        self._mem_bytes = 0
        self._flat: Optional[FlatCache] = None
        self._fused_plan = None   # compute_hybrid_attention's kept launch (key, plan)

    @property
    def capabilities(self) -> CacheCapabilities:
        return self.key_strategy.capabilities

    @property
    def num_tokens(self) -> int:
        return sum(self._lengths)

    @property
    def num_chunks(self) -> int:
        return len(self._lengths)

    def append_chunk(self, key: torch.Tensor, value: torch.Tensor):
        """Quantise and append a [T, Hkv, D] chunk (smaq/store.py:83-95)."""
        self.append_parts([(key, value)])

    def append_parts(self, parts: Sequence[tuple[torch.Tensor, torch.Tensor]]):
        """Append one chunk given as consecutive [T_i, Hkv, D] pieces -- a ring
        flush hands over the ring's exact tokens followed by the new ones
        without joining them first.  Same result as ``append_chunk`` of their
        concatenation."""
        T = sum(k.shape[0] for k, _ in parts)
        if self._hist is None and not self._chunks and codec_kind(self.key_strategy) is not None:
            self._hist = ColumnHistory(self.key_strategy, self.num_kv_heads, self.head_dim, self.value_bits,
                                       self.value_group_size, self.device)
        if self._hist is not None:
            # [T, Hkv, D] -> [Hkv, T, D] views: every head is one lane of rows
            self._mem_bytes += self._hist.append([(k.transpose(0, 1), v.transpose(0, 1)) for k, v in parts])
        else:
            key = parts[0][0] if len(parts) == 1 else torch.cat([k for k, _ in parts])
            value = parts[0][1] if len(parts) == 1 else torch.cat([v for _, v in parts])
            k = key.transpose(0, 1).unsqueeze(0)
            v = value.transpose(0, 1).unsqueeze(0)
            key_q = self.key_strategy.quantize(k)
            val_q = quantize_values(v, bits=self.value_bits, group_size=self.value_group_size)
            self._chunks.append((key_q, val_q))
            self._mem_bytes += self.key_strategy.memory_bytes(key_q) + _value_bytes(val_q)
        self._lengths.append(T)
        self._flat = None

    def get_flat_cache(self) -> Optional[FlatCache]:
        """Head-major flattened history (smaq/store.py:97-114)."""
        if not self._lengths:
            return None
        if self._flat is not None:
            return self._flat
        if self._hist is not None:
            if self._hist.n == 0:
                return None
            key_q, vq = self._hist.key_quantized(), self._hist.value_quantized()
        else:
            s = self.key_strategy
            flat = [(s.flatten_quantized(k), _flatten_value_q(v)) for k, v in self._chunks]
            if len(flat) == 1:
                key_q, vq = flat[0]
            else:
                key_q = s.concat_quantized([k for k, _ in flat])
                vq = _concat_value_q([v for _, v in flat])
        self._flat = FlatCache(key_q=key_q, value_q=vq, num_tokens=self.num_tokens)
        return self._flat

    def memory_bytes(self) -> int:
        """Key strategy bytes plus value bytes with 16-bit metadata, summed over
        the appended chunks (smaq/store.py:116-124)."""
        return self._mem_bytes

    def allocated_bytes(self) -> int:
        """Device bytes the compressed history actually holds (not in the
        reference): the column buffers at their capacity (up to twice
        ``memory_bytes`` after a doubling), or the quantised chunks' tensors
        for strategies without a column encoder."""
        if self._hist is not None:
            return self._hist.allocated_bytes()
        total = 0
        for k, v in self._chunks:
            for t in (*_tensors_of(k), v.data, v.scales, v.zeros):
                total += t.nelement() * t.element_size()
        return total

    def reset(self):
        self._lengths.clear()
        self._hist = None
        self._chunks.clear()
        self._mem_bytes = 0
        self._flat = None
        self._fused_plan = None   # compute_hybrid_attention's kept launch


def _tensors_of(q) -> list:
    """The tensors of a quantised key chunk (any strategy's NamedTuple)."""
    return [t for t in (q if isinstance(q, tuple) else ()) if isinstance(t, torch.Tensor)]


def _value_bytes(vq: ValueQuantized) -> int:
    """Value bytes of a chunk, metadata counted at 2 bytes (smaq/store.py:120-123)."""
    return vq.data.nelement() + vq.scales.nelement() * 2 + vq.zeros.nelement() * 2


def _flatten_value_q(value_q: ValueQuantized) -> ValueQuantized:
    """(1, H, T, ...) -> (H, T, ...) (smaq/store.py:133-141)."""
    bits = value_q.bits if len(value_q) > 3 else 2
    return ValueQuantized(*(t.reshape(-1, *t.shape[-2:]).contiguous() for t in value_q[:3]), bits=bits)


def _concat_value_q(chunks: list[ValueQuantized]) -> ValueQuantized:
    """Token-dim concatenation (smaq/store.py:144-152)."""
    bits = chunks[0].bits if len(chunks[0]) > 3 else 2
    return ValueQuantized(*(torch.cat([c[i] for c in chunks], dim=-2) for i in range(3)), bits=bits)
