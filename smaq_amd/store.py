"""Compressed KV store (drop-in for smaq/store.py).

History is quantised chunk by chunk on append (key strategy + value packer,
both HIP kernels) and exposed as a head-major ``FlatCache``: per KV head,
key codes [N, P], norms [N], value bytes [N, D/vpb], scales and zeros
[N, D/group] -- the layout the fused attention kernel streams.

Appends write into preallocated, geometrically grown GPU buffers, so a new
chunk costs a copy of that chunk only (the reference re-concatenates the
whole history on the first read after every append, smaq/store.py:97-114).
"""

from __future__ import annotations

from typing import Any, NamedTuple, Optional

import torch

from smaq_amd.calibration import IdentityCalibrationProvider
from smaq_amd.core import CacheCapabilities, CalibrationProvider
from smaq_amd.kv_cache import ValueQuantized, quantize_values
from smaq_amd.quantizer import default_device
from smaq_amd.strategies import SMAQFullMetricScalarStrategy


class FlatCache(NamedTuple):
    """Flattened view for fast read access (smaq/store.py:20-25)."""

    key_q: Any
    value_q: ValueQuantized
    num_tokens: int


class _Column:
    """One per-token tensor field stored [Hkv, capacity, *tail], grown x2."""

    def __init__(self):
        self.buf: Optional[torch.Tensor] = None

    def append(self, chunk: torch.Tensor, n_old: int) -> None:
        # chunk [Hkv, T, *tail]
        n_new = n_old + chunk.shape[1]
        if self.buf is None or self.buf.shape[1] < n_new:
            cap = max(n_new, 2 * (0 if self.buf is None else self.buf.shape[1]), 256)
            grown = torch.empty((chunk.shape[0], cap, *chunk.shape[2:]), dtype=chunk.dtype, device=chunk.device)
            if self.buf is not None and n_old:
                grown[:, :n_old].copy_(self.buf[:, :n_old])
            self.buf = grown
        self.buf[:, n_old:n_new].copy_(chunk)

    def view(self, n: int) -> torch.Tensor:
        return self.buf[:, :n]


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
        sigma = Sigma_q
        if sigma is None:
            sigma = self.calibration_provider.get_sigma_q(layer_idx, head_dim, device=self.device)
        self.key_strategy = key_strategy or SMAQFullMetricScalarStrategy(
            dim=head_dim, Sigma_q=sigma, bits=key_bits, device=self.device, dtype=torch.float32)
        self.quantizer = self.key_strategy
        self._key_chunks: list[Any] = []
        self._value_chunks: list[ValueQuantized] = []
        self._chunk_lengths: list[int] = []
        self._flat: Optional[FlatCache] = None
        # append-only GPU columns (used for strategies with fused kernels)
        self._cols: dict[str, _Column] = {}
        self._n = 0
        self._key_meta: Optional[tuple] = None
        self._mem_bytes = 0

    @property
    def capabilities(self) -> CacheCapabilities:
        return self.key_strategy.capabilities

    @property
    def num_tokens(self) -> int:
        return sum(self._chunk_lengths)

    @property
    def num_chunks(self) -> int:
        return len(self._chunk_lengths)

    def append_chunk(self, key: torch.Tensor, value: torch.Tensor):
        """Quantise and append a [T, Hkv, D] chunk (smaq/store.py:83-95)."""
        chunk_len = key.shape[0]
        k = key.transpose(0, 1).unsqueeze(0)
        v = value.transpose(0, 1).unsqueeze(0)
        key_q = self.key_strategy.quantize(k)
        val_q = quantize_values(v, bits=self.value_bits, group_size=self.value_group_size)
        self._mem_bytes += self.key_strategy.memory_bytes(key_q) + _value_bytes(val_q)
        self._chunk_lengths.append(chunk_len)
        if self._append_columns(key_q, val_q):
            # the columns hold the chunk; the chunk tensors are released
            self._key_chunks.clear()
            self._value_chunks.clear()
        else:
            self._key_chunks.append(key_q)
            self._value_chunks.append(val_q)
        self._flat = None

    def _append_columns(self, key_q: Any, val_q: ValueQuantized) -> bool:
        """Copy the chunk into the columns; False (columns dropped) for key
        layouts they do not handle."""
        fields = _key_fields(key_q)
        if fields is None or (self._n and not self._cols):
            if self._cols:
                raise ValueError("key chunks of different layouts in one store")
            return False
        meta, tensors = fields
        if self._key_meta is not None and self._key_meta != meta:
            raise ValueError("key chunks of different layouts in one store")
        self._key_meta = meta
        tensors = dict(tensors)
        tensors["v_data"] = val_q.data.reshape(-1, *val_q.data.shape[-2:])
        tensors["v_scales"] = val_q.scales.reshape(-1, *val_q.scales.shape[-2:])
        tensors["v_zeros"] = val_q.zeros.reshape(-1, *val_q.zeros.shape[-2:])
        n_old = self._n
        for name, t in tensors.items():
            self._cols.setdefault(name, _Column()).append(t, n_old)
        self._n = n_old + tensors["v_data"].shape[1]
        return True

    def get_flat_cache(self) -> Optional[FlatCache]:
        """Head-major flattened history (smaq/store.py:97-114)."""
        if not self._chunk_lengths:
            return None
        if self._flat is not None:
            return self._flat
        n = self._n
        if self._cols and self._key_meta is not None:
            kind, bits_or_nb, block_dim = self._key_meta
            if kind == "scalar":
                from smaq_amd.quantizer import SMAQQuantized
                key_q = SMAQQuantized(indices=self._cols["k_codes"].view(n), norms=self._cols["k_norms"].view(n),
                                      bits=bits_or_nb)
            else:
                from smaq_amd.block_vq import BlockVQQuantized
                key_q = BlockVQQuantized(indices=self._cols["k_codes"].view(n), n_blocks=bits_or_nb,
                                         block_dim=block_dim)
            vq = ValueQuantized(data=self._cols["v_data"].view(n), scales=self._cols["v_scales"].view(n),
                                zeros=self._cols["v_zeros"].view(n), bits=self.value_bits)
        else:
            s = self.key_strategy
            if len(self._key_chunks) == 1:
                key_q = s.flatten_quantized(self._key_chunks[0])
                vq = _flatten_value_q(self._value_chunks[0])
            else:
                key_q = s.concat_quantized([s.flatten_quantized(c) for c in self._key_chunks])
                vq = _concat_value_q([_flatten_value_q(c) for c in self._value_chunks])
        self._flat = FlatCache(key_q=key_q, value_q=vq, num_tokens=self.num_tokens)
        return self._flat

    def memory_bytes(self) -> int:
        """Per-chunk key bytes plus value bytes with 16-bit metadata, summed
        over the appended chunks (smaq/store.py:116-124)."""
        return self._mem_bytes

    def reset(self):
        self._key_chunks.clear()
        self._value_chunks.clear()
        self._chunk_lengths.clear()
        self._flat = None
        self._cols = {}
        self._n = 0
        self._key_meta = None
        self._mem_bytes = 0


def _key_fields(key_q: Any):
    """Per-token key tensors of a quantised chunk as [Hkv, T, ...] views, or
    None for layouts the columns do not handle."""
    from smaq_amd.block_vq import BlockVQQuantized
    from smaq_amd.quantizer import SMAQQuantized
    if isinstance(key_q, SMAQQuantized):
        ind = key_q.indices
        return ("scalar", key_q.bits, 0), {
            "k_codes": ind.reshape(-1, *ind.shape[-2:]),
            "k_norms": key_q.norms.reshape(-1, key_q.norms.shape[-1]),
        }
    if isinstance(key_q, BlockVQQuantized):
        ind = key_q.indices
        return ("block_vq", key_q.n_blocks, key_q.block_dim), {"k_codes": ind.reshape(-1, *ind.shape[-2:])}
    return None


def _value_bytes(vq: ValueQuantized) -> int:
    """Value bytes of a chunk, metadata counted at 2 bytes (smaq/store.py:120-123)."""
    return vq.data.nelement() + vq.scales.nelement() * 2 + vq.zeros.nelement() * 2


def _flatten_value_q(value_q: ValueQuantized) -> ValueQuantized:
    """(1, H, T, ...) -> (H, T, ...) (smaq/store.py:133-141)."""
    bits = value_q.bits if len(value_q) > 3 else 2
    return ValueQuantized(
        data=value_q.data.reshape(-1, value_q.data.shape[-2], value_q.data.shape[-1]).contiguous(),
        scales=value_q.scales.reshape(-1, value_q.scales.shape[-2], value_q.scales.shape[-1]).contiguous(),
        zeros=value_q.zeros.reshape(-1, value_q.zeros.shape[-2], value_q.zeros.shape[-1]).contiguous(),
        bits=bits,
    )


def _concat_value_q(chunks: list[ValueQuantized]) -> ValueQuantized:
    """Token-dim concatenation (smaq/store.py:144-152)."""
    bits = chunks[0].bits if len(chunks[0]) > 3 else 2
    return ValueQuantized(data=torch.cat([c.data for c in chunks], dim=-2),
                          scales=torch.cat([c.scales for c in chunks], dim=-2),
                          zeros=torch.cat([c.zeros for c in chunks], dim=-2), bits=bits)
