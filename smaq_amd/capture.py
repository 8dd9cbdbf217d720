"""Recent-window capture (drop-in for smaq/capture.py).

``RingBuffer`` keeps the newest tokens exact; once it is full, the next write
returns the whole ring as overflow, which ``KVCaptureEngine`` hands to the
compressed store (where the HIP encoders run).  Plain tensor copies.
"""

from __future__ import annotations

from typing import Optional, TYPE_CHECKING

import torch

if TYPE_CHECKING:
    from smaq_amd.store import CompressedKVStore


class RingBuffer:
    """Fixed-capacity window of exact K/V [capacity, Hkv, D] (smaq/capture.py:18-110)."""

    __slots__ = ("capacity", "num_kv_heads", "head_dim", "device", "dtype", "_k", "_v", "_pos",
                 "_total_written")

    def __init__(self, capacity: int, num_kv_heads: int, head_dim: int, device: torch.device,
                 dtype: torch.dtype = torch.bfloat16):
        self.capacity = capacity
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.device = device
        self.dtype = dtype
        self._k = torch.zeros(capacity, num_kv_heads, head_dim, device=device, dtype=dtype)
        self._v = torch.zeros(capacity, num_kv_heads, head_dim, device=device, dtype=dtype)
        self._pos = 0
        self._total_written = 0

    @property
    def size(self) -> int:
        return self._pos

    @property
    def total_written(self) -> int:
        return self._total_written

    def write(self, key: torch.Tensor, value: torch.Tensor,
              num_tokens: int) -> Optional[tuple[torch.Tensor, torch.Tensor]]:
        """Append tokens; when the ring is full and more arrive, its whole
        content is returned as overflow and the ring restarts (smaq/capture.py:60-91)."""
        spill_k, spill_v = [], []
        done = 0
        while done < num_tokens:
            if self._pos >= self.capacity:
                spill_k.append(self._k[: self._pos].clone())
                spill_v.append(self._v[: self._pos].clone())
                self._pos = 0
            n = min(num_tokens - done, self.capacity - self._pos)
            self._k[self._pos: self._pos + n] = key[done: done + n]
            self._v[self._pos: self._pos + n] = value[done: done + n]
            self._pos += n
            done += n
        self._total_written += num_tokens
        if spill_k:
            return torch.cat(spill_k, dim=0), torch.cat(spill_v, dim=0)
        return None

    def drain(self) -> Optional[tuple[torch.Tensor, torch.Tensor]]:
        if self._pos == 0:
            return None
        k, v = self._k[: self._pos].clone(), self._v[: self._pos].clone()
        self._pos = 0
        return k, v

    def peek(self) -> Optional[tuple[torch.Tensor, torch.Tensor]]:
        if self._pos == 0:
            return None
        return self._k[: self._pos], self._v[: self._pos]

    def reset(self):
        self._pos = 0
        self._total_written = 0


class KVCaptureEngine:
    """Routes prefill/decode tokens to the ring and ring overflow to the store
    (smaq/capture.py:113-194)."""

    def __init__(self, store: "CompressedKVStore", ring_capacity: int = 128, device: torch.device | None = None,
                 dtype: torch.dtype = torch.bfloat16):
        self.store = store
        self.ring = RingBuffer(capacity=ring_capacity, num_kv_heads=store.num_kv_heads, head_dim=store.head_dim,
                               device=device or store.device, dtype=dtype)
        self._prefill_done = False

    @property
    def total_compressed_tokens(self) -> int:
        return self.store.num_tokens

    @property
    def total_buffered_tokens(self) -> int:
        return self.ring.size

    @property
    def total_tokens(self) -> int:
        return self.total_compressed_tokens + self.total_buffered_tokens

    def ingest_prefill(self, key: torch.Tensor, value: torch.Tensor, num_tokens: int):
        """All but the last ``capacity`` tokens go to the store
        (smaq/capture.py:145-153); like the reference, a write that overflows a
        partly filled ring drops that overflow."""
        if num_tokens <= self.ring.capacity:
            self.ring.write(key[:num_tokens], value[:num_tokens], num_tokens)
        else:
            n_c = num_tokens - self.ring.capacity
            self.store.append_chunk(key[:n_c], value[:n_c])
            self.ring.write(key[n_c:num_tokens], value[n_c:num_tokens], self.ring.capacity)
        self._prefill_done = True

    def ingest_prefill_from_paged_cache(self, kv_cache_tensor: torch.Tensor, num_tokens: int,
                                        block_table: torch.Tensor, block_size: int):
        """Gather a prefill from a vLLM paged KV tensor [2, blocks, bs, Hkv, D]
        (smaq/capture.py:155-177)."""
        nblk = (num_tokens + block_size - 1) // block_size
        phys = block_table[:nblk].to(kv_cache_tensor.device, torch.long)
        k = kv_cache_tensor[0].index_select(0, phys).reshape(-1, *kv_cache_tensor.shape[3:])[:num_tokens]
        v = kv_cache_tensor[1].index_select(0, phys).reshape(-1, *kv_cache_tensor.shape[3:])[:num_tokens]
        self.ingest_prefill(k, v, num_tokens)

    def ingest_decode(self, key: torch.Tensor, value: torch.Tensor, num_tokens: int):
        """(smaq/capture.py:179-183)"""
        overflow = self.ring.write(key[:num_tokens], value[:num_tokens], num_tokens)
        if overflow is not None:
            self.store.append_chunk(*overflow)

    def flush(self):
        data = self.ring.drain()
        if data is not None:
            self.store.append_chunk(*data)

    def reset(self):
        self.ring.reset()
        self.store.reset()
        self._prefill_done = False
