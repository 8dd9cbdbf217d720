"""Recent-window capture (drop-in for smaq/capture.py).

``RingBuffer`` holds the newest tokens of one layer exact, ``[capacity, Hkv,
D]``.  Its wrap rule is the reference's (smaq/capture.py:60-91): when a write
finds the ring full and tokens remain, the ring's whole content leaves as
overflow and filling restarts at slot 0.  Seen as one token stream -- the
ring's p tokens followed by the n written -- that rule cuts the stream into
``capacity``-token windows and spills every window but the last, so a write
is computed in one step: m = (p + n - 1) // capacity windows spill (none
when p + n <= capacity), i.e. the ring's p tokens and the first
m * capacity - p written tokens, and the ring keeps the remaining ones.

``KVCaptureEngine`` routes tokens: prefill tails and decode tokens into the
ring, prefill heads and ring spills into the compressed store.  A spill is
handed to the store as two pieces -- a view of the ring's slots and a view of
the written tokens -- which the store's HIP encoders read in place and write
straight into its append-only columns; nothing is joined or cloned.  (The
reference clones the ring, concatenates the pieces and re-concatenates the
store's whole history on the next read.)
"""

from __future__ import annotations

from typing import Callable, Optional, Sequence, TYPE_CHECKING

import torch

if TYPE_CHECKING:
    from smaq_amd.store import CompressedKVStore

Pieces = Sequence[tuple[torch.Tensor, torch.Tensor]]


class RingBuffer:
    """Fixed-capacity exact window of K/V [capacity, Hkv, D] (smaq/capture.py:18-110)."""

    def __init__(self, capacity: int, num_kv_heads: int, head_dim: int, device: torch.device,
                 dtype: torch.dtype = torch.bfloat16):
        if capacity <= 0:
            raise ValueError(f"ring capacity must be positive, got {capacity}")
        self.capacity = capacity
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.device = device
        self.dtype = dtype
        self._slots_k = torch.zeros(capacity, num_kv_heads, head_dim, device=device, dtype=dtype)
        self._slots_v = torch.zeros(capacity, num_kv_heads, head_dim, device=device, dtype=dtype)
        self._fill = 0       # occupied slots [0, _fill)
        self._written = 0    # tokens ever written

    @property
    def size(self) -> int:
        return self._fill

    @property
    def total_written(self) -> int:
        return self._written

    def _advance(self, key: torch.Tensor, value: torch.Tensor, n: int,
                 spill: Optional[Callable[[Pieces], None]]) -> None:
        """Write n tokens; the spilled window(s), if any, go to ``spill`` as
        pieces in token order before any slot is overwritten (None drops
        them).  Written tokens take the ring's dtype and device first, as
        writing them into the slots does."""
        if n <= 0:
            return
        key = key[:n].to(device=self.device, dtype=self.dtype)
        value = value[:n].to(device=self.device, dtype=self.dtype)
        p, C = self._fill, self.capacity
        stream = p + n
        spilled = (stream - 1) // C * C          # tokens of the stream that leave
        if spilled and spill is not None:
            pieces = []
            if p:
                pieces.append((self._slots_k[:p], self._slots_v[:p]))
            pieces.append((key[:spilled - p], value[:spilled - p]))
            spill(pieces)
        keep_from = max(spilled - p, 0)           # first written token that stays
        at = p if spilled == 0 else 0
        self._slots_k[at:at + n - keep_from].copy_(key[keep_from:])
        self._slots_v[at:at + n - keep_from].copy_(value[keep_from:])
        self._fill = stream - spilled
        self._written += n

    def write(self, key: torch.Tensor, value: torch.Tensor,
              num_tokens: int) -> Optional[tuple[torch.Tensor, torch.Tensor]]:
        """Append tokens; returns the overflow (its own tensors) when the ring
        wrapped, else None (smaq/capture.py:60-91)."""
        out: list[tuple[torch.Tensor, torch.Tensor]] = []

        def keep(pieces: Pieces) -> None:
            out.append((torch.cat([k for k, _ in pieces]), torch.cat([v for _, v in pieces])))

        self._advance(key, value, num_tokens, keep)
        return out[0] if out else None

    def drain(self) -> Optional[tuple[torch.Tensor, torch.Tensor]]:
        """The buffered tokens (copies); the ring is left empty."""
        if self._fill == 0:
            return None
        k, v = self._slots_k[:self._fill].clone(), self._slots_v[:self._fill].clone()
        self._fill = 0
        return k, v

    def peek(self) -> Optional[tuple[torch.Tensor, torch.Tensor]]:
        """Views of the buffered tokens, oldest first."""
        if self._fill == 0:
            return None
        return self._slots_k[:self._fill], self._slots_v[:self._fill]

    def reset(self):
        self._fill = 0
        self._written = 0


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
        """The newest ``capacity`` tokens go to the ring, the older ones to the
        store (smaq/capture.py:145-153).  As in the reference, a spill caused
        by writing into a partly filled ring is dropped, not stored."""
        C = self.ring.capacity
        head = max(0, num_tokens - C)
        if head:
            self.store.append_chunk(key[:head], value[:head])
        self.ring._advance(key[head:num_tokens], value[head:num_tokens], num_tokens - head, None)
        self._prefill_done = True

    def ingest_prefill_from_paged_cache(self, kv_cache_tensor: torch.Tensor, num_tokens: int,
                                        block_table: torch.Tensor, block_size: int):
        """A prefill read out of a vLLM paged KV tensor [2, blocks, block_size,
        Hkv, D] through the sequence's block table (smaq/capture.py:155-177):
        one gather of the needed blocks, then ``ingest_prefill``."""
        nblk = -(-num_tokens // block_size)
        phys = block_table[:nblk].to(kv_cache_tensor.device, torch.long)
        kv = kv_cache_tensor.index_select(1, phys)                   # [2, nblk, bs, Hkv, D]
        kv = kv.reshape(2, nblk * block_size, *kv_cache_tensor.shape[3:])[:, :num_tokens]
        self.ingest_prefill(kv[0], kv[1], num_tokens)

    def _to_store(self, pieces: Pieces) -> None:
        """One chunk given as pieces: in place for a store that takes pieces,
        else joined for a store with only the reference's ``append_chunk``."""
        append_parts = getattr(self.store, "append_parts", None)
        if append_parts is not None:
            append_parts(pieces)
        else:
            self.store.append_chunk(torch.cat([k for k, _ in pieces]), torch.cat([v for _, v in pieces]))

    def ingest_decode(self, key: torch.Tensor, value: torch.Tensor, num_tokens: int):
        """Decode tokens into the ring; a spill is encoded into the store
        directly from the ring's slots and the new tokens (smaq/capture.py:179-183)."""
        self.ring._advance(key, value, num_tokens, self._to_store)

    def flush(self):
        """Move the buffered tokens into the store (smaq/capture.py:185-189)."""
        pieces = self.ring.peek()
        if pieces is not None:
            self._to_store([pieces])
            self.ring._fill = 0

    def reset(self):
        self.ring.reset()
        self.store.reset()
        self._prefill_done = False
