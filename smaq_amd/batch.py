"""Batched quantized-KV caches for serving: many sequences per launch.

``compute_hybrid_attention`` serves one store (one sequence, as the
reference's store is used).  Decode over a batch needs every sequence's
history in one launch; two layouts are provided, both read by the same fused
HIP kernels through ``score.launch_fused_attention``:

* ``QuantizedKVBatch`` -- contiguous: per KV head, sequences back to back
  (row = h * total_tokens + seq_start[b] + t).
* ``PagedQuantizedKV`` -- paged: fixed-size physical blocks of ``block_size``
  tokens addressed through a per-sequence block table, the layout of vLLM's
  paged KV cache (row = (block * Hkv + h) * block_size + t % block_size).

Both hold, per token-head row: packed key codes, key norm, packed value
bytes, value scales and zeros -- the FlatCache fields of ``store.py``.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import torch

from smaq_amd import _native
from smaq_amd.kv_cache import quantize_values
from smaq_amd.score import AttentionPlan


def _encode_rows(strategy, keys_rows: torch.Tensor, values_rows: torch.Tensor, value_bits: int, group: int):
    """Encode [..., D] rows with the strategy's key codec and the value packer."""
    kq = strategy.quantize(keys_rows)
    vq = quantize_values(values_rows, bits=value_bits, group_size=group)
    codes = kq.indices
    norms = getattr(kq, "norms", None)
    return codes, norms, vq.data, vq.scales, vq.zeros


class QuantizedKVBatch:
    """Contiguous batched history: fields shaped [Hkv, total_tokens, ...]."""

    def __init__(self, strategy, codes, norms, v_data, v_scales, v_zeros, seq_lens: Sequence[int],
                 value_bits: int, value_group: int):
        self.strategy = strategy
        self.codes, self.norms = codes, norms
        self.v_data, self.v_scales, self.v_zeros = v_data, v_scales, v_zeros
        self.seq_lens = [int(x) for x in seq_lens]
        self.value_bits, self.value_group = value_bits, value_group
        dev = codes.device
        starts = [0]
        for n in self.seq_lens[:-1]:
            starts.append(starts[-1] + n)
        self.uniform = len(set(self.seq_lens)) == 1
        self.seq_start = torch.tensor(starts, dtype=torch.int64, device=dev)
        self.hist_len = torch.tensor(self.seq_lens, dtype=torch.int64, device=dev)
        self.num_kv_heads = codes.shape[0]
        self.total = codes.shape[1]

    @classmethod
    def encode(cls, strategy, keys: Sequence[torch.Tensor], values: Sequence[torch.Tensor], value_bits: int = 2,
               value_group: int = 32) -> "QuantizedKVBatch":
        """keys/values: per sequence [N_b, Hkv, D] (or one [B, N, Hkv, D] tensor)."""
        if isinstance(keys, torch.Tensor):
            keys, values = list(keys.unbind(0)), list(values.unbind(0))
        lens = [k.shape[0] for k in keys]
        k = torch.cat(list(keys), dim=0).transpose(0, 1)    # [Hkv, total, D] view
        v = torch.cat(list(values), dim=0).transpose(0, 1)
        codes, norms, vd, vs, vz = _encode_rows(strategy, k, v, value_bits, value_group)
        return cls(strategy, codes, norms, vd, vs, vz, lens, value_bits, value_group)

    def nbytes_per_token_head(self) -> int:
        n = self.codes.shape[-1] * self.codes.element_size()
        if self.norms is not None:
            n += self.norms.element_size()
        n += self.v_data.shape[-1] + 2 * self.v_scales.shape[-1] * self.v_scales.element_size()
        return n

    def plan(self, query: torch.Tensor, scale: Optional[float] = None, recent_k: Optional[torch.Tensor] = None,
             recent_v: Optional[torch.Tensor] = None, recent_len: Optional[torch.Tensor] = None,
             impl: int = 0) -> AttentionPlan:
        """A reusable decode launch for queries shaped like ``query`` ([B, Hq, D]
        or [B, T, Hq, D]); see ``score.AttentionPlan``."""
        q = query.unsqueeze(1) if query.dim() == 3 else query
        D = q.shape[-1]
        scale = 1.0 / math.sqrt(D) if scale is None else scale
        max_r = 0 if recent_k is None else recent_k.shape[1]
        return AttentionPlan(
            query=q, fused=self.strategy.fused_history(), key_codes=self.codes, key_norms=self.norms,
            val_data=self.v_data, val_scales=self.v_scales, val_zeros=self.v_zeros, val_bits=self.value_bits,
            val_group=self.value_group, n_kv_heads=self.num_kv_heads,
            hist_len=None if self.uniform else self.hist_len, max_hist_len=max(self.seq_lens),
            hist_seq_start=None if self.uniform else self.seq_start, hist_head_stride=self.total,
            recent_k=recent_k, recent_v=recent_v, recent_len=recent_len, max_recent_len=max_r,
            scale=scale, out_dtype=query.dtype, hist_pos_offset=0, impl=impl)

    def attention(self, query: torch.Tensor, scale: Optional[float] = None,
                  recent_k: Optional[torch.Tensor] = None, recent_v: Optional[torch.Tensor] = None,
                  recent_len: Optional[torch.Tensor] = None, impl: int = 0) -> torch.Tensor:
        """query [B, Hq, D] (one decode token per sequence) or [B, T, Hq, D];
        recent_k/v [B, R, Hkv, D] with per-sequence recent_len.  Returns the
        query's shape in its dtype.  ``impl``: 0 automatic, 1 generic kernels,
        2 matrix-core decode kernel, 3 matrix-core prefill kernel."""
        out = self.plan(query, scale, recent_k, recent_v, recent_len, impl).run(query)
        return out.squeeze(1) if query.dim() == 3 else out


class PagedQuantizedKV:
    """Paged history: pools [num_blocks, Hkv, block_size, ...] plus block tables."""

    def __init__(self, strategy, codes, norms, v_data, v_scales, v_zeros, block_table: torch.Tensor,
                 seq_lens: Sequence[int], block_size: int, value_bits: int, value_group: int):
        self.strategy = strategy
        self.codes, self.norms = codes, norms
        self.v_data, self.v_scales, self.v_zeros = v_data, v_scales, v_zeros
        self.block_table = block_table.to(torch.int32).contiguous()
        self.seq_lens = [int(x) for x in seq_lens]
        self.block_size = block_size
        self.value_bits, self.value_group = value_bits, value_group
        self.num_kv_heads = codes.shape[1]
        self.hist_len = torch.tensor(self.seq_lens, dtype=torch.int64, device=codes.device)

    @classmethod
    def encode(cls, strategy, keys: Sequence[torch.Tensor], values: Sequence[torch.Tensor],
               block_table: torch.Tensor, num_blocks: int, block_size: int = 16, value_bits: int = 2,
               value_group: int = 32) -> "PagedQuantizedKV":
        """Scatter per-sequence [N_b, Hkv, D] keys/values into physical blocks
        (block_table [B, max_blocks]) and encode the pools in place order."""
        dev = keys[0].device
        hkv, D = keys[0].shape[1], keys[0].shape[2]
        kp = torch.zeros(num_blocks, block_size, hkv, D, dtype=keys[0].dtype, device=dev)
        vp = torch.zeros(num_blocks, block_size, hkv, D, dtype=values[0].dtype, device=dev)
        bt = block_table.to(dev, torch.long)
        for b, (k, v) in enumerate(zip(keys, values)):
            n = k.shape[0]
            nblk = (n + block_size - 1) // block_size
            pad = nblk * block_size - n
            kk = torch.cat([k, k.new_zeros(pad, hkv, D)]).reshape(nblk, block_size, hkv, D)
            vv = torch.cat([v, v.new_zeros(pad, hkv, D)]).reshape(nblk, block_size, hkv, D)
            kp.index_copy_(0, bt[b, :nblk], kk)
            vp.index_copy_(0, bt[b, :nblk], vv)
        codes, norms, vd, vs, vz = _encode_rows(strategy, kp.permute(0, 2, 1, 3), vp.permute(0, 2, 1, 3),
                                                value_bits, value_group)
        return cls(strategy, codes, norms, vd, vs, vz, block_table, [k.shape[0] for k in keys], block_size,
                   value_bits, value_group)

    def plan(self, query: torch.Tensor, scale: Optional[float] = None, impl: int = 0,
             query_positions: Optional[torch.Tensor] = None) -> AttentionPlan:
        """A reusable launch for queries shaped like ``query`` ([B, Hq, D] or
        [B, T, Hq, D]); ``query_positions`` int64 [B, T] masks history token
        j for query t when j > query_positions[b, t]."""
        q = query.unsqueeze(1) if query.dim() == 3 else query
        D = q.shape[-1]
        scale = 1.0 / math.sqrt(D) if scale is None else scale
        return AttentionPlan(
            query=q, fused=self.strategy.fused_history(), key_codes=self.codes, key_norms=self.norms,
            val_data=self.v_data, val_scales=self.v_scales, val_zeros=self.v_zeros, val_bits=self.value_bits,
            val_group=self.value_group, n_kv_heads=self.num_kv_heads, hist_len=self.hist_len,
            max_hist_len=max(self.seq_lens), block_table=self.block_table, block_size=self.block_size,
            scale=scale, out_dtype=query.dtype, query_positions=query_positions, impl=impl)

    def nbytes_per_token_head(self) -> int:
        n = self.codes.shape[-1] + (self.norms.element_size() if self.norms is not None else 0)
        return n + self.v_data.shape[-1] + 2 * self.v_scales.shape[-1] * self.v_scales.element_size()

    def attention(self, query: torch.Tensor, scale: Optional[float] = None, impl: int = 0,
                  query_positions: Optional[torch.Tensor] = None) -> torch.Tensor:
        """query [B, Hq, D] -> [B, Hq, D], or [B, T, Hq, D] -> [B, T, Hq, D]."""
        out = self.plan(query, scale, impl, query_positions).run(query)
        return out.squeeze(1) if query.dim() == 3 else out


def require_native() -> None:
    """Raise now if libsmaq_hip.so cannot be loaded."""
    _native.lib()
