"""Concrete attention backends (drop-in for smaq/backends.py)."""

from __future__ import annotations

from smaq_amd.core import AttentionBackend
from smaq_amd.score import compute_hybrid_attention


class TorchHybridAttentionBackend(AttentionBackend):
    """Compressed history plus exact tail (smaq/backends.py:9-20).  The name
    is kept for drop-in use; the computation is the fused HIP attention."""

    def compute(self, query, store, recent_k, recent_v, num_query_heads, scale=None):
        return compute_hybrid_attention(query=query, store=store, recent_k=recent_k, recent_v=recent_v,
                                        num_query_heads=num_query_heads, scale=scale)


HipHybridAttentionBackend = TorchHybridAttentionBackend
