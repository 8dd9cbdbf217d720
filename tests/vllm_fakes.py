"""Stand-ins for the vLLM objects the adapter touches (vLLM is not installed).

Only the attributes the reference adapter reads are modelled
(smaq/integration/vllm.py:113-442): a flash-style attention impl with
``do_kv_cache_update`` / ``forward``, an MLA impl with ``forward_mqa``, the
attention metadata fields, and a model runner with
``compilation_config.static_forward_context``, ``device`` and ``kv_caches``.
The flash impl's forward is exact paged attention over its own fp32 math.
"""

from __future__ import annotations

import math
from types import SimpleNamespace

import torch


class FakeFlashImpl:
    def __init__(self, num_heads: int, num_kv_heads: int, head_size: int, scale: float | None = None):
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_size = head_size
        self.scale = 1.0 / math.sqrt(head_size) if scale is None else scale
        self.calls: list[str] = []

    def do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping):
        self.calls.append("update")
        write_paged(kv_cache, key, value, slot_mapping)

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None, output_scale=None,
                output_block_scale=None):
        self.calls.append("forward")
        if attn_metadata is None:
            return query
        if getattr(attn_metadata, "seq_lens", None) is None:     # prefill step without paged metadata
            return torch.zeros_like(query)
        res = exact_paged_decode(query, kv_cache, attn_metadata, self.num_heads, self.num_kv_heads,
                                 self.head_size, self.scale)
        if output is not None:
            output[: res.shape[0]].copy_(res.reshape(output[: res.shape[0]].shape))
            return output
        return res


class FakeFlashImplNoUpdate(FakeFlashImpl):
    """An impl whose K/V are captured in forward (no do_kv_cache_update)."""

    def __getattribute__(self, name):
        if name == "do_kv_cache_update":
            raise AttributeError(name)
        return super().__getattribute__(name)


class FakeMLAImpl:
    def __init__(self, num_kv_heads: int = 1, kv_lora_rank: int = 64):
        self.num_kv_heads = num_kv_heads
        self.kv_lora_rank = kv_lora_rank
        self.calls: list[str] = []

    def do_kv_cache_update(self, kv_c_normed, k_pe, kv_cache, slot_mapping, kv_cache_dtype, k_scale):
        self.calls.append("mla_update")

    def forward_mqa(self, q, kv_c_and_k_pe_cache, attn_metadata, layer):
        self.calls.append("mla_forward")
        return q


def write_paged(kv_cache: torch.Tensor, key, value, slot_mapping) -> None:
    """vLLM's reshape_and_cache: token i goes to slot slot_mapping[i]."""
    if kv_cache.dim() != 5:
        return
    hkv, d = kv_cache.shape[3], kv_cache.shape[4]
    slots = slot_mapping.to(torch.long)
    keep = slots >= 0
    kv_cache[0].view(-1, hkv, d)[slots[keep]] = key[: slots.shape[0]][keep].to(kv_cache.dtype)
    kv_cache[1].view(-1, hkv, d)[slots[keep]] = value[: slots.shape[0]][keep].to(kv_cache.dtype)


def exact_paged_decode(query, kv_cache, meta, hq, hkv, d, scale):
    """fp32 attention of one query token per sequence over its paged K/V."""
    n = meta.num_actual_tokens
    q = query[:n].reshape(n, hq, d).float()
    bs = kv_cache.shape[2]
    outs = []
    for b in range(n):
        L = int(meta.seq_lens[b])
        blocks = meta.block_table[b, : (L + bs - 1) // bs].to(torch.long)
        k = kv_cache[0][blocks].reshape(-1, hkv, d)[:L].float()
        v = kv_cache[1][blocks].reshape(-1, hkv, d)[:L].float()
        g = hq // hkv
        kk = k.repeat_interleave(g, dim=1).transpose(0, 1)        # [hq, L, d]
        vv = v.repeat_interleave(g, dim=1).transpose(0, 1)
        w = torch.softmax((q[b][:, None, :] * kk).sum(-1) * scale, dim=-1)
        outs.append((w[:, :, None] * vv).sum(1))
    return torch.stack(outs).to(query.dtype)


def make_runner(impls: dict, device, kv_caches: dict | None = None, num_heads: dict | None = None):
    """A model runner whose static forward context maps layer names to
    attention modules holding the given impls (and optional kv_cache lists)."""
    ctx = {}
    caches = []
    for name, impl in impls.items():
        mod = SimpleNamespace(impl=impl)
        if num_heads and name in num_heads:
            mod.num_heads = num_heads[name]
        if kv_caches and name in kv_caches:
            mod.kv_cache = [kv_caches[name]]
            caches.append(kv_caches[name])
        ctx[name] = mod
    ctx["not_attention"] = SimpleNamespace(weight=None)
    return SimpleNamespace(compilation_config=SimpleNamespace(static_forward_context=ctx), device=device,
                           kv_caches=caches)


def meta(num_actual_tokens: int, max_query_len: int, **kw):
    return SimpleNamespace(num_actual_tokens=num_actual_tokens, max_query_len=max_query_len, **kw)
