"""vLLM adapter (drop-in for smaq/integration/vllm.py).

Hooks a vLLM model runner's attention layers so that their K/V writes feed a
SMAQ capture engine (exact recent ring + compressed store, both per layer) and
decode steps can be served from compressed history plus the exact ring through
the fused HIP attention.  The modes, hook points and fall-backs follow the
reference (smaq/integration/vllm.py:27-272):

* ``off`` / ``capture_only``: the layer's own forward runs; in
  ``capture_only`` its K/V are captured as well.
* ``hybrid``: decode steps (``max_query_len == 1``) of flash-style layers are
  answered by ``compute_hybrid_attention`` once the store holds at least 16
  tokens; prefill runs the layer's own forward (or, with ``no_alloc``, causal
  SDPA over the step's own tokens).
* ``full_smaq``: accepted, and served like the reference (the layer's forward,
  or zeros with ``no_alloc``).
* MLA layers are detected and left as pass-through.

Paged serving (an extension; ``install_hooks(..., paged=True)``): instead of
one store per layer that mixes every sequence's tokens (the reference's
design, smaq/integration/vllm.py:83-95), each layer keeps compressed pools
laid out like vLLM's own paged KV cache -- physical block ``blk`` of the
pools holds the compressed rows of vLLM's block ``blk``.  Every K/V write is
encoded straight into the rows its ``slot_mapping`` names, and a decode step
of the whole batch is one launch of the paged matrix-core decode kernel over
vLLM's ``block_table`` and ``seq_lens``, written into ``output``.

vLLM itself is not a dependency: the hooks only touch the attributes named
above (``impl.forward``, ``impl.do_kv_cache_update``, ``attn_metadata``
fields, ``model_runner.compilation_config.static_forward_context``).
"""

from __future__ import annotations

import logging
import math
import types
from collections import OrderedDict
from dataclasses import dataclass, field
from typing import Optional

import torch
import torch.nn.functional as F

from smaq_amd.capture import KVCaptureEngine
from smaq_amd.score import MIN_HISTORY_FOR_SMAQ, compute_hybrid_attention
from smaq_amd.store import CompressedKVStore

# the reference's logger name (smaq/integration/vllm.py:25), so that a
# deployment's logging configuration carries over
logger = logging.getLogger("smaq.integration.vllm")

MODE_OFF = "off"
MODE_CAPTURE_ONLY = "capture_only"
MODE_HYBRID = "hybrid"
MODE_FULL_SMAQ = "full_smaq"
_VALID_MODES = (MODE_OFF, MODE_CAPTURE_ONLY, MODE_HYBRID, MODE_FULL_SMAQ)

# One process-wide mode, read by every hooked layer on each call (not
# thread-safe, like the reference's module global).
_GLOBAL_MODE = MODE_CAPTURE_ONLY


def set_mode(mode: str) -> None:
    """Switch every hooked layer's behaviour (smaq/integration/vllm.py:36-41)."""
    global _GLOBAL_MODE
    if mode not in _VALID_MODES:
        raise ValueError(f"Invalid mode: {mode}. Valid: {_VALID_MODES}")
    _GLOBAL_MODE = mode
    logger.info("[SMAQ] Mode set to %s", mode)


def get_mode() -> str:
    return _GLOBAL_MODE


@dataclass
class LayerConfig:
    """Per-layer configuration (smaq/integration/vllm.py:48-62)."""

    head_dim: int
    num_kv_heads: int
    num_query_heads: int
    Sigma_q: Optional[torch.Tensor] = None
    key_bits: int = 3
    value_bits: int = 2
    value_group_size: int = 32
    ring_capacity: int = 128
    layer_idx: int = 0
    backend_kind: str = "flash"
    device: torch.device = field(default_factory=lambda: torch.device("cuda"))
    paged: bool = False


class PagedLayerCache:
    """Compressed pools shaped like a vLLM paged KV cache of one layer.

    Row of (physical block ``blk``, KV head ``h``, offset ``o``) is
    ``(blk * Hkv + h) * block_size + o`` in every field: key codes [rows, P]
    uint8, key norms [rows], value bytes [rows, D/vpb], value scales and zeros
    [rows, D/group] -- the paged layout the fused kernels read.  Pools are
    allocated on the first write, from the size of vLLM's cache tensor.
    """

    # decode plans kept per layer (least recently used dropped first)
    MAX_PLANS = 8

    def __init__(self, store: CompressedKVStore):
        self.store = store           # supplies the key strategy and value format
        self.num_blocks = 0
        self.block_size = 0
        self.pools: Optional[dict[str, torch.Tensor]] = None
        self.tokens_written = 0
        self._plans: "OrderedDict[tuple, object]" = OrderedDict()

    @staticmethod
    def cache_geometry(kv_cache: torch.Tensor, num_kv_heads: int, head_dim: int) -> tuple[int, int]:
        """(num_blocks, block_size) of a flash-layout cache [2, blocks, bs, Hkv, D]."""
        if kv_cache is None or kv_cache.dim() != 5 or kv_cache.shape[0] != 2 \
                or tuple(kv_cache.shape[3:]) != (num_kv_heads, head_dim):
            raise ValueError("paged SMAQ needs a [2, num_blocks, block_size, num_kv_heads, head_dim] KV cache; got "
                             f"{None if kv_cache is None else tuple(kv_cache.shape)}")
        return int(kv_cache.shape[1]), int(kv_cache.shape[2])

    def ensure(self, num_blocks: int, block_size: int, key_dtype: torch.dtype, value_dtype: torch.dtype,
               device: torch.device) -> None:
        if self.pools is not None:
            if (num_blocks, block_size) != (self.num_blocks, self.block_size):
                raise ValueError("vLLM KV cache geometry changed under a hooked layer")
            return
        st = self.store
        hkv, D = st.num_kv_heads, st.head_dim
        rows = num_blocks * hkv * block_size
        probe = torch.zeros(1, 1, 1, D, dtype=key_dtype, device=device)
        kq = st.key_strategy.quantize(probe)
        vpb = max(1, 8 // st.value_bits)
        pools = {"k_codes": torch.zeros(rows, kq.indices.shape[-1], dtype=kq.indices.dtype, device=device),
                 "v_data": torch.zeros(rows, (D + vpb - 1) // vpb, dtype=torch.uint8, device=device),
                 "v_scales": torch.zeros(rows, D // st.value_group_size, dtype=value_dtype, device=device),
                 "v_zeros": torch.zeros(rows, D // st.value_group_size, dtype=value_dtype, device=device)}
        norms = getattr(kq, "norms", None)
        if norms is not None:
            pools["k_norms"] = torch.zeros(rows, dtype=norms.dtype, device=device)
        self.pools = pools
        self.num_blocks, self.block_size = num_blocks, block_size

    def write(self, key: torch.Tensor, value: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        """Encode tokens key/value [T, Hkv, D] into the rows of their slots
        (slot = block * block_size + offset; negative slots are padding)."""
        from smaq_amd.kv_cache import quantize_values
        st = self.store
        hkv, D = st.num_kv_heads, st.head_dim
        slots = slot_mapping.to(key.device, torch.int64).reshape(-1)
        T = min(int(slots.shape[0]), key.shape[0])
        key = key[:T].reshape(T, hkv, D)
        value = value[:T].reshape(T, hkv, D)
        slots = slots[:T]
        keep = slots >= 0
        if not bool(keep.all()):
            key, value, slots = key[keep], value[keep], slots[keep]
            T = int(slots.shape[0])
        if T == 0:
            return
        kq = st.key_strategy.quantize(key.unsqueeze(0))        # rows (t, h), dense
        vq = quantize_values(value.unsqueeze(0), bits=st.value_bits, group_size=st.value_group_size)
        bs = self.block_size
        h = torch.arange(hkv, device=key.device)
        rows = (((slots // bs)[:, None] * hkv + h[None, :]) * bs + (slots % bs)[:, None]).reshape(-1)
        fields = {"k_codes": kq.indices, "v_data": vq.data, "v_scales": vq.scales, "v_zeros": vq.zeros}
        if "k_norms" in self.pools:
            fields["k_norms"] = kq.norms
        for name, t in fields.items():
            pool = self.pools[name]
            self.pools[name].index_copy_(0, rows, t.reshape(rows.shape[0], *pool.shape[1:]))
        self.tokens_written += T

    def memory_bytes(self) -> int:
        if self.pools is None:
            return 0
        return sum(t.numel() * t.element_size() for t in self.pools.values())

    @staticmethod
    def length_bucket(max_seq_len: int) -> int:
        """The plan's length bound for a step whose longest sequence has
        max_seq_len tokens: the next power of two (at least 16), so that a
        growing batch re-uses one plan per doubling of its longest context."""
        return max(16, 1 << (max(int(max_seq_len), 1) - 1).bit_length())

    def _plan(self, query: torch.Tensor, block_table: torch.Tensor, max_seq_len: int, num_query_heads: int,
              scale: float, out_dtype: torch.dtype):
        """The cached decode plan for this batch shape (built on first use)."""
        from smaq_amd.score import AttentionPlan
        st = self.store
        B = query.shape[0]
        bound = self.length_bucket(max_seq_len)
        key = (B, int(block_table.shape[1]), num_query_heads, float(scale), out_dtype, query.dtype, bound,
               query.device)
        plan = self._plans.get(key)
        if plan is not None:
            self._plans.move_to_end(key)
            return plan
        pools = self.pools
        plan = AttentionPlan(
            query=query.reshape(B, 1, num_query_heads, st.head_dim), fused=st.key_strategy.fused_history(),
            key_codes=pools["k_codes"], key_norms=pools.get("k_norms"), val_data=pools["v_data"],
            val_scales=pools["v_scales"], val_zeros=pools["v_zeros"], val_bits=st.value_bits,
            val_group=st.value_group_size, n_kv_heads=st.num_kv_heads,
            hist_len=torch.zeros(B, dtype=torch.int64, device=query.device), max_hist_len=bound,
            block_table=block_table[:B], block_size=self.block_size, scale=scale, out_dtype=out_dtype)
        self._plans[key] = plan
        while len(self._plans) > self.MAX_PLANS:
            self._plans.popitem(last=False)
        return plan

    def decode(self, query: torch.Tensor, block_table: torch.Tensor, seq_lens: torch.Tensor, max_seq_len: int,
               num_query_heads: int, scale: float, out: torch.Tensor) -> None:
        """One decode token per sequence: query [B, Hq, D] over each
        sequence's ``seq_lens[b]`` tokens (``max_seq_len`` >= every one of
        them) through its block table; the result is written to out
        [B, Hq, D] (out's dtype).  The launch is prepared once per batch
        shape and re-used: a step copies the lengths into the plan, points it
        at the block table and writes straight into ``out`` when out is
        contiguous."""
        B = query.shape[0]
        plan = self._plan(query, block_table, max_seq_len, num_query_heads, scale, out.dtype)
        plan.set_lengths(hist_len=seq_lens)
        plan.set_block_table(block_table)
        q = query.reshape(B, 1, num_query_heads, self.store.head_dim)
        if out.is_contiguous():
            plan.run_into(q, out)
        else:
            out.copy_(plan.run(q).reshape(out.shape))

    def reset(self) -> None:
        self.tokens_written = 0
        self._plans.clear()


@dataclass
class LayerState:
    """Per-layer runtime state (smaq/integration/vllm.py:65-80)."""

    config: LayerConfig
    store: CompressedKVStore
    engine: KVCaptureEngine
    _log_count: int = 0
    paged: Optional[PagedLayerCache] = None
    # decode plan of the reference layout and what it was built for
    ref_plan: Optional[object] = None
    ref_plan_key: Optional[tuple] = None

    @property
    def supports_hybrid(self) -> bool:
        return self.config.backend_kind == "flash"

    def reset(self):
        self.engine.reset()
        if self.paged is not None:
            self.paged.reset()
        self.ref_plan = self.ref_plan_key = None
        self._log_count = 0


def _create_layer_state(cfg: LayerConfig) -> LayerState:
    store = CompressedKVStore(head_dim=cfg.head_dim, num_kv_heads=cfg.num_kv_heads, Sigma_q=cfg.Sigma_q,
                              key_bits=cfg.key_bits, value_bits=cfg.value_bits,
                              value_group_size=cfg.value_group_size, device=cfg.device, layer_idx=cfg.layer_idx)
    engine = KVCaptureEngine(store=store, ring_capacity=cfg.ring_capacity, device=cfg.device)
    return LayerState(config=cfg, store=store, engine=engine,
                      paged=PagedLayerCache(store) if cfg.paged else None)


def _infer_num_query_heads(attn_module, impl) -> int:
    """First non-empty of module.num_heads, module.num_attention_heads,
    impl.num_heads, else the KV head count (smaq/integration/vllm.py:98-106)."""
    for cand in (getattr(attn_module, "num_heads", None), getattr(attn_module, "num_attention_heads", None),
                 getattr(impl, "num_heads", None)):
        if cand:
            return int(cand)
    return int(impl.num_kv_heads)


def _is_mla_impl(impl) -> bool:
    """MLA impls expose forward_mqa + do_kv_cache_update and no forward
    (smaq/integration/vllm.py:109-110)."""
    return hasattr(impl, "forward_mqa") and hasattr(impl, "do_kv_cache_update") and not hasattr(impl, "forward")


def _capture(state: LayerState, key, value, num_tokens: int) -> None:
    """One token goes to the ring as decode, more as a prefill
    (smaq/integration/vllm.py:124-128)."""
    if num_tokens <= 1:
        state.engine.ingest_decode(key, value, num_tokens)
    else:
        state.engine.ingest_prefill(key, value, num_tokens)


def _paged_write(state: LayerState, key, value, kv_cache, slot_mapping) -> None:
    """Encode a K/V write into the layer's pools; their geometry comes from
    vLLM's cache tensor on the first write (afterwards that tensor may be the
    placeholder free_kv_cache leaves)."""
    pc = state.paged
    if pc.pools is None or (kv_cache is not None and kv_cache.dim() == 5):
        nb, bs = PagedLayerCache.cache_geometry(kv_cache, state.config.num_kv_heads, state.config.head_dim)
        pc.ensure(nb, bs, key.dtype, value.dtype, key.device)
    pc.write(key, value, slot_mapping)


def _make_patched_kv_update(orig_fn, state: LayerState, no_alloc: bool = False):
    """K/V writes: the layer's own write (unless no_alloc), then capture
    (smaq/integration/vllm.py:113-130).  Paged layers encode into their pools."""

    def patched(self_impl, layer, key, value, kv_cache, slot_mapping):
        if not no_alloc:
            orig_fn(self_impl, layer, key, value, kv_cache, slot_mapping)
        if _GLOBAL_MODE == MODE_OFF:
            return
        if state.paged is not None:
            _paged_write(state, key, value, kv_cache, slot_mapping)
            return
        _capture(state, key, value, int(slot_mapping.shape[0]))

    return patched


def _no_alloc_prefill_attention(state: LayerState, self_impl, query, key, value, attn_metadata):
    """Causal SDPA over the step's own tokens, GQA by repetition
    (smaq/integration/vllm.py:133-163)."""
    cfg = state.config
    n = attn_metadata.num_actual_tokens
    q, k, v = query[:n], key[:n], value[:n]
    if q.dim() == 2:
        q = q.view(n, cfg.num_query_heads, cfg.head_dim)
    if k.dim() == 2:
        k = k.view(n, cfg.num_kv_heads, cfg.head_dim)
        v = v.view(n, cfg.num_kv_heads, cfg.head_dim)
    if cfg.num_query_heads != cfg.num_kv_heads:
        rep = cfg.num_query_heads // cfg.num_kv_heads
        k = k.repeat_interleave(rep, dim=1)
        v = v.repeat_interleave(rep, dim=1)
    scale = getattr(self_impl, "scale", 1.0 / math.sqrt(cfg.head_dim))
    out = F.scaled_dot_product_attention(q.unsqueeze(0).transpose(1, 2), k.unsqueeze(0).transpose(1, 2),
                                         v.unsqueeze(0).transpose(1, 2), is_causal=True, scale=scale)
    return out.squeeze(0).transpose(0, 1)


def _deliver(result: torch.Tensor, query: torch.Tensor, output: Optional[torch.Tensor], n: int, cfg: LayerConfig):
    """Return a [n, Hq, D] result the way the layer's caller expects it:
    copied into ``output`` when given, else shaped like the query
    (smaq/integration/vllm.py:208-218,245-255)."""
    flat = result.reshape(n, cfg.num_query_heads * cfg.head_dim).to(query.dtype)
    if output is not None:
        dst = output[:n]
        dst.copy_((result if dst.dim() == 3 else flat).to(dst.dtype))
        return output
    return result.to(query.dtype) if query.dim() == 3 else flat


def _paged_decode(state: LayerState, self_impl, query, attn_metadata, output):
    """Whole-batch decode from the paged pools; None when the batch is not a
    pure decode batch this path serves."""
    cfg, pc = state.config, state.paged
    if pc is None or pc.pools is None:
        return None
    seq_lens = getattr(attn_metadata, "seq_lens", None)
    block_table = getattr(attn_metadata, "block_table", None)
    if seq_lens is None or block_table is None:
        return None
    n = attn_metadata.num_actual_tokens
    if int(seq_lens.shape[0]) != n:
        return None
    max_len = getattr(attn_metadata, "max_seq_len", None)
    max_len = int(seq_lens.max()) if max_len is None else int(max_len)
    if max_len < MIN_HISTORY_FOR_SMAQ:
        return None
    q = query[:n].reshape(n, cfg.num_query_heads, cfg.head_dim)
    scale = getattr(self_impl, "scale", None)
    scale = 1.0 / math.sqrt(cfg.head_dim) if scale is None else float(scale)
    if output is not None and output[:n].is_contiguous() and output.dtype == query.dtype:
        dst = output[:n].view(n, cfg.num_query_heads, cfg.head_dim)
        pc.decode(q, block_table, seq_lens, max_len, cfg.num_query_heads, scale, dst)
        return output
    res = torch.empty(n, cfg.num_query_heads, cfg.head_dim, dtype=query.dtype, device=query.device)
    pc.decode(q, block_table, seq_lens, max_len, cfg.num_query_heads, scale, res)
    return _deliver(res, query, output, n, cfg)


def _reference_layout_decode(state: LayerState, self_impl, q: torch.Tensor, flat, query, output):
    """The reference layout's decode step (one store per layer, the exact
    ring as the recent window: smaq/integration/vllm.py:224-255) through a
    plan kept on the layer.  The plan is rebuilt only when the history
    changes (a ring spill, or its columns growing) or the step's shape does;
    otherwise a step sets the ring's fill and launches, writing straight into
    ``output`` when it is a contiguous buffer of the query's dtype.  None
    when the store has no fused kernel description or the ring is empty (the
    caller then takes the one-shot path)."""
    from smaq_amd.score import AttentionPlan, _flat_tensors
    cfg, store, ring = state.config, state.store, state.engine.ring
    fh = getattr(store.quantizer, "fused_history", None)
    fused = fh() if fh is not None else None
    fill = ring.size
    if fused is None or fill == 0:
        return None
    n = q.shape[0]
    scale = getattr(self_impl, "scale", None)
    scale = 1.0 / math.sqrt(cfg.head_dim) if scale is None else float(scale)
    (codes, norms, vdata, vsc, vz), stride = _flat_tensors(flat)
    hist = (codes, norms, vdata, vsc, vz)
    key = (n, q.dtype, q.device, scale, flat.num_tokens, stride,
           tuple(0 if t is None else t.data_ptr() for t in hist), ring._slots_k.data_ptr(), ring.capacity)
    if state.ref_plan_key != key:
        state.ref_plan = AttentionPlan(
            query=q.unsqueeze(0), fused=fused, key_codes=codes, key_norms=norms, val_data=vdata, val_scales=vsc,
            val_zeros=vz, val_bits=store.value_bits, val_group=store.value_group_size, n_kv_heads=store.num_kv_heads,
            hist_len=None, max_hist_len=flat.num_tokens, hist_head_stride=stride,
            recent_k=ring._slots_k.unsqueeze(0), recent_v=ring._slots_v.unsqueeze(0),
            recent_len=torch.full((1,), fill, dtype=torch.int64, device=q.device), max_recent_len=ring.capacity,
            scale=scale, out_dtype=q.dtype, recent_pos_offset=flat.num_tokens)
        state.ref_plan_key = key
    else:
        state.ref_plan.set_lengths(recent_len=fill)
    plan = state.ref_plan
    if output is not None and output.dtype == q.dtype and output[:n].is_contiguous():
        plan.run_into(q.unsqueeze(0), output[:n])
        return output
    return _deliver(plan.run(q.unsqueeze(0)).squeeze(0), query, output, n, cfg)


def _make_patched_forward(orig_fn, state: LayerState, no_alloc: bool = False, capture_in_forward: bool = False):
    """Attention forward with SMAQ serving (smaq/integration/vllm.py:166-272)."""

    def call_orig(self_impl, layer, query, key, value, kv_cache, attn_metadata, output, output_scale,
                  output_block_scale):
        return orig_fn(self_impl, layer, query, key, value, kv_cache, attn_metadata, output, output_scale,
                       output_block_scale)

    def patched(self_impl, layer, query, key, value, kv_cache, attn_metadata, output=None, output_scale=None,
                output_block_scale=None):
        mode = _GLOBAL_MODE
        args = (self_impl, layer, query, key, value, kv_cache, attn_metadata, output, output_scale,
                output_block_scale)
        if capture_in_forward and mode != MODE_OFF and attn_metadata is not None:
            n = getattr(attn_metadata, "num_actual_tokens", key.shape[0])
            if state.paged is not None:
                _paged_write(state, key[:n], value[:n], kv_cache, attn_metadata.slot_mapping[:n])
            else:
                _capture(state, key[:n], value[:n], n)
        if mode in (MODE_OFF, MODE_CAPTURE_ONLY) or attn_metadata is None:
            return call_orig(*args)
        cfg = state.config
        if attn_metadata.max_query_len > 1:
            if no_alloc:
                n = attn_metadata.num_actual_tokens
                res = _no_alloc_prefill_attention(state, self_impl, query, key, value, attn_metadata)
                return _deliver(res, query, output, n, cfg)
            return call_orig(*args)
        if mode == MODE_HYBRID and state.supports_hybrid:
            if state.paged is not None:
                res = _paged_decode(state, self_impl, query, attn_metadata, output)
                if res is not None:
                    return res
            else:
                flat = state.store.get_flat_cache()
                if flat is not None and flat.num_tokens >= MIN_HISTORY_FOR_SMAQ:
                    n = attn_metadata.num_actual_tokens
                    q = query[:n]
                    if q.dim() == 2:
                        q = q.view(n, cfg.num_query_heads, cfg.head_dim)
                    res = _reference_layout_decode(state, self_impl, q, flat, query, output)
                    if res is not None:
                        return res
                    recent = state.engine.ring.peek()
                    res = compute_hybrid_attention(query=q, store=state.store,
                                                   recent_k=recent[0] if recent else None,
                                                   recent_v=recent[1] if recent else None,
                                                   num_query_heads=cfg.num_query_heads,
                                                   scale=getattr(self_impl, "scale", None))
                    return _deliver(res, query, output, n, cfg)
        if no_alloc:
            n = getattr(attn_metadata, "num_actual_tokens", query.shape[0])
            if query.dim() == 3:
                return torch.zeros_like(query[:n])
            return torch.zeros(n, cfg.num_query_heads * cfg.head_dim, dtype=query.dtype, device=query.device)
        return call_orig(*args)

    return patched


def _make_patched_mla_update(orig_fn, state: LayerState):
    """MLA K/V writes pass through; the first one is logged
    (smaq/integration/vllm.py:275-284)."""

    def patched(self_impl, kv_c_normed, k_pe, kv_cache, slot_mapping, kv_cache_dtype, k_scale):
        orig_fn(self_impl, kv_c_normed, k_pe, kv_cache, slot_mapping, kv_cache_dtype, k_scale)
        if state._log_count < 1:
            logger.info("[SMAQ] MLA update observed on layer %s; MLA path is not active yet.", state.config.layer_idx)
            state._log_count += 1

    return patched


def _make_patched_mla_forward(orig_fn, state: LayerState):
    """MLA forward passes through (smaq/integration/vllm.py:287-293)."""

    def patched(self_impl, q, kv_c_and_k_pe_cache, attn_metadata, layer):
        return orig_fn(self_impl, q, kv_c_and_k_pe_cache, attn_metadata, layer)

    return patched


def _bind(impl, name: str, fn) -> None:
    """Replace impl.<name> with fn bound to impl."""
    setattr(impl, name, types.MethodType(lambda self, *a, _p=fn, **kw: _p(self, *a, **kw), impl))


def install_hooks(
    model_runner,
    calibration_covariances: Optional[dict[str, torch.Tensor]] = None,
    key_bits: int = 3,
    value_bits: int = 2,
    value_group_size: int = 32,
    ring_capacity: int = 128,
    initial_layers_count: int = 4,
    initial_layers_key_bits: int | None = None,
    mode: str = MODE_CAPTURE_ONLY,
    no_alloc: bool = False,
    paged: bool = False,
) -> dict[str, LayerState]:
    """Hook every attention layer of the runner's static forward context
    (smaq/integration/vllm.py:296-399).  The first ``initial_layers_count``
    layers use ``initial_layers_key_bits`` (default ``min(key_bits + 1, 4)``).
    ``paged=True`` selects the paged pools for flash layers (module doc)."""
    global _GLOBAL_MODE
    _GLOBAL_MODE = mode
    if initial_layers_key_bits is None:
        initial_layers_key_bits = min(key_bits + 1, 4)
    static_ctx = model_runner.compilation_config.static_forward_context
    device = model_runner.device
    states: dict[str, LayerState] = {}
    layer_idx = 0
    for name, module in static_ctx.items():
        impl = getattr(module, "impl", None)
        if impl is None:
            continue
        hkv = getattr(impl, "num_kv_heads", None)
        if hkv is None:
            continue
        if hasattr(impl, "head_size"):
            head_dim = int(impl.head_size)
        elif hasattr(impl, "kv_lora_rank"):
            head_dim = int(impl.kv_lora_rank)
        else:
            continue
        kind = "mla" if _is_mla_impl(impl) else "flash"
        cfg = LayerConfig(
            head_dim=head_dim, num_kv_heads=int(hkv), num_query_heads=_infer_num_query_heads(module, impl),
            Sigma_q=None if calibration_covariances is None else calibration_covariances.get(name),
            key_bits=initial_layers_key_bits if layer_idx < initial_layers_count else key_bits,
            value_bits=value_bits, value_group_size=min(value_group_size, head_dim), ring_capacity=ring_capacity,
            layer_idx=layer_idx, backend_kind=kind, device=device, paged=paged and kind == "flash")
        state = _create_layer_state(cfg)
        states[name] = state
        if kind == "flash":
            separate_update = hasattr(impl, "do_kv_cache_update")
            if separate_update:
                _bind(impl, "do_kv_cache_update",
                      _make_patched_kv_update(impl.do_kv_cache_update.__func__, state, no_alloc=no_alloc))
            _bind(impl, "forward", _make_patched_forward(impl.forward.__func__, state, no_alloc=no_alloc,
                                                         capture_in_forward=not separate_update))
        else:
            if hasattr(impl, "do_kv_cache_update"):
                _bind(impl, "do_kv_cache_update", _make_patched_mla_update(impl.do_kv_cache_update.__func__, state))
            if hasattr(impl, "forward_mqa"):
                _bind(impl, "forward_mqa", _make_patched_mla_forward(impl.forward_mqa.__func__, state))
        impl._smaq_layer_state = state
        layer_idx += 1
    model_runner._smaq_layer_states = states
    model_runner._smaq_no_alloc = no_alloc
    logger.info("[SMAQ] Hooks installed on %s layers (mode=%s, no_alloc=%s, paged=%s)", len(states), mode,
                no_alloc, paged)
    return states


def free_kv_cache(model_runner) -> int:
    """Replace the paged KV cache tensors of hooked flash layers with a
    one-byte placeholder; returns the bytes released
    (smaq/integration/vllm.py:402-442).  Paged SMAQ layers read their pools,
    not vLLM's cache, so their decode keeps working afterwards."""
    states = getattr(model_runner, "_smaq_layer_states", None)
    if not states:
        logger.warning("[SMAQ] No layer states found, nothing to free")
        return 0
    static_ctx = model_runner.compilation_config.static_forward_context
    tiny = torch.zeros(1, dtype=torch.int8, device=model_runner.device)
    targets = [static_ctx[name] for name, st in states.items() if st.supports_hybrid and name in static_ctx]
    doomed = set()
    freed = 0
    for module in targets:
        kv = getattr(module, "kv_cache", None)
        if kv and len(kv) > 0:
            doomed.add(kv[0].data_ptr())
    for module in targets:
        kv = getattr(module, "kv_cache", None)
        if kv and len(kv) > 0:
            freed += kv[0].nelement() * kv[0].element_size()
            kv[0] = tiny
    caches = model_runner.kv_caches
    for i in range(len(caches)):
        entry = caches[i]
        if isinstance(entry, list):
            for j in range(len(entry)):
                if hasattr(entry[j], "data_ptr") and entry[j].data_ptr() in doomed:
                    entry[j] = tiny
        elif hasattr(entry, "data_ptr") and entry.data_ptr() in doomed:
            caches[i] = tiny
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    logger.info("[SMAQ] Freed %.0f MB KV cache", freed / 1e6)
    return freed


def get_stats(model_runner) -> dict:
    """Per-layer and total token / memory counts (smaq/integration/vllm.py:445-476).
    Paged layers report the tokens written to and the bytes of their pools."""
    states = getattr(model_runner, "_smaq_layer_states", None)
    if not states:
        return {}
    stats = {}
    tot_c = tot_b = tot_m = 0
    for name, st in states.items():
        if st.paged is not None:
            compressed, memory = st.paged.tokens_written, st.paged.memory_bytes()
        else:
            compressed, memory = st.store.num_tokens, st.store.memory_bytes()
        buffered = st.engine.ring.size
        tot_c += compressed
        tot_b += buffered
        tot_m += memory
        stats[name] = {"compressed_tokens": compressed, "buffered_tokens": buffered, "memory_bytes": memory,
                       "supports_hybrid": st.supports_hybrid}
    stats["_totals"] = {"compressed_tokens": tot_c, "buffered_tokens": tot_b, "memory_bytes": tot_m,
                        "layers": len(states)}
    return stats
