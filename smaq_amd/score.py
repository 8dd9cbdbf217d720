"""Hybrid attention over compressed history plus exact recent tokens
(drop-in for smaq/score.py).

``compute_hybrid_attention`` keeps the reference's semantics
(smaq/score.py:23-72): one softmax over the concatenated [history; recent]
logits, history ignored below ``MIN_HISTORY_FOR_SMAQ`` tokens, GQA by head
grouping, each part cast to the query dtype before the sum, zeros when there
is nothing to attend.  For the GPU codecs it is one fused HIP launch sequence
(scores from packed codes, online softmax, in-register value dequantisation);
strategies without a fused description go through their own
``attention_score`` per KV head.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F

from smaq_amd import _native
from smaq_amd.core import AttentionBackend
from smaq_amd.kv_cache import dequantize_values
from smaq_amd.store import CompressedKVStore, FlatCache

MIN_HISTORY_FOR_SMAQ = 16


def _per_sequence_index(t: Optional[torch.Tensor], batch: int, dev: torch.device, what: str):
    """A per-sequence length/start tensor as the kernels read it: int64,
    contiguous, on the attention's device, one entry per sequence.  Callers
    hand in vLLM's int32 ``seq_lens`` or host tensors; both are converted here
    (the kernel dereferences the raw pointer as ``const long long*``)."""
    if t is None:
        return None
    if t.dtype.is_floating_point or t.dtype == torch.bool or t.dtype.is_complex:
        raise ValueError(f"{what} must be an integer tensor, got {t.dtype}")
    t = t.reshape(-1)
    if t.numel() < batch:
        raise ValueError(f"{what} has {t.numel()} entries for {batch} sequences")
    return t[:batch].to(dev, torch.int64).contiguous()


def _own_copy(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    """A private copy of a per-sequence index tensor: the plan's buffer,
    updated in place on re-use, never the caller's tensor."""
    return None if t is None else t.clone()


class AttentionPlan:
    """A prepared fused-attention launch.

    Parameters, workspace, output and the fp32/rotated query buffers are
    allocated once; ``run(query)`` copies the new query in and re-launches.
    Decode loops reuse one plan per step shape, so a step costs the kernel
    launches only.  Shapes: query [B, T, Hq, D]; history fields are
    row-indexed per-token tensors (see include/smaq_hip.h); recent_k/v
    [B, R, Hkv, D].
    """

    def __init__(
        self,
        *,
        query: torch.Tensor,
        fused,
        key_codes: Optional[torch.Tensor],
        key_norms: Optional[torch.Tensor],
        val_data: Optional[torch.Tensor],
        val_scales: Optional[torch.Tensor],
        val_zeros: Optional[torch.Tensor],
        val_bits: int,
        val_group: int,
        n_kv_heads: int,
        hist_len: Optional[torch.Tensor],
        max_hist_len: int,
        hist_seq_start: Optional[torch.Tensor] = None,
        hist_head_stride: int = 0,
        block_table: Optional[torch.Tensor] = None,
        block_size: int = 0,
        recent_k: Optional[torch.Tensor] = None,
        recent_v: Optional[torch.Tensor] = None,
        recent_len: Optional[torch.Tensor] = None,
        max_recent_len: int = 0,
        scale: float,
        out_dtype: torch.dtype,
        query_positions: Optional[torch.Tensor] = None,
        hist_pos_offset: int = 0,
        recent_pos_offset: int = 0,
        impl: int = 0,
    ):
        dev = _native.require_gpu(query, key_codes, val_data, recent_k)
        self.device = dev
        B, T, Hq, D = query.shape
        self.shape = (B, T, Hq, D)
        self.fused = fused
        has_hist = fused is not None and max_hist_len > 0
        has_recent = recent_k is not None and max_recent_len > 0
        p = _native.AttnParams()
        p.batch, p.q_len, p.n_q_heads, p.n_kv_heads, p.head_dim = B, T, Hq, n_kv_heads, D
        p.scale = float(scale)
        p.impl = int(impl)   # 0 auto, 1 generic, 2 matrix-core decode, 3 matrix-core prefill
        keep = []
        self.q_exact = torch.empty(B, T, Hq, D, dtype=torch.float32, device=dev)
        p.q_exact = self.q_exact.data_ptr()
        if query_positions is not None:
            if query_positions.numel() != B * T or query_positions.dtype.is_floating_point:
                raise ValueError(f"query_positions must be {B * T} integer positions ([batch, q_len])")
            qp = query_positions.to(dev, torch.int64).contiguous()
            self._positions = qp
            p.q_positions = qp.data_ptr()
        p.hist_pos_offset = int(hist_pos_offset)
        p.recent_pos_offset = int(recent_pos_offset)
        self.q_hist = None
        self.rot_t = None
        self._q_raw = None
        self.hist_len = None        # the plan's own per-sequence length buffers
        self.recent_len = None      # (int64; updated in place by set_lengths)
        self._block_table = None
        self._recent = None         # (keys, values) the plan reads; rebound by set_recent
        if has_hist:
            if fused.rot_t is not None:
                # The library rotates the raw query itself (inside the decode
                # kernel when that kernel serves the call, else by one launch
                # into q_hist).
                self.q_hist = torch.empty_like(self.q_exact)
                self.rot_t = fused.rot_t.to(dev, torch.float32).contiguous()
                self.rot_scale = None if fused.rot_scale is None else fused.rot_scale.to(dev, torch.float32).contiguous()
                p.q_hist = self.q_hist.data_ptr()
                p.rot_mt = self.rot_t.data_ptr()
                p.rot_scale = None if self.rot_scale is None else self.rot_scale.data_ptr()
            else:
                p.q_hist = self.q_exact.data_ptr()
            # split arrival counters (zero; every call leaves them zero): the
            # decode kernel merges its own splits, no combine launch
            self.arrivals = torch.zeros(B * n_kv_heads, dtype=torch.int32, device=dev)
            p.arrivals = self.arrivals.data_ptr()
            p.has_history = 1
            p.key_bytes = key_codes.data_ptr()
            p.key_row_bytes = key_codes.shape[-1]
            lut = fused.lut.to(dev, torch.float32).contiguous().reshape(-1)
            if fused.kind == "scalar" and lut.numel() < (1 << fused.bits):
                lut = torch.cat([lut, lut.new_zeros((1 << fused.bits) - lut.numel())])
            keep.append(lut)
            p.key_lut = lut.data_ptr()
            if fused.kind == "scalar":
                p.key_format = _native.KEY_SCALAR
                p.key_bits = fused.bits
                p.key_norms = key_norms.data_ptr()
                p.norm_dtype = _native.dtype_code(key_norms.dtype)
            else:
                p.key_format = _native.KEY_BLOCKVQ
                p.vq_blocks, p.vq_block_dim, p.vq_centroids = fused.n_blocks, fused.block_dim, fused.n_centroids
            p.val_bytes = val_data.data_ptr()
            p.val_row_bytes = val_data.shape[-1]
            # rows the pools hold (the decode kernel's range-checked value
            # addressing); 0 when the value array is not one dense block
            p.hist_rows = val_data.numel() // max(1, val_data.shape[-1]) if val_data.is_contiguous() else 0
            p.val_bits, p.val_group = val_bits, val_group
            p.val_scales, p.val_zeros = val_scales.data_ptr(), val_zeros.data_ptr()
            p.val_dtype = _native.dtype_code(val_scales.dtype)
            hist_len = _own_copy(_per_sequence_index(hist_len, B, dev, "hist_len"))
            hist_seq_start = _per_sequence_index(hist_seq_start, B, dev, "hist_seq_start")
            self.hist_len = hist_len
            p.hist_len = None if hist_len is None else hist_len.data_ptr()
            p.hist_seq_start = None if hist_seq_start is None else hist_seq_start.data_ptr()
            p.hist_head_stride = int(hist_head_stride)
            if block_table is not None:
                if block_table.dim() != 2 or block_table.shape[0] < B or block_table.dtype.is_floating_point:
                    raise ValueError(f"block_table must be an integer [>= {B}, max_blocks] tensor, "
                                     f"got {tuple(block_table.shape)} {block_table.dtype}")
                bt = block_table[:B].to(dev, torch.int32).contiguous()
                self._block_table = bt
                p.block_table = bt.data_ptr()
                p.max_blocks = bt.shape[-1]
                p.block_size = int(block_size)
            p.max_hist_len = int(max_hist_len)
            keep += [t for t in (key_codes, key_norms, val_data, val_scales, val_zeros, hist_len, hist_seq_start)
                     if t is not None]
        if has_recent:
            rk, rv = recent_k.contiguous(), recent_v.contiguous()
            recent_len = _own_copy(_per_sequence_index(recent_len, B, dev, "recent_len"))
            self.recent_len = recent_len
            self._recent = (rk, rv)
            p.has_recent = 1
            p.recent_k, p.recent_v = rk.data_ptr(), rv.data_ptr()
            p.recent_dtype = _native.dtype_code(rk.dtype)
            p.recent_len = None if recent_len is None else recent_len.data_ptr()
            p.recent_batch_stride = rk.shape[1] * rk.shape[2] * rk.shape[3]
            p.max_recent_len = int(max_recent_len)
        self.out = torch.empty(B, T, Hq, D, dtype=out_dtype, device=dev)
        p.out = self.out.data_ptr()
        p.out_dtype = _native.dtype_code(out_dtype)
        nbytes = _native.attn_workspace_bytes(p)
        self.workspace = torch.empty(max(nbytes, 4), dtype=torch.uint8, device=dev)
        p.workspace = self.workspace.data_ptr()
        p.workspace_bytes = self.workspace.numel()
        self.params = p
        self._keep = keep

    def load_query(self, query: torch.Tensor) -> None:
        """Hand a query to the plan.  With a rotated codec the library reads
        the query as given (fp32/fp16/bf16, contiguous, 16-byte aligned;
        anything else is copied to fp32 first): it rotates it for the history
        and the recent window reads it directly, so no copy is made.  An
        unrotated codec scores the fp32 copy."""
        q = query.reshape(self.shape)
        if self.rot_t is not None:
            if q.device != self.device:
                q = q.to(self.device)
            if (q.dtype not in (torch.float32, torch.float16, torch.bfloat16) or not q.is_contiguous()
                    or q.data_ptr() % 16):
                q = q.to(torch.float32).clone(memory_format=torch.contiguous_format)
            self._q_raw = q  # kept alive until the next load
            self.params.q_raw = q.data_ptr()
            self.params.q_raw_dtype = _native.dtype_code(q.dtype)
        else:
            self.q_exact.copy_(q)

    def launch(self, phases: int = 0) -> torch.Tensor:
        """Launch the attention phases on the current stream: 0 = all, else a
        mask of 8 (query rotation), 1 (history), 2 (recent), 4 (combine), and
        16 (the history phase reuses the decode schedule an earlier call built
        for the same lengths: the decode kernel alone)."""
        self.params.phases = phases
        _native.attn_hybrid(self.params, self.device)
        return self.out

    def run(self, query: torch.Tensor) -> torch.Tensor:
        self.load_query(query)
        return self.launch()

    # -- re-use across steps: a serving loop keeps one plan per batch shape
    # and rebinds what changes from step to step (lengths, block table,
    # output), so a step allocates nothing and costs its launches only.

    def set_lengths(self, hist_len=None, recent_len=None) -> None:
        """Copy new per-sequence lengths (an integer tensor with >= B entries,
        or one int for every sequence) into the plan's own buffers; the plan
        must have been built with lengths of that kind.  Lengths above the
        plan's maxima are clamped by the kernels."""
        B = self.shape[0]
        for new, own, what in ((hist_len, self.hist_len, "hist_len"), (recent_len, self.recent_len, "recent_len")):
            if new is None:
                continue
            if own is None:
                raise ValueError(f"plan was built without per-sequence {what}")
            if isinstance(new, int):
                own.fill_(new)
                continue
            if new.dtype.is_floating_point or new.dtype == torch.bool or new.reshape(-1).numel() < B:
                raise ValueError(f"{what} must be an integer tensor with >= {B} entries")
            own.copy_(new.reshape(-1)[:B])

    def set_block_table(self, block_table: torch.Tensor) -> None:
        """Point the plan at a block table of the shape it was built with
        ([>= B, max_blocks] integer; copied only if not int32, contiguous and
        on the plan's device)."""
        if self._block_table is None:
            raise ValueError("plan was built without a block table")
        B, mb = self._block_table.shape
        if block_table.dim() != 2 or block_table.shape[0] < B or block_table.shape[1] != mb \
                or block_table.dtype.is_floating_point:
            raise ValueError(f"block_table must be an integer [>= {B}, {mb}] tensor, got "
                             f"{tuple(block_table.shape)} {block_table.dtype}")
        bt = block_table[:B].to(self.device, torch.int32).contiguous()
        self._block_table = bt
        self.params.block_table = bt.data_ptr()

    def set_recent(self, recent_k: torch.Tensor, recent_v: torch.Tensor) -> None:
        """Point the plan at another exact recent window of the shape and
        dtype it was built with ([B, R, Hkv, D]; copied only if not
        contiguous)."""
        if self._recent is None:
            raise ValueError("plan was built without a recent window")
        rk0 = self._recent[0]
        for t in (recent_k, recent_v):
            if t.shape != rk0.shape or t.dtype != rk0.dtype or t.device != rk0.device:
                raise ValueError(f"recent window {tuple(t.shape)} {t.dtype} on {t.device} does not match the plan's "
                                 f"{tuple(rk0.shape)} {rk0.dtype} on {rk0.device}")
        rk, rv = recent_k.contiguous(), recent_v.contiguous()
        self._recent = (rk, rv)
        self.params.recent_k, self.params.recent_v = rk.data_ptr(), rv.data_ptr()

    def set_query_positions(self, query_positions: torch.Tensor) -> None:
        """New causal positions ([batch, q_len] integers) for a plan built
        with positions."""
        if getattr(self, "_positions", None) is None:
            raise ValueError("plan was built without query positions")
        if query_positions.numel() != self._positions.numel() or query_positions.dtype.is_floating_point:
            raise ValueError(f"query_positions must be {self._positions.numel()} integer positions")
        qp = query_positions.to(self.device, torch.int64).contiguous()
        self._positions = qp
        self.params.q_positions = qp.data_ptr()

    def run_into(self, query: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        """``run`` writing the result straight into ``out`` (contiguous, the
        plan's output dtype and element count, on its device); returns out."""
        if (out.dtype != self.out.dtype or out.numel() != self.out.numel() or not out.is_contiguous()
                or out.device != self.device):
            raise ValueError(f"out must be a contiguous {self.out.dtype} tensor of {self.out.numel()} elements "
                             f"on {self.device}")
        self.load_query(query)
        self.params.out = out.data_ptr()
        try:
            _native.attn_hybrid(self.params, self.device)
        finally:
            self.params.out = self.out.data_ptr()
        return out


def launch_fused_attention(*, query: torch.Tensor, **kw) -> torch.Tensor:
    """One-shot fused attention; returns [B, T, Hq, D] in out_dtype."""
    return AttentionPlan(query=query, **kw).run(query)


def _head_stride_rows(t: torch.Tensor):
    """Rows between KV heads of a [Hkv, N, *tail] per-token tensor whose rows
    are dense, or None if its rows are not laid out that way."""
    per_row = 1
    for s in t.shape[2:]:
        per_row *= s
    dense_rows = t.stride(1) == per_row and (t.dim() == 2 or t[0, 0].is_contiguous())
    if not dense_rows or t.stride(0) % per_row:
        return None
    return t.stride(0) // per_row


def _flat_tensors(flat: FlatCache):
    """The FlatCache's per-token tensors plus their common head stride in rows
    (copied to contiguous tensors when the views disagree)."""
    kq, vq = flat.key_q, flat.value_q
    norms = getattr(kq, "norms", None)
    tensors = [kq.indices, norms, vq.data, vq.scales, vq.zeros]
    strides = {_head_stride_rows(t) for t in tensors if t is not None}
    if len(strides) == 1 and None not in strides:
        return tensors, strides.pop()
    return [None if t is None else t.contiguous() for t in tensors], flat.num_tokens


def plan_hybrid_attention(
    query: torch.Tensor,
    store: CompressedKVStore,
    recent_k: Optional[torch.Tensor],
    recent_v: Optional[torch.Tensor],
    num_query_heads: int,
    scale: Optional[float] = None,
    query_positions: Optional[torch.Tensor] = None,
    impl: int = 0,
) -> Optional[AttentionPlan]:
    """The fused launch ``compute_hybrid_attention`` makes for these inputs,
    prepared but not run (a caller that repeats the same shape re-runs it);
    None when the reference semantics need no fused launch (nothing to attend,
    or a strategy without a fused kernel description)."""
    head_dim = store.head_dim
    hkv = store.num_kv_heads
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    flat = store.get_flat_cache()
    has_history = flat is not None and flat.num_tokens >= MIN_HISTORY_FOR_SMAQ
    has_recent = recent_k is not None and recent_k.shape[0] > 0
    if not has_history and not has_recent:
        return None
    if num_query_heads % hkv:
        raise ValueError(f"num_query_heads {num_query_heads} not a multiple of num_kv_heads {hkv}")
    fused = None
    if has_history:
        fh = getattr(store.quantizer, "fused_history", None)
        fused = fh() if fh is not None else None
        if fused is None:
            return None
    n_all = flat.num_tokens if flat is not None else 0
    if has_history:
        (codes, norms, vdata, vsc, vz), stride = _flat_tensors(flat)
        kw = dict(key_codes=codes, key_norms=norms, val_data=vdata, val_scales=vsc, val_zeros=vz,
                  hist_head_stride=stride, max_hist_len=flat.num_tokens)
    else:
        kw = dict(key_codes=None, key_norms=None, val_data=None, val_scales=None, val_zeros=None,
                  max_hist_len=0)
    return AttentionPlan(
        query=query.unsqueeze(0), fused=fused, val_bits=store.value_bits, val_group=store.value_group_size,
        n_kv_heads=hkv, hist_len=None,
        recent_k=recent_k.unsqueeze(0) if has_recent else None,
        recent_v=recent_v.unsqueeze(0) if has_recent else None,
        recent_len=None, max_recent_len=recent_k.shape[0] if has_recent else 0,
        scale=scale, out_dtype=query.dtype,
        query_positions=None if query_positions is None else query_positions.reshape(1, -1),
        hist_pos_offset=0, recent_pos_offset=n_all, impl=impl, **kw)


def _store_plan(query, store, recent_k, recent_v, num_query_heads, scale, query_positions, impl):
    """The fused plan for these inputs, kept on the store between calls: a
    repeated call with the same query shape, the same history (token count
    and column buffers) and a recent window of the same shape rebinds the
    window and positions and launches, without rebuilding the plan."""
    flat = store.get_flat_cache()
    has_recent = recent_k is not None and recent_k.shape[0] > 0
    hist_key = None
    if flat is not None and flat.num_tokens >= MIN_HISTORY_FOR_SMAQ:
        (codes, norms, vdata, vsc, vz), stride = _flat_tensors(flat)
        hist_key = (flat.num_tokens, stride, tuple(0 if t is None else t.data_ptr() for t in
                                                   (codes, norms, vdata, vsc, vz)))
    key = (tuple(query.shape), query.dtype, query.device, num_query_heads, scale, impl, query_positions is None,
           hist_key, None if not has_recent else (tuple(recent_k.shape), recent_k.dtype, recent_k.device))
    cached = getattr(store, "_fused_plan", None)
    if cached is not None and cached[0] == key:
        plan = cached[1]
        if has_recent:
            plan.set_recent(recent_k.unsqueeze(0), recent_v.unsqueeze(0))
        if query_positions is not None:
            plan.set_query_positions(query_positions.reshape(1, -1))
        return plan
    plan = plan_hybrid_attention(query, store, recent_k, recent_v, num_query_heads, scale, query_positions, impl)
    try:
        store._fused_plan = (key, plan) if plan is not None else None
    except AttributeError:
        pass  # a store type that takes no attributes: no caching
    return plan


def compute_hybrid_attention(
    query: torch.Tensor,
    store: CompressedKVStore,
    recent_k: Optional[torch.Tensor],
    recent_v: Optional[torch.Tensor],
    num_query_heads: int,
    scale: Optional[float] = None,
    query_positions: Optional[torch.Tensor] = None,
    impl: int = 0,
) -> torch.Tensor:
    """Attention of query [T, Hq, D] over the store's history and the exact
    recent window [R, Hkv, D] (smaq/score.py:23-72).

    ``query_positions`` (int64 [T], optional) is an extension for chunked
    prefill: key j (history positions 0..N-1, then recent N..N+R-1) is visible
    to query t iff j <= query_positions[t].  None reproduces the reference,
    which applies no mask.  ``impl`` picks the kernels (0 automatic,
    1 generic, 2 matrix-core decode, 3 matrix-core prefill).
    """
    plan = _store_plan(query, store, recent_k, recent_v, num_query_heads, scale, query_positions, impl)
    if plan is not None:
        out = torch.empty(query.shape[0], num_query_heads, store.head_dim, dtype=query.dtype, device=plan.device)
        return plan.run_into(query.unsqueeze(0), out)
    flat = store.get_flat_cache()
    has_history = flat is not None and flat.num_tokens >= MIN_HISTORY_FOR_SMAQ
    has_recent = recent_k is not None and recent_k.shape[0] > 0
    if not has_history and not has_recent:
        return torch.zeros(query.shape[0], num_query_heads, store.head_dim, device=query.device, dtype=query.dtype)
    if num_query_heads % store.num_kv_heads:
        raise ValueError(f"num_query_heads {num_query_heads} not a multiple of num_kv_heads {store.num_kv_heads}")
    return _generic_hybrid(query, store, flat, recent_k, recent_v, num_query_heads,
                           1.0 / math.sqrt(store.head_dim) if scale is None else scale, has_recent, query_positions)


def _generic_hybrid(query, store, flat, recent_k, recent_v, num_query_heads, scale, has_recent,
                    query_positions):
    """Strategies without a fused kernel description: the reference's per-head
    composition (smaq/score.py:61-72,75-124) in GPU tensor ops."""
    hkv = store.num_kv_heads
    g = num_query_heads // hkv
    T, D = query.shape[0], query.shape[-1]
    q = query.float().view(T, hkv, g, D).permute(1, 2, 0, 3)
    kwargs = {"use_kernel": True} if getattr(store.quantizer, "supports_kernel", False) else {}
    per_head = [store.quantizer.attention_score(q[h], store.quantizer.select_head(flat.key_q, h), scale=scale,
                                                **kwargs) for h in range(hkv)]
    parts = [torch.stack(per_head, 0).permute(2, 0, 1, 3).reshape(T, num_query_heads, flat.num_tokens)]
    if has_recent:
        k = recent_k.transpose(0, 1).float().unsqueeze(1)
        s = torch.matmul(q, k.transpose(-2, -1).contiguous()) * scale
        parts.append(s.permute(2, 0, 1, 3).reshape(T, num_query_heads, recent_k.shape[0]))
    logits = torch.cat(parts, dim=-1)
    if query_positions is not None:
        pos = torch.arange(logits.shape[-1], device=logits.device)
        logits = logits.masked_fill((pos[None, :] > query_positions.to(logits.device)[:, None])[:, None, :],
                                    float("-inf"))
    w = F.softmax(logits, dim=-1)

    def apply(weights, values):
        v = values.float().unsqueeze(1)
        wv = weights.float().view(T, hkv, g, weights.shape[-1]).permute(1, 2, 0, 3)
        o = torch.matmul(wv, v)
        return o.permute(2, 0, 1, 3).reshape(T, num_query_heads, D).to(query.dtype)

    n = flat.num_tokens
    o_h = apply(w[..., :n], dequantize_values(flat.value_q, store.value_group_size))
    if not has_recent:
        return o_h
    return o_h + apply(w[..., n:], recent_v.transpose(0, 1))


class HybridAttentionBackend(AttentionBackend):
    """Attention backend over compressed history and exact tail
    (smaq/score.py:141-160)."""

    def compute(self, query, store, recent_k, recent_v, num_query_heads, scale: Optional[float] = None):
        return compute_hybrid_attention(query=query, store=store, recent_k=recent_k, recent_v=recent_v,
                                        num_query_heads=num_query_heads, scale=scale)
