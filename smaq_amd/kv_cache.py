"""Value codec re-exports and the standalone SMAQ KV cache (drop-in for
smaq/kv_cache.py).

``SMAQKVCache`` keeps the newest ``buffer_size`` tokens of a ``[..., T, D]``
key/value stream exact and the older ones compressed.  Its compressed part is
a ``ColumnHistory`` (one lane per leading index, e.g. batch x head): a flush
encodes the tokens leaving the exact window straight into the columns' tail
rows.  The exact window lives in a buffer twice its size in which tokens
occupy a sliding range: appends write at the end, flushes advance the start,
and the range is moved to the front only when the end reaches the buffer's
capacity -- a copy of ``buffer_size`` tokens once per ``buffer_size``
appended tokens.  (The reference concatenates the whole exact buffer on every
append and the whole compressed history on every flush,
smaq/kv_cache.py:176-216.)
"""

from __future__ import annotations

import math
from typing import Any, Optional

import torch

from smaq_amd import _native
from smaq_amd.calibration import IdentityCalibrationProvider
from smaq_amd.columns import ColumnHistory, codec_kind
from smaq_amd.core import CacheCapabilities, CalibrationProvider
from smaq_amd.quantizer import default_device
from smaq_amd.strategies import SMAQFullMetricScalarStrategy
from smaq_amd.value_codec import (ValueQuantized, dequantize_values, quantize_values,  # noqa: F401
                                  unpack_values)


class _ExactWindow:
    """The newest tokens of a [*lead, T, D] stream, in order, as a view of a
    buffer of twice the window size."""

    def __init__(self):
        self.k: Optional[torch.Tensor] = None
        self.v: Optional[torch.Tensor] = None
        self.start = self.end = 0

    @property
    def size(self) -> int:
        return self.end - self.start

    def views(self):
        if self.k is None or self.size == 0:
            return None, None
        return self.k[..., self.start:self.end, :], self.v[..., self.start:self.end, :]

    def push(self, key: torch.Tensor, value: torch.Tensor, window: int) -> None:
        t = key.shape[-2]
        if self.k is None:
            cap = max(2 * window, t)
            self.k = key.new_empty(*key.shape[:-2], cap, key.shape[-1])
            self.v = value.new_empty(*value.shape[:-2], cap, value.shape[-1])
        elif key.shape[:-2] != self.k.shape[:-2] or key.shape[-1] != self.k.shape[-1]:
            raise ValueError(f"appended keys {tuple(key.shape)} do not continue the cache's "
                             f"{tuple(self.k.shape[:-2])} x {self.k.shape[-1]} stream")
        if key.dtype != self.k.dtype or value.dtype != self.v.dtype:
            # widen, as concatenating tensors of two float dtypes does
            self.k = self.k.to(torch.promote_types(self.k.dtype, key.dtype))
            self.v = self.v.to(torch.promote_types(self.v.dtype, value.dtype))
        if self.end + t > self.k.shape[-2]:
            n = self.size
            cap = max(self.k.shape[-2], n + t)
            k2 = self.k.new_empty(*self.k.shape[:-2], cap, self.k.shape[-1])
            v2 = self.v.new_empty(*self.v.shape[:-2], cap, self.v.shape[-1])
            k2[..., :n, :].copy_(self.k[..., self.start:self.end, :])
            v2[..., :n, :].copy_(self.v[..., self.start:self.end, :])
            self.k, self.v, self.start, self.end = k2, v2, 0, n
        self.k[..., self.end:self.end + t, :].copy_(key)
        self.v[..., self.end:self.end + t, :].copy_(value)
        self.end += t

    def pop_front(self, n: int):
        """Views of the oldest n tokens; they leave the window (the views stay
        valid until the next push)."""
        k, v = self.k[..., self.start:self.start + n, :], self.v[..., self.start:self.start + n, :]
        self.start += n
        return k, v


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
        if key_strategy is None:
            sigma = Sigma_q if Sigma_q is not None else self.calibration_provider.get_sigma_q(
                layer_idx, head_dim, device=self.device)
            key_strategy = SMAQFullMetricScalarStrategy(dim=head_dim, Sigma_q=sigma, bits=key_bits,
                                                        device=self.device, dtype=torch.float32)
        self.key_quantizer = key_strategy
        self.seq_len = 0
        self._lead: Optional[tuple[int, ...]] = None
        self._hist: Optional[ColumnHistory] = None
        # strategies without a column encoder keep quantised chunks
        self._chunks: list[tuple[Any, ValueQuantized]] = []
        self._joined: Optional[tuple[Any, ValueQuantized]] = None
        self._exact = _ExactWindow()

    @property
    def capabilities(self) -> CacheCapabilities:
        return self.key_quantizer.capabilities

    # -- compressed history ------------------------------------------------
    @property
    def key_quantized(self):
        if self._hist is not None:
            return self._hist.key_quantized(self._lead)
        joined = self._join()
        return None if joined is None else joined[0]

    @property
    def value_quantized(self) -> Optional[ValueQuantized]:
        if self._hist is not None:
            return self._hist.value_quantized(self._lead)
        joined = self._join()
        return None if joined is None else joined[1]

    def _join(self):
        if not self._chunks:
            return None
        if self._joined is None:
            ks = [k for k, _ in self._chunks]
            vs = [v for _, v in self._chunks]
            key_q = ks[0] if len(ks) == 1 else self.key_quantizer.concat_quantized(ks)
            val_q = vs[0] if len(vs) == 1 else ValueQuantized(
                data=torch.cat([v.data for v in vs], dim=-2), scales=torch.cat([v.scales for v in vs], dim=-2),
                zeros=torch.cat([v.zeros for v in vs], dim=-2), bits=self.value_bits)
            self._joined = (key_q, val_q)
        return self._joined

    def _compress(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Append [*lead, n, D] tokens to the compressed history."""
        if keys.shape[-2] == 0:
            return
        lead = tuple(keys.shape[:-2])
        if self._lead is None:
            self._lead = lead
        elif lead != self._lead:
            raise ValueError(f"keys with leading shape {lead} do not continue the cache's {self._lead}")
        if self._hist is None and not self._chunks and codec_kind(self.key_quantizer) is not None:
            lanes = math.prod(lead) if lead else 1
            self._hist = ColumnHistory(self.key_quantizer, lanes, self.head_dim, self.value_bits,
                                       self.value_group_size, self.device)
        if self._hist is not None:
            d = keys.shape[-1]
            self._hist.append([(keys.reshape(-1, keys.shape[-2], d), values.reshape(-1, values.shape[-2], d))])
        else:
            self._chunks.append((self.key_quantizer.quantize(keys),
                                 quantize_values(values, bits=self.value_bits, group_size=self.value_group_size)))
            self._joined = None

    # -- exact window --------------------------------------------------------
    @property
    def key_buffer(self) -> Optional[torch.Tensor]:
        return self._exact.views()[0]

    @property
    def value_buffer(self) -> Optional[torch.Tensor]:
        return self._exact.views()[1]

    # -- cache protocol (smaq/kv_cache.py:154-290) -------------------------
    def prefill(self, keys: torch.Tensor, values: torch.Tensor):
        """Compress all but the newest ``buffer_size`` tokens, keep those exact
        (smaq/kv_cache.py:154-174)."""
        n = keys.shape[-2]
        self.seq_len = n
        n_old = max(0, n - self.buffer_size)
        # a prefill replaces the exact window, and the compressed history too
        # when it compresses tokens (the reference assigns both)
        self._exact = _ExactWindow()
        if n_old:
            self._lead, self._hist, self._chunks, self._joined = None, None, [], None
        self._compress(keys[..., :n_old, :], values[..., :n_old, :])
        self._exact.push(keys[..., n_old:, :], values[..., n_old:, :], self.buffer_size)

    def append(self, key: torch.Tensor, value: torch.Tensor):
        """Add tokens to the exact window; whatever no longer fits in
        ``buffer_size`` is compressed (smaq/kv_cache.py:176-216)."""
        self.seq_len += key.shape[-2]
        self._exact.push(key, value, self.buffer_size)
        over = self._exact.size - self.buffer_size
        if over > 0:
            self._compress(*self._exact.pop_front(over))

    def attention_scores(self, query: torch.Tensor, scale: float | None = None) -> torch.Tensor:
        """[compressed, exact] scores along the key axis, no softmax
        (smaq/kv_cache.py:218-241)."""
        if scale is None:
            scale = 1.0 / math.sqrt(self.head_dim)
        parts = []
        kq = self.key_quantized
        if kq is not None:
            kw = {"use_kernel": True} if getattr(self.key_quantizer, "supports_kernel", False) else {}
            parts.append(self.key_quantizer.attention_score(query, kq, scale=scale, **kw))
        kb = self.key_buffer
        if kb is not None:
            # (a contiguous right operand: batched bf16 products of a transposed view are avoided)
            parts.append(torch.matmul(query, kb.transpose(-2, -1).contiguous()) * scale)
        if not parts:
            return query.new_empty(*query.shape[:-2], query.shape[-2], 0)
        return torch.cat(parts, dim=-1)

    def attend(self, attn_weights: torch.Tensor) -> torch.Tensor:
        """Weights over [compressed, exact] applied to the dequantised and the
        exact values (smaq/kv_cache.py:243-267)."""
        out = None
        col = 0
        vq = self.value_quantized
        if vq is not None:
            nq = vq.data.shape[-2]
            w = attn_weights[..., col:col + nq]
            bits = vq.bits if len(vq) > 3 else 2
            if (w.is_cuda and w.dtype == torch.float32 and w.shape[:-2] == vq.data.shape[:-2]
                    and _native.apply_values_supported(self.head_dim, bits, self.value_group_size)):
                # the packed codes decoded inside the weighted sum: no fp32
                # value rows (512 B per token-head at D = 128) are written
                out = _native.apply_values(w, vq.data, vq.scales, vq.zeros, bits, self.value_group_size)
            else:
                out = torch.matmul(w, dequantize_values(vq, self.value_group_size))
            col += nq
        vb = self.value_buffer
        if vb is not None:
            part = torch.matmul(attn_weights[..., col:col + vb.shape[-2]], vb)
            out = part if out is None else out + part
        if out is None:
            return attn_weights.new_zeros(*attn_weights.shape[:-1], self.head_dim)
        return out

    def memory_bytes(self) -> dict[str, int]:
        """Byte accounting with 16-bit metadata and 2-byte exact elements
        (smaq/kv_cache.py:269-287)."""
        kq, vq = self.key_quantized, self.value_quantized
        keys = self.key_quantizer.memory_bytes(kq) if kq is not None else 0
        vals = 0 if vq is None else vq.data.nelement() + 2 * vq.scales.nelement() + 2 * vq.zeros.nelement()
        kb, vb = self.key_buffer, self.value_buffer
        buf = 0 if kb is None else 2 * (kb.nelement() + vb.nelement())
        return {"quantized_keys": keys, "quantized_values": vals, "buffer": buf, "total": keys + vals + buf}

    def allocated_bytes(self) -> int:
        """Device bytes held (not in the reference): the compressed columns at
        their capacity (up to twice the filled rows) or the quantised chunks,
        plus the exact window's buffers (twice the window: it slides through
        one buffer and compacts when it reaches the end)."""
        def nb(t):
            return 0 if t is None else t.nelement() * t.element_size()
        hist = self._hist.allocated_bytes() if self._hist is not None else 0
        for kq, vq in self._chunks:
            hist += sum(nb(t) for t in (kq if isinstance(kq, tuple) else ()) if isinstance(t, torch.Tensor))
            hist += nb(vq.data) + nb(vq.scales) + nb(vq.zeros)
        return hist + nb(self._exact.k) + nb(self._exact.v)

    def get_seq_length(self) -> int:
        return self.seq_len
