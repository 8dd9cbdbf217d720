"""Append-only compressed history in per-field GPU columns.

The fused attention kernels read the history as per-token rows of five fields
(key codes, key norms, value bytes, value scales, value zeros), head-major:
row (lane, t) of a field lives at ``lane * capacity + t``.  ``ColumnHistory``
keeps each field as one ``[lanes, capacity, *tail]`` buffer (a lane is one KV
head of one sequence) and appends by encoding the new tokens of every lane
straight into rows ``[n, n + T)`` with the HIP key codec and value packer:
the encoders take an output row stride, so there is no intermediate
quantised chunk and no copy.  When a buffer is full its capacity doubles (one
copy of the filled rows, amortised O(1) per token).

The reference keeps a list of quantised chunks and re-concatenates all of
them on the first read after every append (smaq/store.py:83-114,
smaq/kv_cache.py:190-216); both of its consumers sit on this class here.
"""

from __future__ import annotations

from typing import Any, Optional, Sequence

import torch

from smaq_amd.block_vq import BlockVQQuantized, SMAQBlockVQ
from smaq_amd.value_codec import ValueQuantized, pack_values_into
from smaq_amd.quantizer import SMAQQuantized, SMAQQuantizer
from smaq_amd.weighted_scalar import RotationAdapter

_MIN_CAPACITY = 256


def codec_kind(strategy: Any) -> Optional[str]:
    """'scalar' or 'block_vq' when the strategy's codec can encode into
    columns, else None (the caller keeps quantised chunks instead)."""
    qz = getattr(strategy, "quantizer", None)
    if isinstance(qz, (SMAQQuantizer, RotationAdapter)):
        return "scalar"
    if isinstance(qz, SMAQBlockVQ):
        return "block_vq"
    return None


class ColumnHistory:
    """Compressed history of ``lanes`` independent (sequence, KV head) lanes,
    all holding the same number of tokens ``n``."""

    def __init__(self, strategy: Any, lanes: int, head_dim: int, value_bits: int, value_group: int,
                 device: torch.device):
        self.kind = codec_kind(strategy)
        if self.kind is None:
            raise ValueError(f"{type(strategy).__name__} has no column encoder")
        self.strategy = strategy
        self.lanes, self.head_dim = lanes, head_dim
        self.value_bits, self.value_group = value_bits, value_group
        self.device = device
        self.n = 0
        self.capacity = 0
        self._bufs: dict[str, torch.Tensor] = {}
        self._dtypes: Optional[tuple[torch.dtype, torch.dtype]] = None   # (key, value) storage dtypes

    # -- layout -----------------------------------------------------------
    def _fields(self, kdt: torch.dtype, vdt: torch.dtype) -> dict[str, tuple[tuple[int, ...], torch.dtype]]:
        D = self.head_dim
        qz = self.strategy.quantizer
        vpb = 4 if self.value_bits == 2 else (2 if self.value_bits == 4 else 1)
        f = {}
        if self.kind == "scalar":
            kvpb = max(1, 8 // qz.bits)
            f["k_codes"] = ((-(-D // kvpb),), torch.uint8)
            f["k_norms"] = ((), kdt)
        else:
            f["k_codes"] = ((qz.n_blocks,), torch.uint8)
        f["v_data"] = ((D // vpb,), torch.uint8)
        f["v_scales"] = ((D // self.value_group,), vdt)
        f["v_zeros"] = ((D // self.value_group,), vdt)
        return f

    def _reserve(self, need: int) -> None:
        if need <= self.capacity:
            return
        cap = max(need, 2 * self.capacity, _MIN_CAPACITY)
        for name, (tail, dt) in self._fields(*self._dtypes).items():
            grown = torch.empty((self.lanes, cap, *tail), dtype=dt, device=self.device)
            old = self._bufs.get(name)
            if old is not None and self.n:
                grown[:, :self.n].copy_(old[:, :self.n])
            self._bufs[name] = grown
        self.capacity = cap

    def _promote(self, kdt: torch.dtype, vdt: torch.dtype) -> bool:
        """Chunks of another float dtype than the columns': widen the columns
        to the promoted dtype (fp16 + bf16 -> fp32, exact), as concatenating
        the reference's chunks would.  Returns True when the new chunk must be
        encoded in its own dtype and converted (the kernels write the key /
        value dtype)."""
        ck, cv = self._dtypes
        if (kdt, vdt) == (ck, cv):
            return False
        pk, pv = torch.promote_types(ck, kdt), torch.promote_types(cv, vdt)
        if (pk, pv) != (ck, cv):
            for name, (tail, dt) in self._fields(pk, pv).items():
                if self._bufs[name].dtype != dt:
                    self._bufs[name] = self._bufs[name].to(dt)
            self._dtypes = (pk, pv)
        return True

    # -- append -----------------------------------------------------------
    def append(self, parts: Sequence[tuple[torch.Tensor, torch.Tensor]]) -> int:
        """Encode the pieces (each keys, values [lanes, T_i, D]) in order into
        rows [n, n + sum T_i) of every lane.  Returns the reference's byte
        count for the appended tokens (key strategy bytes + value bytes with
        16-bit metadata, smaq/store.py:116-124)."""
        parts = [(k, v) for k, v in parts if k.shape[1] > 0]
        if not parts:
            return 0
        kdt, vdt = parts[0][0].dtype, parts[0][1].dtype
        if self._dtypes is None:
            self._dtypes = (kdt, vdt)
        T = sum(k.shape[1] for k, _ in parts)
        self._reserve(self.n + T)
        off = self.n
        nbytes = 0
        for k, v in parts:
            if k.shape[0] != self.lanes or v.shape[:2] != k.shape[:2]:
                raise ValueError(f"chunk rows {tuple(k.shape[:2])} / {tuple(v.shape[:2])} do not match "
                                 f"{self.lanes} lanes")
            t = k.shape[1]
            convert = self._promote(k.dtype, v.dtype)
            views = {name: buf[:, off:off + t] for name, buf in self._bufs.items()}
            if convert:
                tmp = {name: torch.empty(view.shape, dtype=view.dtype if view.dtype == torch.uint8 else
                                         (k.dtype if name == "k_norms" else v.dtype), device=self.device)
                       for name, view in views.items()}
                self._encode(k, v, tmp)
                for name, view in views.items():
                    view.copy_(tmp[name])
            else:
                self._encode(k, v, views)
            nbytes += self._bytes(views)
            off += t
        self.n += T
        return nbytes

    def _encode(self, k: torch.Tensor, v: torch.Tensor, out: dict[str, torch.Tensor]) -> None:
        qz = self.strategy.quantizer
        if self.kind == "scalar":
            qz.encode_into(k, out["k_codes"], out["k_norms"])
        else:
            qz.encode_into(k, out["k_codes"])
        pack_values_into(v, self.value_bits, self.value_group, out["v_data"], out["v_scales"], out["v_zeros"])

    def _bytes(self, views: dict[str, torch.Tensor]) -> int:
        kq = self._key_q(views, self.strategy.quantizer)
        vb = views["v_data"].nelement() + 2 * views["v_scales"].nelement() + 2 * views["v_zeros"].nelement()
        return self.strategy.memory_bytes(kq) + vb

    # -- read -------------------------------------------------------------
    def _key_q(self, f: dict[str, torch.Tensor], qz):
        if self.kind == "scalar":
            return SMAQQuantized(indices=f["k_codes"], norms=f["k_norms"], bits=qz.bits)
        return BlockVQQuantized(indices=f["k_codes"], n_blocks=qz.n_blocks, block_dim=qz.block_dim)

    def allocated_bytes(self) -> int:
        """Device bytes the column buffers hold: every field at ``capacity``
        rows, which is up to twice the filled rows (capacity doubles when a
        buffer is full; a grow holds the old and the new buffer until the
        copy is done)."""
        return sum(buf.nelement() * buf.element_size() for buf in self._bufs.values())

    def filled(self, lead: Optional[tuple[int, ...]] = None) -> dict[str, torch.Tensor]:
        """Rows [0, n) of every field, [lanes, n, *tail] (or [*lead, n, *tail]
        with prod(lead) == lanes; views, nothing is copied)."""
        out = {}
        for name, buf in self._bufs.items():
            view = buf[:, :self.n]
            out[name] = view if lead is None else view.reshape(*lead, *view.shape[1:])
        return out

    def key_quantized(self, lead: Optional[tuple[int, ...]] = None):
        return self._key_q(self.filled(lead), self.strategy.quantizer) if self.n else None

    def value_quantized(self, lead: Optional[tuple[int, ...]] = None) -> Optional[ValueQuantized]:
        if not self.n:
            return None
        f = self.filled(lead)
        return ValueQuantized(data=f["v_data"], scales=f["v_scales"], zeros=f["v_zeros"], bits=self.value_bits)
