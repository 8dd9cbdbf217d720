"""The value bit-packer (drop-in for the value half of smaq/kv_cache.py).

Per group of ``group_size`` elements: asymmetric min/max quantisation to
``bits`` bits (scale = max((max - min) / (2^bits - 1), 1e-10), zero = min,
code = clamp(round_half_even((v - zero) / scale)), every op rounded to the
value dtype), 2-bit codes packed four per byte and 4-bit codes two per byte,
low bits first.  Packing and dequantisation are HIP kernels.
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from smaq_amd import _native


class ValueQuantized(NamedTuple):
    """Bit-packed values (smaq/kv_cache.py:20-26)."""

    data: torch.Tensor
    scales: torch.Tensor
    zeros: torch.Tensor
    bits: int = 2


def _bits(vq: ValueQuantized) -> int:
    return vq.bits if len(vq) > 3 else 2


def unpack_values(vq: ValueQuantized) -> torch.Tensor:
    """Per-element uint8 codes from the packed bytes (smaq/kv_cache.py:29-47):
    field j of byte p is element vpb * p + j."""
    bits = _bits(vq)
    p = vq.data
    vpb = 4 if bits == 2 else (2 if bits == 4 else 1)
    if vpb == 1:
        return p
    shifts = torch.arange(0, 8, bits, dtype=torch.uint8, device=p.device)
    return ((p.unsqueeze(-1) >> shifts) & ((1 << bits) - 1)).reshape(*p.shape[:-1], p.shape[-1] * vpb)


def quantize_values(v: torch.Tensor, bits: int = 2, group_size: int = 32) -> ValueQuantized:
    """Groupwise asymmetric quantisation (smaq/kv_cache.py:50-91), HIP kernel."""
    data, scales, zeros = _native.pack_values(v, bits, group_size)
    return ValueQuantized(data=data, scales=scales, zeros=zeros, bits=bits)


def pack_values_into(v: torch.Tensor, bits: int, group_size: int, data: torch.Tensor, scales: torch.Tensor,
                     zeros: torch.Tensor) -> None:
    """quantize_values of v [lanes, T, D] written into column views
    [lanes, T, ...] (rows dense per lane, lanes a fixed stride apart)."""
    _native.pack_values(v, bits, group_size, out=(data, scales, zeros))


def dequantize_values(vq: ValueQuantized, group_size: int = 32) -> torch.Tensor:
    """fp32 code * scale + zero (smaq/kv_cache.py:94-103), HIP kernel."""
    return _native.dequant_values(vq.data, vq.scales, vq.zeros, _bits(vq), group_size)
