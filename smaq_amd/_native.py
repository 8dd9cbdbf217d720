"""ctypes binding of libsmaq_hip.so (the C ABI declared in include/smaq_hip.h).

This is the only module that talks to the native library.  Every op here
validates its tensors, allocates outputs with torch on the tensors' device,
launches on torch's current stream and maps a non-zero status to an
exception: ``ValueError`` for invalid arguments (the reference's own error
type for bad shapes), ``RuntimeError`` for anything else.  There is no second
code path: if the library is missing, or a tensor is not on a GPU, the call
raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # imported before the library so one HIP runtime is shared

_LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libsmaq_hip.so"
_lib = None

F32, F16, BF16 = 0, 1, 2
_DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}
KEY_SCALAR, KEY_BLOCKVQ = 0, 1

c_void_p, c_int, c_ll, c_float = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_float
c_ull_p = ctypes.POINTER(ctypes.c_ulonglong)


class AttnParams(ctypes.Structure):
    """Mirror of ``smaq_attn_params`` (include/smaq_hip.h)."""

    _fields_ = [
        ("batch", c_int), ("q_len", c_int), ("n_q_heads", c_int), ("n_kv_heads", c_int),
        ("head_dim", c_int), ("scale", c_float),
        ("q_hist", c_void_p), ("q_exact", c_void_p), ("q_positions", c_void_p),
        ("has_history", c_int), ("key_format", c_int), ("key_bytes", c_void_p),
        ("key_row_bytes", c_int), ("key_bits", c_int), ("key_norms", c_void_p),
        ("norm_dtype", c_int), ("key_lut", c_void_p),
        ("vq_blocks", c_int), ("vq_block_dim", c_int), ("vq_centroids", c_int),
        ("val_bytes", c_void_p), ("val_row_bytes", c_int), ("val_bits", c_int),
        ("val_group", c_int), ("val_scales", c_void_p), ("val_zeros", c_void_p),
        ("val_dtype", c_int),
        ("hist_len", c_void_p), ("hist_seq_start", c_void_p), ("hist_head_stride", c_ll),
        ("block_table", c_void_p), ("max_blocks", c_int), ("block_size", c_int),
        ("hist_pos_offset", c_ll),
        ("has_recent", c_int), ("recent_k", c_void_p), ("recent_v", c_void_p),
        ("recent_dtype", c_int), ("recent_len", c_void_p), ("recent_batch_stride", c_ll),
        ("recent_pos_offset", c_ll),
        ("out", c_void_p), ("out_dtype", c_int),
        ("workspace", c_void_p), ("workspace_bytes", c_ll),
        ("max_hist_len", c_ll), ("max_recent_len", c_ll),
        ("phases", c_int), ("impl", c_int),
        ("arrivals", c_void_p),
        ("q_raw", c_void_p), ("q_raw_dtype", c_int), ("rot_mt", c_void_p), ("rot_scale", c_void_p),
        ("hist_rows", c_ll),
    ]


_SIGS = {
    "smaq_version": (c_int, []),
    "smaq_last_error": (ctypes.c_char_p, []),
    "smaq_pack_values": (c_int, [c_void_p, c_int, c_ll, c_ll, c_ll, c_ll, c_ll, c_int, c_int, c_int,
                                 c_void_p, c_void_p, c_void_p, c_void_p]),
    "smaq_dequant_values": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_ll, c_int, c_int,
                                    c_int, c_void_p, c_void_p]),
    "smaq_encode_scalar": (c_int, [c_void_p, c_int, c_ll, c_ll, c_ll, c_ll, c_ll, c_int, c_void_p,
                                   c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p,
                                   c_void_p, c_void_p]),
    "smaq_rotate_rows": (c_int, [c_void_p, c_int, c_ll, c_int, c_void_p, c_void_p, c_void_p,
                                 c_void_p]),
    "smaq_dequant_scalar": (c_int, [c_void_p, c_void_p, c_int, c_ll, c_int, c_int, c_void_p,
                                    c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    "smaq_scores_scalar": (c_int, [c_void_p, c_ll, c_ll, c_ll, c_int, c_void_p, c_int, c_void_p,
                                   c_int, c_void_p, c_int, c_float, c_void_p, c_int, c_void_p]),
    "smaq_encode_blockvq": (c_int, [c_void_p, c_int, c_ll, c_ll, c_ll, c_ll, c_ll, c_int, c_int, c_int,
                                    c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "smaq_dequant_blockvq": (c_int, [c_void_p, c_ll, c_int, c_int, c_int, c_void_p, c_void_p,
                                     c_void_p]),
    "smaq_blockvq_shape": (c_int, [c_void_p, c_int, c_ll, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "smaq_kmeanspp_update": (c_int, [c_void_p, c_int, c_ll, c_int, c_void_p, c_int, c_void_p, c_void_p]),
    "smaq_kmeans_update": (c_int, [c_void_p, c_void_p, c_int, c_ll, c_int, c_int, c_void_p, c_void_p]),
    "smaq_attn_workspace_bytes": (c_ll, [ctypes.POINTER(AttnParams)]),
    "smaq_attn_hybrid": (c_int, [ctypes.POINTER(AttnParams), c_void_p]),
    "smaq_attn_hybrid_noalloc": (c_int, [ctypes.POINTER(AttnParams), c_void_p]),
    "smaq_probe_read": (c_int, [c_void_p, c_ll, c_void_p, c_void_p]),
    "smaq_apply_values_workspace_bytes": (c_ll, [c_ll, c_ll, c_ll, c_int]),
    "smaq_apply_values": (c_int, [c_void_p, c_ll, c_ll, c_ll, c_ll, c_ll, c_int, c_void_p, c_ll, c_int, c_int,
                                  c_void_p, c_void_p, c_ll, c_int, c_void_p, c_void_p, c_ll, c_void_p]),
}

# Size of the built-in workspace of smaq_attn_hybrid_noalloc
# (SMAQ_NOALLOC_SCRATCH_BYTES in include/smaq_hip.h).
NOALLOC_SCRATCH_BYTES = 32 << 20

EXPORTED = tuple(_SIGS)


def library_path() -> Path:
    return _LIB_PATH


def lib():
    """Loads libsmaq_hip.so once; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise RuntimeError(
                f"smaq_amd native library missing at {_LIB_PATH}; build it with "
                "`python -m smaq_amd.csrc.build` (hipcc --offload-arch=gfx950)")
        handle = ctypes.CDLL(str(_LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def _check(status: int, what: str) -> None:
    if status == 0:
        return
    msg = lib().smaq_last_error().decode(errors="replace")
    if status == -1:
        raise ValueError(msg or f"{what}: invalid argument")
    raise RuntimeError(f"{what} failed ({status}): {msg}")


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise ValueError(f"unsupported dtype {dt}; expected float32, float16 or bfloat16") from None


def require_gpu(*tensors) -> torch.device:
    """All tensors must live on one GPU: the kernels have no CPU path."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(
                "smaq_amd runs its codecs and attention as HIP kernels; got a tensor on "
                f"{t.device}. Move inputs to the GPU (cuda device).")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def row_view(x: torch.Tensor):
    """Express x[..., D] (last dim contiguous) as rows r = o * n_inner + i at
    offset o * s_outer + i * s_inner.  Returns None if no such 2-level form
    exists (the caller then makes the tensor contiguous)."""
    if x.dim() == 0 or x.stride(-1) != 1:
        return None
    lead = [(s, st) for s, st in zip(x.shape[:-1], x.stride()[:-1]) if s != 1]
    if not lead:
        return 1, 1, 0, 0
    # merge dims that are already contiguous with each other
    merged = [list(lead[0])]
    for s, st in lead[1:]:
        ps, pst = merged[-1]
        if pst == s * st:
            merged[-1] = [ps * s, st]
        else:
            merged.append([s, st])
    if len(merged) == 1:
        (n, st), = merged
        return 1, n, 0, st
    if len(merged) == 2:
        (no, so), (ni, si) = merged
        return no, ni, so, si
    return None


def _rows_args(x: torch.Tensor):
    rv = row_view(x)
    if rv is None:
        x = x.contiguous()
        rv = row_view(x)
    return x, rv


def _column_rows(x: torch.Tensor, outs):
    """Row mapping for an encode whose outputs are views into per-head
    columns: x is [O, I, D] (last dim contiguous), every output is [O, I,
    *tail] with a dense tail, consecutive rows along I and O-rows a common
    multiple apart (a [Hkv, capacity, ...] column sliced to its tail rows).
    Returns (x, (O, I, s_outer, s_inner), out_outer) with out_outer the
    output rows between consecutive O (0 when O == 1: dense)."""
    if x.dim() != 3:
        raise ValueError(f"encode into columns takes [O, I, D] input, got {tuple(x.shape)}")
    if x.stride(-1) != 1:
        x = x.contiguous()
    O, I = x.shape[0], x.shape[1]
    out_outer = None
    for t in outs:
        if t is None:
            continue
        if tuple(t.shape[:2]) != (O, I):
            raise ValueError(f"output view {tuple(t.shape)} does not match the input rows [{O}, {I}]")
        row = 1
        for s in t.shape[2:]:
            row *= s
        tail_ok = t.dim() == 2 or t[0, 0].is_contiguous()
        if not tail_ok or (I > 1 and t.stride(1) != row) or (O > 1 and t.stride(0) % row):
            raise ValueError("output view rows must be dense along the token dim")
        oo = t.stride(0) // row if O > 1 else 0
        if out_outer is None:
            out_outer = oo
        elif oo != out_outer:
            raise ValueError("output views disagree on their head stride")
    if out_outer is not None and O > 1 and out_outer < I:
        raise ValueError("output views overlap (head stride below the token count)")
    return x, (O, I, x.stride(0), x.stride(1)), (out_outer or 0)


# ---------------------------------------------------------------- values ---

def _value_row_bytes(D: int, bits: int) -> int:
    return D // (4 if bits == 2 else (2 if bits == 4 else 1))


def pack_values(v: torch.Tensor, bits: int, group_size: int, out=None):
    """quantize_values on the GPU -> (data u8 [..., D/vpb], scales, zeros [..., D/G]).
    With ``out`` = (data, scales, zeros) column views (see ``_column_rows``)
    the packed rows are written there instead and ``out`` is returned."""
    dev = require_gpu(v, *(out or ()))
    D = v.shape[-1]
    if D % group_size != 0:
        raise ValueError(f"head_dim {D} must be divisible by group_size {group_size}")
    lead = v.shape[:-1]
    vpb = 4 if bits == 2 else (2 if bits == 4 else 1)
    if D % vpb != 0:
        raise ValueError(f"head_dim {D} must be divisible by {vpb} for {bits}-bit packing")
    if out is None:
        v, (no, ni, so, si) = _rows_args(v)
        oo = 0
        data = torch.empty(*lead, D // vpb, dtype=torch.uint8, device=dev)
        scales = torch.empty(*lead, D // group_size, dtype=v.dtype, device=dev)
        zeros = torch.empty_like(scales)
    else:
        data, scales, zeros = out
        if (data.dtype != torch.uint8 or scales.dtype != v.dtype or zeros.dtype != v.dtype
                or data.shape[-1] != D // vpb or scales.shape[-1] != D // group_size or zeros.shape != scales.shape):
            raise ValueError("pack_values: output views of the wrong dtype or width")
        v, (no, ni, so, si), oo = _column_rows(v, out)
    _check(lib().smaq_pack_values(_ptr(v), dtype_code(v.dtype), no, ni, so, si, oo, D, bits, group_size,
                                  _ptr(data), _ptr(scales), _ptr(zeros), _stream(dev)),
           "smaq_pack_values")
    return data, scales, zeros


def dequant_values(data, scales, zeros, bits: int, group_size: int) -> torch.Tensor:
    dev = require_gpu(data, scales, zeros)
    data, scales, zeros = data.contiguous(), scales.contiguous(), zeros.contiguous()
    vpb = 4 if bits == 2 else (2 if bits == 4 else 1)
    D = data.shape[-1] * vpb
    rows = data.numel() // max(1, data.shape[-1])
    out = torch.empty(*data.shape[:-1], D, dtype=torch.float32, device=dev)
    _check(lib().smaq_dequant_values(_ptr(data), _ptr(scales), _ptr(zeros), dtype_code(scales.dtype),
                                     rows, D, bits, group_size, _ptr(out), _stream(dev)),
           "smaq_dequant_values")
    return out


def apply_values_supported(D: int, bits: int, group_size: int) -> bool:
    """Whether smaq_apply_values takes this value layout: a row of D codes is
    a power-of-two number (<= 64) of 4-byte words, each inside one group."""
    vpb = 4 if bits == 2 else (2 if bits == 4 else 1)
    dpl = 4 * vpb
    if not (1 <= bits <= 8 and 0 < D <= 512 and group_size > 0 and D % group_size == 0 and D % dpl == 0):
        return False
    lanes = D // dpl
    return lanes <= 64 and lanes & (lanes - 1) == 0 and group_size % dpl == 0


def apply_values(w: torch.Tensor, data: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, bits: int,
                 group_size: int) -> torch.Tensor:
    """w [*lead, nq, N] fp32 applied to packed values data [*lead, N, D/vpb]
    (scales, zeros [*lead, N, D/group]) -> [*lead, nq, D] fp32, the value
    rows decoded on the fly.  Row-dense views with the lead dims a fixed stride
    apart (column buffers) are read in place."""
    dev = require_gpu(w, data, scales, zeros)
    if w.dtype != torch.float32:
        raise ValueError(f"apply_values: weights must be float32, got {w.dtype}")
    if scales.dtype != zeros.dtype or scales.shape != zeros.shape:
        raise ValueError("apply_values: scales and zeros differ in dtype or shape")
    lead, (nq, N) = tuple(w.shape[:-2]), tuple(w.shape[-2:])
    if tuple(data.shape[:-2]) != lead or data.shape[-2] != N or tuple(scales.shape[:-1]) != tuple(data.shape[:-1]):
        raise ValueError(f"apply_values: weights {tuple(w.shape)} do not match values {tuple(data.shape)}")
    vpb = 4 if bits == 2 else (2 if bits == 4 else 1)
    rb, ng = data.shape[-1], scales.shape[-1]
    D = rb * vpb
    if ng * group_size != D:
        raise ValueError(f"apply_values: {ng} groups of {group_size} do not cover head_dim {D}")
    batch = 1
    for x in lead:
        batch *= int(x)
    out = torch.empty(*lead, nq, D, dtype=torch.float32, device=dev)
    if batch == 0 or nq == 0:
        return out
    w3 = w.reshape(batch, nq, N)
    if N > 1 and w3.stride(2) != 1:
        w3 = w3.contiguous()
    d3 = data.reshape(batch, N, rb)
    if d3.stride(2) != 1 or (N > 1 and d3.stride(1) != rb):
        d3 = d3.contiguous()
    s3, z3 = scales.reshape(batch, N, ng), zeros.reshape(batch, N, ng)
    if (s3.stride() != z3.stride() or s3.stride(2) != 1 or (N > 1 and s3.stride(1) != ng)):
        s3, z3 = s3.contiguous(), z3.contiguous()
    ws_bytes = lib().smaq_apply_values_workspace_bytes(batch, nq, N, D)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes > 0 else None
    _check(lib().smaq_apply_values(_ptr(w3), w3.stride(0), w3.stride(1), batch, nq, N, D, _ptr(d3), d3.stride(0),
                                   bits, group_size, _ptr(s3), _ptr(z3), s3.stride(0), dtype_code(s3.dtype),
                                   _ptr(out), _ptr(ws), max(ws_bytes, 0), _stream(dev)),
           "smaq_apply_values")
    return out


# ---------------------------------------------------------------- scalar ---

class TieCounter:
    """Device-side counter the encoders add boundary/argmin ties into."""

    def __init__(self, device):
        self.t = torch.zeros(1, dtype=torch.int64, device=device)

    def ptr(self):
        return ctypes.c_void_p(self.t.data_ptr())

    def value(self) -> int:
        return int(self.t.item())


def encode_scalar(k: torch.Tensor, Mt: torch.Tensor, bounds: torch.Tensor, bits: int,
                  coord_scales: torch.Tensor | None = None, ties: TieCounter | None = None, out=None):
    """Scalar key encoder -> (packed codes u8 [..., ceil(D/vpb)], norms [...] in k.dtype).
    With ``out`` = (codes, norms) column views (see ``_column_rows``) the rows
    are written there instead and ``out`` is returned."""
    dev = require_gpu(k, Mt, bounds, coord_scales, *(out or ()))
    D = k.shape[-1]
    lead = k.shape[:-1]
    vpb = max(1, 8 // bits)
    if out is None:
        k, (no, ni, so, si) = _rows_args(k)
        oo = 0
        codes = torch.empty(*lead, (D + vpb - 1) // vpb, dtype=torch.uint8, device=dev)
        norms = torch.empty(lead, dtype=k.dtype, device=dev)
    else:
        codes, norms = out
        if codes.dtype != torch.uint8 or codes.shape[-1] != (D + vpb - 1) // vpb or norms.dtype != k.dtype:
            raise ValueError("encode_scalar: output views of the wrong dtype or width")
        k, (no, ni, so, si), oo = _column_rows(k, out)
    Mt = Mt.to(torch.float32).contiguous()
    bounds = bounds.to(torch.float32).contiguous()
    cs = None if coord_scales is None else coord_scales.to(torch.float32).contiguous()
    _check(lib().smaq_encode_scalar(_ptr(k), dtype_code(k.dtype), no, ni, so, si, oo, D, _ptr(Mt), _ptr(cs),
                                    _ptr(bounds), bounds.numel(), bits, _ptr(codes), _ptr(norms),
                                    ties.ptr() if ties else None, _stream(dev)),
           "smaq_encode_scalar")
    return codes, norms


def rotate_rows(x: torch.Tensor, Mt: torch.Tensor, coord_scales: torch.Tensor | None = None):
    """(x @ M^T) [* coord_scales] in fp32, Mt = M^T contiguous."""
    dev = require_gpu(x, Mt, coord_scales)
    D = x.shape[-1]
    xc = x.contiguous()
    mt = Mt.to(torch.float32).contiguous()
    out = torch.empty(*x.shape[:-1], Mt.shape[1], dtype=torch.float32, device=dev)
    cs = None if coord_scales is None else coord_scales.to(torch.float32).contiguous()
    _check(lib().smaq_rotate_rows(_ptr(xc), dtype_code(xc.dtype), xc.numel() // max(D, 1), D, _ptr(mt),
                                  _ptr(cs), _ptr(out), _stream(dev)), "smaq_rotate_rows")
    return out


def rotate_rows_into(x: torch.Tensor, Mt: torch.Tensor, coord_scales, out: torch.Tensor) -> None:
    """In-place variant of rotate_rows: x contiguous, out fp32 of x's shape."""
    D = x.shape[-1]
    _check(lib().smaq_rotate_rows(_ptr(x), dtype_code(x.dtype), x.numel() // max(D, 1), D, _ptr(Mt),
                                  _ptr(coord_scales), _ptr(out), _stream(x.device)), "smaq_rotate_rows")


def dequant_scalar(codes, norms, bits: int, D: int, centroids, Mt, inv_scales=None,
                   out_dtype=torch.float32):
    dev = require_gpu(codes, norms, centroids, Mt, inv_scales)
    codes, norms = codes.contiguous(), norms.contiguous()
    cents = centroids.to(torch.float32).contiguous()
    mt = Mt.to(torch.float32).contiguous()
    rows = norms.numel()
    out = torch.empty(*norms.shape, D, dtype=out_dtype, device=dev)
    inv = None if inv_scales is None else inv_scales.to(torch.float32).contiguous()
    _check(lib().smaq_dequant_scalar(_ptr(codes), _ptr(norms), dtype_code(norms.dtype), rows, D, bits,
                                     _ptr(cents), _ptr(inv), _ptr(mt), _ptr(out), dtype_code(out_dtype),
                                     _stream(dev)), "smaq_dequant_scalar")
    return out


def scores_scalar(qrot: torch.Tensor, codes: torch.Tensor, norms: torch.Tensor, bits: int,
                  centroids: torch.Tensor, scale, out_dtype):
    """qrot [B, nq, D] fp32, codes [B, N, P], norms [B, N] -> [B, nq, N]."""
    dev = require_gpu(qrot, codes, norms, centroids)
    B, nq, D = qrot.shape
    N = codes.shape[1]
    # bind every converted copy to a name: its storage must outlive the launch
    q, c, n = qrot.contiguous(), codes.contiguous(), norms.contiguous()
    cents = centroids.to(torch.float32).contiguous()
    out = torch.empty(B, nq, N, dtype=out_dtype, device=dev)
    _check(lib().smaq_scores_scalar(_ptr(q), B, nq, N, D, _ptr(c), bits, _ptr(n), dtype_code(n.dtype),
                                    _ptr(cents), 0 if scale is None else 1,
                                    0.0 if scale is None else float(scale), _ptr(out), dtype_code(out_dtype),
                                    _stream(dev)), "smaq_scores_scalar")
    return out


# -------------------------------------------------------------- block VQ ---

def encode_blockvq(k: torch.Tensor, E_blocks: torch.Tensor, centroids: torch.Tensor,
                   ties: TieCounter | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Block-VQ key encoder -> uint8 indices [..., n_blocks].  With ``out``
    an index column view (see ``_column_rows``) the rows are written there
    instead and ``out`` is returned."""
    dev = require_gpu(k, E_blocks, centroids, out)
    nb, nc, bd = centroids.shape
    if k.shape[-1] != nb * bd:
        raise ValueError(f"key dim {k.shape[-1]} != n_blocks * block_dim = {nb * bd}")
    lead = k.shape[:-1]
    if out is None:
        k, (no, ni, so, si) = _rows_args(k)
        oo = 0
        idx = torch.empty(*lead, nb, dtype=torch.uint8, device=dev)
    else:
        if out.dtype != torch.uint8 or out.shape[-1] != nb:
            raise ValueError("encode_blockvq: output view of the wrong dtype or width")
        k, (no, ni, so, si), oo = _column_rows(k, (out,))
        idx = out
    eb = E_blocks.to(torch.float32).contiguous()
    cents = centroids.to(torch.float32).contiguous()
    _check(lib().smaq_encode_blockvq(_ptr(k), dtype_code(k.dtype), no, ni, so, si, oo, nb, bd, nc, _ptr(eb),
                                     _ptr(cents), _ptr(idx), ties.ptr() if ties else None, _stream(dev)),
           "smaq_encode_blockvq")
    return idx


def blockvq_shape(k: torch.Tensor, E_blocks: torch.Tensor) -> torch.Tensor:
    """Shaped calibration keys: k [N, nb * bd] -> x [nb, N, bd] fp32 (x = k_b E_b^T)."""
    dev = require_gpu(k, E_blocks)
    nb, bd, _ = E_blocks.shape
    if k.dim() != 2 or k.shape[1] != nb * bd:
        raise ValueError(f"keys must be [N, {nb * bd}], got {tuple(k.shape)}")
    kc = k.contiguous()
    eb = E_blocks.to(torch.float32).contiguous()
    x = torch.empty(nb, k.shape[0], bd, dtype=torch.float32, device=dev)
    _check(lib().smaq_blockvq_shape(_ptr(kc), dtype_code(kc.dtype), kc.shape[0], nb, bd, _ptr(eb), _ptr(x),
                                    _stream(dev)), "smaq_blockvq_shape")
    return x


def kmeanspp_update(x: torch.Tensor, pick: torch.Tensor, dmin: torch.Tensor, first: bool) -> None:
    """dmin [nb, N] <- (first ? d : min(dmin, d)), d = squared distance to x[b][pick[b]]."""
    dev = require_gpu(x, pick, dmin)
    nb, n, bd = x.shape
    if pick.shape != (nb,) or dmin.shape != (nb, n) or dmin.dtype != torch.float32 or not dmin.is_contiguous():
        raise ValueError("kmeanspp_update: pick must be [n_blocks], dmin a contiguous fp32 [n_blocks, N]")
    pk = pick.to(torch.int64).contiguous()
    xc = x.contiguous()
    _check(lib().smaq_kmeanspp_update(_ptr(xc), nb, n, bd, _ptr(pk), 1 if first else 0, _ptr(dmin), _stream(dev)),
           "smaq_kmeanspp_update")


def kmeans_update(x: torch.Tensor, idx: torch.Tensor, centroids: torch.Tensor) -> None:
    """centroids [nb, nc, bd] <- per-cluster means of x [nb, N, bd] under idx [N, nb] (in place)."""
    dev = require_gpu(x, idx, centroids)
    nb, n, bd = x.shape
    nc = centroids.shape[1]
    if (idx.shape != (n, nb) or idx.dtype != torch.uint8 or centroids.shape != (nb, nc, bd)
            or centroids.dtype != torch.float32 or not centroids.is_contiguous()):
        raise ValueError("kmeans_update: idx must be uint8 [N, n_blocks], centroids contiguous fp32 "
                         "[n_blocks, n_centroids, block_dim]")
    xc, ic = x.contiguous(), idx.contiguous()
    _check(lib().smaq_kmeans_update(_ptr(xc), _ptr(ic), nb, n, bd, nc, _ptr(centroids), _stream(dev)),
           "smaq_kmeans_update")


def dequant_blockvq(idx: torch.Tensor, decoded: torch.Tensor) -> torch.Tensor:
    dev = require_gpu(idx, decoded)
    nb, nc, bd = decoded.shape
    if idx.dtype != torch.uint8:
        if int(idx.max()) > 255 or int(idx.min()) < 0:
            raise ValueError("block-VQ indices must be in [0, 255]")
        idx = idx.to(torch.uint8)
    idx = idx.contiguous()
    dec = decoded.to(torch.float32).contiguous()
    rows = idx.numel() // nb
    out = torch.empty(*idx.shape[:-1], nb * bd, dtype=torch.float32, device=dev)
    _check(lib().smaq_dequant_blockvq(_ptr(idx), rows, nb, bd, nc, _ptr(dec), _ptr(out), _stream(dev)),
           "smaq_dequant_blockvq")
    return out


# ------------------------------------------------------------- attention ---

def attn_workspace_bytes(p: AttnParams) -> int:
    n = lib().smaq_attn_workspace_bytes(ctypes.byref(p))
    if n < 0:
        raise ValueError("invalid attention parameters")
    return int(n)


def attn_hybrid(p: AttnParams, device: torch.device) -> None:
    """Launches the fused attention described by p (workspace already set)."""
    _check(lib().smaq_attn_hybrid(ctypes.byref(p), _stream(device)), "smaq_attn_hybrid")


def probe_read(x: torch.Tensor, sink: torch.Tensor) -> None:
    """Streaming read of x's bytes (smaq_probe_read), launched on the current
    stream; sink is a 4-byte-or-larger device tensor the probe may write."""
    require_gpu(x, sink)
    if not x.is_contiguous():
        raise ValueError("probe_read needs a contiguous tensor")
    nbytes = x.numel() * x.element_size() // 16 * 16
    _check(lib().smaq_probe_read(_ptr(x), nbytes, _ptr(sink), _stream(x.device)), "smaq_probe_read")


def attn_hybrid_noalloc(p: AttnParams, device: torch.device) -> None:
    """Launches the fused attention described by p with the library's
    built-in per-GPU workspace (p.workspace is ignored; nothing is allocated).
    Raises ValueError when the shapes need more than NOALLOC_SCRATCH_BYTES.
    Calls that overlap on one GPU share that workspace and race."""
    _check(lib().smaq_attn_hybrid_noalloc(ctypes.byref(p), _stream(device)), "smaq_attn_hybrid_noalloc")
