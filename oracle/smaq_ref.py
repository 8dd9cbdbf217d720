"""Torch-CPU restatement of the reference SMAQ hot path (test infrastructure).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py`` for who may import it.

Every function below restates, op for op and on CPU tensors, one piece of the
reference (``/root/reference/smaq/...``, cited per function).  "Op for op"
matters: the reference's exact bits come from torch-CPU kernels, so the
restatement uses the same torch ops in the same order, on the same dtypes.
The CPU semantics these ops have on this torch build (2.10, MKL) were pinned
by running torch itself:

* ``A @ B`` (fp32, >= 6 rows) accumulates each output with a sequential FMA
  chain over k = 0..K-1 (MKL sgemm micro-kernel order).
* ``x.norm(dim=-1)`` (fp32) accumulates squares into 8 FMA partial sums
  (element d -> partial d % 8), adds the partials left to right, then takes a
  correctly rounded sqrt.  bf16/fp16 inputs accumulate in fp32 the same way.
* ``x.pow(2).sum(-1)`` over 8 elements: sequential, multiply then add.
* ``Tensor.sqrt`` (vectorised) is monotone but not correctly rounded
  (<= 0.56 ulp); it only matters inside ``cdist`` where it can merge two
  nearly equal squared distances (a counted argmin tie).
* bf16/fp16 elementwise ops compute in fp32 and round once (RNE) to the
  tensor dtype; ``clamp(min=1e-10)`` converts the bound to the tensor dtype.

PINNING -- what checks each function (tests/test_oracle_*.py):

* pack_codes / unpack_codes: brute-force bit loop on small inputs + round trip.
* scalar_tables / midpoint_tables: scipy.stats.norm.ppf closed form (1e-6),
  ordering and symmetry invariants.
* build_metric / ssf_log: diagonal-Sigma closed form, E @ E_inv = I,
  det(E) = 1 (volume normalisation), symmetry of E^2 eigenvalues.
* fit_sigma_centered: numpy's biased covariance (np.cov bias=True) with a
  mean offset that the uncentred and the N-1 forms visibly miss; one- and
  two-row closed forms; shift invariance.
* smaq_dequantize: E (k_hat / n) = c[code] with codes from a bit loop (E in
  place of E_inv fails by orders of magnitude); identity metric bit-exact
  c[code] * n; diagonal metric closed form.
* smaq_scores: diagonal-metric float64 loop; q . (n E^-1 c[code]) * scale
  with E^-1 from a float64 solve of the encoder metric; query dtype output.
* blockvq_scores: float64 per-block gather loop (16x8, 64x2, 4x32 blocks),
  flipped block order fails; keys on codewords give the plain dot product.
* scalar_encode: codes equal a float64 numpy recomputation except where y is
  within 1e-6 (relative) of a decision boundary; norms within 1 ulp of fp64;
  zero key, unit-basis keys, saturation special cases.
* blockvq_encode: brute-force float64 nearest centroid on small inputs (ties
  within 1e-6 relative excluded); identity metric reduces to plain VQ.
* kmeans: golden vector written by importing the reference (tests/golden).
* quantize_values / dequantize_values: hand-computed known-answer vectors,
  |v - v_hat| <= scale/2 (+1 ulp) bound, min -> 0 / max -> 2^b-1 codes,
  constant-group clamp.
* hybrid_attention: float64 softmax(q K^T) V closed form on dequantized
  K/V; MIN_HISTORY rule; empty -> zeros; GQA head mapping.
"""

from __future__ import annotations

import math
from typing import NamedTuple, Optional

import torch
import torch.nn.functional as F

MIN_HISTORY_FOR_SMAQ = 16  # smaq/score.py:20


# ---------------------------------------------------------------------------
# Spectral metric (host side)                       smaq/ssf.py:8-29
# ---------------------------------------------------------------------------

def ssf_log(eigvals: torch.Tensor, c: float = 5.0) -> torch.Tensor:
    """smaq/ssf.py:8-18 -- log-compressed, volume-normalised spectrum."""
    shaped = torch.log1p(c * eigvals.clamp(min=0))
    logs = torch.log(shaped.clamp(min=1e-8))
    logs = logs - logs.mean()
    return torch.exp(logs)


def build_metric(sigma: torch.Tensor, c: float = 5.0):
    """smaq/ssf.py:21-29 -- E = V diag(sqrt s) V^T, E_inv = V diag(1/sqrt s) V^T."""
    evals, evecs = torch.linalg.eigh(sigma)
    s = ssf_log(evals, c)
    e = evecs @ torch.diag(s.sqrt()) @ evecs.T
    e_inv = evecs @ torch.diag(1.0 / s.sqrt()) @ evecs.T
    return e, e_inv


def _normal_ppf(p: torch.Tensor) -> torch.Tensor:
    """smaq/quantizer.py:58-60."""
    return math.sqrt(2.0) * torch.erfinv((2.0 * p) - 1.0)


def scalar_tables(bits: int, dtype=torch.float32):
    """smaq/quantizer.py:96-119 -- Gaussian-quantile centroids and boundaries.

    Returns (centroids [2^b], boundaries [2^b+1] with +-inf ends,
    decision_boundaries [2^b-1]).
    """
    probs = torch.linspace(0.0, 1.0, (2 ** bits) + 2, dtype=torch.float32)[1:-1]
    centroids = _normal_ppf(probs).to(dtype)
    bp = torch.linspace(0.0, 1.0, (2 ** bits) + 1, dtype=torch.float32)
    boundaries = _normal_ppf(bp.clamp(1e-6, 1.0 - 1e-6)).to(dtype)
    boundaries[0] = -float("inf")
    boundaries[-1] = float("inf")
    return centroids, boundaries, boundaries[1:-1].contiguous()


def midpoint_tables(bits: int, dtype=torch.float32, centroids=None, boundaries=None):
    """smaq/weighted_scalar.py:22-51 -- RotationAdapter codebook (midpoint cuts)."""
    if centroids is None:
        probs = torch.linspace(0.0, 1.0, (2 ** bits) + 2, dtype=torch.float32)[1:-1]
        centroids = _normal_ppf(probs).to(dtype)
    else:
        centroids = centroids.to(dtype)
    if boundaries is None:
        mids = 0.5 * (centroids[:-1] + centroids[1:])
        boundaries = torch.empty(centroids.shape[0] + 1, dtype=dtype)
        boundaries[0] = -float("inf")
        boundaries[-1] = float("inf")
        boundaries[1:-1] = mids
    else:
        boundaries = boundaries.to(dtype)
    return centroids, boundaries, boundaries[1:-1].contiguous()


def diag_metric_scales(sigma, rotation=None, c: float = 5.0, min_scale: float = 1e-6):
    """smaq/weighted_scalar.py:54-87 -- per-coordinate scales of R M R^T."""
    sigma = sigma.to(torch.float32)
    evals, evecs = torch.linalg.eigh(sigma)
    metric = evecs @ torch.diag(ssf_log(evals, c=c)) @ evecs.T
    if rotation is not None:
        rotation = rotation.to(torch.float32)
        metric = rotation @ metric @ rotation.T
    diag = metric.diagonal(dim1=-2, dim2=-1).clamp(min=min_scale)
    scales = diag.sqrt()
    logs = torch.log(scales)
    return torch.exp(logs - logs.mean())


def fit_sigma_centered(queries: torch.Tensor) -> torch.Tensor:
    """smaq/quantizer.py:121-129 -- centred query covariance used by fit()."""
    q = queries.float()
    centered = q - q.mean(dim=0, keepdim=True)
    return (centered.T @ centered) / max(1, centered.shape[0])


# ---------------------------------------------------------------------------
# Bit packing                                   smaq/quantizer.py:34-55
# ---------------------------------------------------------------------------

def pack_codes(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """smaq/quantizer.py:34-46 -- vpb = max(1, 8 // bits) codes per byte, first
    code in the low bits, last dim zero-padded to a multiple of vpb."""
    vpb = max(1, 8 // bits)
    lead = codes.shape[:-1]
    d = codes.shape[-1]
    pd = ((d + vpb - 1) // vpb) * vpb
    c8 = codes.to(torch.uint8)
    if pd > d:
        c8 = F.pad(c8, (0, pd - d), value=0)
    grouped = c8.reshape(*lead, -1, vpb)
    shifts = torch.arange(vpb, dtype=torch.uint8) * bits
    return (grouped << shifts).sum(dim=-1, dtype=torch.uint8)


def unpack_codes(packed: torch.Tensor, bits: int, d: int) -> torch.Tensor:
    """smaq/quantizer.py:49-55 -- inverse of pack_codes, int64 codes."""
    vpb = max(1, 8 // bits)
    mask = (1 << bits) - 1
    shifts = torch.arange(vpb, dtype=torch.uint8) * bits
    out = ((packed.unsqueeze(-1) >> shifts) & mask).reshape(*packed.shape[:-1], -1)
    return out[..., :d].long()


# ---------------------------------------------------------------------------
# Scalar key codec (SMAQQuantizer / RotationAdapter)
# ---------------------------------------------------------------------------

class ScalarQ(NamedTuple):
    """smaq/quantizer.py:26-31 (SMAQQuantized)."""
    indices: torch.Tensor
    norms: torch.Tensor
    bits: int


def scalar_encode(k: torch.Tensor, M: torch.Tensor, decision_boundaries: torch.Tensor,
                  bits: int, coord_scales: Optional[torch.Tensor] = None) -> ScalarQ:
    """SMAQQuantizer.quantize (smaq/quantizer.py:138-145) when coord_scales is
    None, with M = E; RotationAdapter.quantize (smaq/weighted_scalar.py:347-355)
    otherwise, with M = rotation.
    """
    norms = k.norm(dim=-1, keepdim=False)
    k_unit = k / (norms.unsqueeze(-1) + 1e-10)
    y = torch.matmul(k_unit.float(), M.float().T)
    if coord_scales is not None:
        y = y * coord_scales.float()
    idx = torch.searchsorted(decision_boundaries, y.contiguous())
    return ScalarQ(pack_codes(idx, bits), norms, bits)


def scalar_y(k: torch.Tensor, M: torch.Tensor, coord_scales=None) -> torch.Tensor:
    """The pre-quantisation coordinates y of scalar_encode (for tie analysis)."""
    norms = k.norm(dim=-1, keepdim=False)
    k_unit = k / (norms.unsqueeze(-1) + 1e-10)
    y = torch.matmul(k_unit.float(), M.float().T)
    if coord_scales is not None:
        y = y * coord_scales.float()
    return y


def smaq_dequantize(q: ScalarQ, centroids, E_inv, dim: int) -> torch.Tensor:
    """smaq/quantizer.py:147-152."""
    idx = unpack_codes(q.indices, q.bits, dim)
    y_hat = centroids[idx]
    k_hat = torch.matmul(y_hat.float(), E_inv.T)
    return (k_hat * q.norms.unsqueeze(-1)).to(E_inv.dtype)


def rotation_dequantize(q: ScalarQ, centroids, inv_coord_scales, rotation, dim: int) -> torch.Tensor:
    """smaq/weighted_scalar.py:357-363."""
    idx = unpack_codes(q.indices, q.bits, dim)
    shaped = centroids[idx]
    rot_hat = shaped.float() * inv_coord_scales.float()
    k_hat = torch.matmul(rot_hat, rotation.float())
    return (k_hat * q.norms.unsqueeze(-1)).to(rotation.dtype)


def smaq_scores(query, q: ScalarQ, centroids, E_inv, dim: int, scale=None) -> torch.Tensor:
    """smaq/quantizer.py:154-184 with smaq/triton_kernels.py:102-114 (the
    torch path the library's own callers always reach)."""
    q_rot = torch.matmul(query.float(), E_inv.T)
    idx = unpack_codes(q.indices, q.bits, dim)
    y_hat = centroids[idx]
    s = torch.matmul(q_rot.float(), y_hat.float().transpose(-2, -1))
    s = s * q.norms.unsqueeze(-2)
    if scale is not None:
        s = s * scale
    return s.to(query.dtype)


def rotation_scores(query, q: ScalarQ, centroids, inv_coord_scales, rotation, dim: int, scale=None):
    """smaq/weighted_scalar.py:342-345,365-379."""
    q_rot = torch.matmul(query.float(), rotation.T.float()) * inv_coord_scales.float()
    idx = unpack_codes(q.indices, q.bits, dim)
    shaped = centroids[idx]
    s = torch.matmul(q_rot.float(), shaped.float().transpose(-2, -1))
    s = s * q.norms.unsqueeze(-2)
    if scale is not None:
        s = s * scale
    return s.to(query.dtype)


# ---------------------------------------------------------------------------
# Block-VQ key codec                                 smaq/block_vq.py
# ---------------------------------------------------------------------------

class BlockQ(NamedTuple):
    """smaq/block_vq.py:25-30 (BlockVQQuantized)."""
    indices: torch.Tensor
    n_blocks: int
    block_dim: int


def kmeans(data: torch.Tensor, n_centroids: int, n_iters: int = 20, seed: int = 42) -> torch.Tensor:
    """smaq/block_vq.py:37-79 -- k-means++ seeding then Lloyd iterations.

    The RNG stream (one randint, then n_centroids-1 multinomial draws from one
    generator) decides the codebook; it is pinned by a golden vector.
    """
    n, d = data.shape
    gen = torch.Generator(device=data.device).manual_seed(seed)
    if n <= n_centroids:
        out = torch.zeros((n_centroids, d), dtype=data.dtype)
        out[:n] = data
        return out
    chosen = [torch.randint(n, (1,), generator=gen).item()]
    for _ in range(n_centroids - 1):
        dmin = torch.cdist(data, data[chosen]).min(dim=1).values
        w = dmin.square()
        tot = w.sum()
        w = w / tot if tot > 0 else torch.full((n,), 1.0 / n, dtype=data.dtype)
        chosen.append(torch.multinomial(w, 1, generator=gen).item())
    cents = data[chosen].clone()
    for _ in range(n_iters):
        assign = torch.cdist(data, cents).argmin(dim=1)
        acc = torch.zeros_like(cents)
        cnt = torch.zeros(n_centroids)
        acc.index_add_(0, assign, data)
        cnt.index_add_(0, assign, torch.ones(n))
        live = cnt > 0
        acc[live] /= cnt[live].unsqueeze(1)
        acc[~live] = cents[~live]
        cents = acc
    return cents


def blockvq_fit(keys, queries, block_dim=8, n_centroids=256, c=5.0, iters=20, seed=42):
    """smaq/block_vq.py:160-210 -- per-block uncentred Sigma_q, metric, k-means,
    pre-decoded centroids.  Returns (E_blocks, E_inv_blocks, centroids, decoded)."""
    N, D = keys.shape
    Es, Eis, Cs, Ds = [], [], [], []
    for bi in range(D // block_dim):
        sl = slice(bi * block_dim, (bi + 1) * block_dim)
        qb = queries[:, sl].float()
        sig = (qb.T @ qb) / N
        E, Ei = build_metric(sig, c=c)
        shaped = keys[:, sl].float() @ E.T
        cents = kmeans(shaped, n_centroids, iters, seed + bi)
        Es.append(E)
        Eis.append(Ei)
        Cs.append(cents)
        Ds.append(cents @ Ei.T)
    return torch.stack(Es), torch.stack(Eis), torch.stack(Cs), torch.stack(Ds)


def blockvq_encode(k: torch.Tensor, E_blocks, centroids) -> BlockQ:
    """smaq/block_vq.py:216-244 -- per block: x = k_b @ E_b^T, cdist, argmin."""
    nb, _, bd = centroids.shape
    D = nb * bd
    lead = k.shape[:-1]
    kf = k.reshape(-1, D).float()
    out = []
    for bi in range(nb):
        sl = slice(bi * bd, (bi + 1) * bd)
        x = kf[:, sl] @ E_blocks[bi].T
        out.append(torch.cdist(x, centroids[bi]).argmin(dim=-1))
    return BlockQ(torch.stack(out, dim=-1).reshape(*lead, nb), nb, bd)


def blockvq_distances(k: torch.Tensor, E_blocks, centroids) -> torch.Tensor:
    """cdist values of blockvq_encode, [rows, n_blocks, n_centroids] (tie analysis)."""
    nb, _, bd = centroids.shape
    kf = k.reshape(-1, nb * bd).float()
    return torch.stack([torch.cdist(kf[:, bi * bd:(bi + 1) * bd] @ E_blocks[bi].T, centroids[bi])
                        for bi in range(nb)], dim=1)


def blockvq_dequantize(q: BlockQ, decoded) -> torch.Tensor:
    """smaq/block_vq.py:246-267 -- pure LUT of pre-decoded centroids."""
    lead = q.indices.shape[:-1]
    idx = q.indices.reshape(-1, q.n_blocks).long()
    parts = [decoded[bi][idx[:, bi]] for bi in range(q.n_blocks)]
    return torch.cat(parts, dim=-1).reshape(*lead, q.n_blocks * q.block_dim)


def blockvq_scores(query, q: BlockQ, decoded, scale=None):
    """smaq/block_vq.py:273-297."""
    k_hat = blockvq_dequantize(q, decoded)
    s = torch.matmul(query.float(), k_hat.float().transpose(-2, -1))
    if scale is not None:
        s = s * scale
    return s.to(query.dtype)


# ---------------------------------------------------------------------------
# Value codec                                      smaq/kv_cache.py:20-103
# ---------------------------------------------------------------------------

class ValueQ(NamedTuple):
    """smaq/kv_cache.py:20-26 (ValueQuantized)."""
    data: torch.Tensor
    scales: torch.Tensor
    zeros: torch.Tensor
    bits: int = 2


def quantize_values(v: torch.Tensor, bits: int = 2, group_size: int = 32) -> ValueQ:
    """smaq/kv_cache.py:50-91 -- groupwise asymmetric min/max quantisation."""
    shape = v.shape
    d = shape[-1]
    if d % group_size != 0:
        raise ValueError(f"head_dim {d} must be divisible by group_size {group_size}")
    g = v.reshape(*shape[:-1], d // group_size, group_size)
    lo = g.min(dim=-1, keepdim=True).values
    hi = g.max(dim=-1, keepdim=True).values
    levels = (2 ** bits) - 1
    scale = ((hi - lo) / levels).clamp(min=1e-10)
    codes = ((g - lo) / scale).round().clamp(0, levels).to(torch.uint8).reshape(*shape[:-1], d)
    if bits == 2:
        q4 = codes.reshape(*shape[:-1], d // 4, 4)
        codes = q4[..., 0] | (q4[..., 1] << 2) | (q4[..., 2] << 4) | (q4[..., 3] << 6)
    elif bits == 4:
        q2 = codes.reshape(*shape[:-1], d // 2, 2)
        codes = q2[..., 0] | (q2[..., 1] << 4)
    return ValueQ(codes, scale.squeeze(-1), lo.squeeze(-1), bits)


def unpack_values(vq: ValueQ) -> torch.Tensor:
    """smaq/kv_cache.py:29-47."""
    p = vq.data
    if vq.bits == 2:
        return torch.stack([(p >> s) & 3 for s in (0, 2, 4, 6)], dim=-1).reshape(*p.shape[:-1], p.shape[-1] * 4)
    if vq.bits == 4:
        return torch.stack([p & 15, (p >> 4) & 15], dim=-1).reshape(*p.shape[:-1], p.shape[-1] * 2)
    return p


def dequantize_values(vq: ValueQ, group_size: int = 32) -> torch.Tensor:
    """smaq/kv_cache.py:94-103 -- fp32 code * scale + zero."""
    data = unpack_values(vq).float()
    d = data.shape[-1]
    data = data.reshape(*data.shape[:-1], d // group_size, group_size)
    return (data * vq.scales.unsqueeze(-1) + vq.zeros.unsqueeze(-1)).reshape(*data.shape[:-2], d)


# ---------------------------------------------------------------------------
# Store + hybrid attention              smaq/store.py, smaq/score.py
# ---------------------------------------------------------------------------

class Codec:
    """The strategy seam (smaq/strategies.py:100-255): quantize + per-head scores."""

    def quantize(self, keys):
        raise NotImplementedError

    def scores(self, query, key_q, scale):
        raise NotImplementedError

    def flatten(self, key_q):
        raise NotImplementedError

    def concat(self, chunks):
        raise NotImplementedError

    def select_head(self, key_q, h):
        raise NotImplementedError


class ScalarCodec(Codec):
    """SMAQFullMetricScalarStrategy / SMAQQuantizer (smaq/strategies.py:143-168)
    or, with rotation/coord scales, RotationAdapter (smaq/weighted_scalar.py)."""

    def __init__(self, dim, bits, E=None, E_inv=None, centroids=None, decision_boundaries=None,
                 rotation=None, coord_scales=None):
        self.dim, self.bits = dim, bits
        self.rotation = rotation
        self.coord_scales = coord_scales
        if rotation is None:
            c, _, db = scalar_tables(bits)
            self.E, self.E_inv = E, E_inv
        else:
            c, _, db = midpoint_tables(bits)
            self.inv_coord_scales = 1.0 / coord_scales.clamp(min=1e-6)
        self.centroids = c if centroids is None else centroids
        self.decision_boundaries = db if decision_boundaries is None else decision_boundaries

    def quantize(self, keys):
        if self.rotation is None:
            return scalar_encode(keys, self.E, self.decision_boundaries, self.bits)
        return scalar_encode(keys, self.rotation, self.decision_boundaries, self.bits, self.coord_scales)

    def dequantize(self, q):
        if self.rotation is None:
            return smaq_dequantize(q, self.centroids, self.E_inv, self.dim)
        return rotation_dequantize(q, self.centroids, self.inv_coord_scales, self.rotation, self.dim)

    def scores(self, query, q, scale):
        if self.rotation is None:
            return smaq_scores(query, q, self.centroids, self.E_inv, self.dim, scale)
        return rotation_scores(query, q, self.centroids, self.inv_coord_scales, self.rotation, self.dim, scale)

    def flatten(self, q):
        """smaq/strategies.py:118-123."""
        return ScalarQ(q.indices.reshape(-1, q.indices.shape[-2], q.indices.shape[-1]).contiguous(),
                       q.norms.reshape(-1, q.norms.shape[-1]).contiguous(), q.bits)

    def concat(self, chunks):
        """smaq/strategies.py:125-130."""
        return ScalarQ(torch.cat([c.indices for c in chunks], dim=-2),
                       torch.cat([c.norms for c in chunks], dim=-1), chunks[0].bits)

    def select_head(self, q, h):
        """smaq/strategies.py:132-137."""
        return ScalarQ(q.indices[h], q.norms[h], q.bits)


class BlockVQCodec(Codec):
    """SMAQBlockVQStrategy (smaq/strategies.py:195-255)."""

    def __init__(self, E_blocks, centroids, decoded):
        self.E_blocks, self.centroids, self.decoded = E_blocks, centroids, decoded

    def quantize(self, keys):
        return blockvq_encode(keys, self.E_blocks, self.centroids)

    def dequantize(self, q):
        return blockvq_dequantize(q, self.decoded)

    def scores(self, query, q, scale):
        return blockvq_scores(query, q, self.decoded, scale)

    def flatten(self, q):
        return BlockQ(q.indices.reshape(-1, q.indices.shape[-2], q.indices.shape[-1]).contiguous(),
                      q.n_blocks, q.block_dim)

    def concat(self, chunks):
        return BlockQ(torch.cat([c.indices for c in chunks], dim=-2), chunks[0].n_blocks, chunks[0].block_dim)

    def select_head(self, q, h):
        return BlockQ(q.indices[h], q.n_blocks, q.block_dim)


class FlatCache(NamedTuple):
    """smaq/store.py:20-25."""
    key_q: object
    value_q: ValueQ
    num_tokens: int


class Store:
    """CompressedKVStore restated (smaq/store.py:28-124)."""

    def __init__(self, codec: Codec, head_dim, num_kv_heads, value_bits=2, value_group_size=32):
        self.codec = codec
        self.head_dim, self.num_kv_heads = head_dim, num_kv_heads
        self.value_bits = value_bits
        self.value_group_size = min(value_group_size, head_dim)   # smaq/store.py:48
        self.kc, self.vc, self.lens = [], [], []

    @property
    def num_tokens(self):
        return sum(self.lens)

    def append_chunk(self, key, value):
        """smaq/store.py:83-95 -- [T, Hkv, D] -> [1, Hkv, T, D], quantise."""
        k = key.transpose(0, 1).unsqueeze(0)
        v = value.transpose(0, 1).unsqueeze(0)
        self.kc.append(self.codec.quantize(k))
        self.vc.append(quantize_values(v, bits=self.value_bits, group_size=self.value_group_size))
        self.lens.append(key.shape[0])

    def get_flat_cache(self):
        """smaq/store.py:97-114 and :133-152."""
        if not self.kc:
            return None
        kq = self.codec.concat([self.codec.flatten(c) for c in self.kc])

        def flat_v(vq):
            return ValueQ(vq.data.reshape(-1, vq.data.shape[-2], vq.data.shape[-1]).contiguous(),
                          vq.scales.reshape(-1, vq.scales.shape[-2], vq.scales.shape[-1]).contiguous(),
                          vq.zeros.reshape(-1, vq.zeros.shape[-2], vq.zeros.shape[-1]).contiguous(),
                          vq.bits)
        fv = [flat_v(c) for c in self.vc]
        vq = ValueQ(torch.cat([c.data for c in fv], dim=-2), torch.cat([c.scales for c in fv], dim=-2),
                    torch.cat([c.zeros for c in fv], dim=-2), fv[0].bits)
        return FlatCache(kq, vq, self.num_tokens)


def _hist_scores(query, flat, codec, g, hkv, scale):
    """smaq/score.py:75-96 -- per-KV-head loop, [T, Hq, N] fp32 logits."""
    q = query.float().view(query.shape[0], hkv, g, query.shape[-1]).permute(1, 2, 0, 3)
    per_head = [codec.scores(q[h], codec.select_head(flat.key_q, h), scale) for h in range(hkv)]
    return torch.stack(per_head, 0).permute(2, 0, 1, 3).reshape(query.shape[0], query.shape[1], flat.num_tokens)


def _exact_scores(query, recent_k, g, hkv, scale):
    """smaq/score.py:99-110."""
    q = query.float().view(query.shape[0], hkv, g, query.shape[-1]).permute(1, 2, 0, 3)
    k = recent_k.transpose(0, 1).float().unsqueeze(1)
    s = torch.einsum("hgtd,hgnd->hgtn", q, k) * scale
    return s.permute(2, 0, 1, 3).reshape(query.shape[0], query.shape[1], recent_k.shape[0])


def _apply(weights, values, g, hkv, out_dtype):
    """smaq/score.py:113-124."""
    v = values.float().unsqueeze(1)
    w = weights.float().view(weights.shape[0], hkv, g, weights.shape[-1]).permute(1, 2, 0, 3)
    o = torch.einsum("hgtn,hgnd->hgtd", w, v)
    return o.permute(2, 0, 1, 3).reshape(weights.shape[0], hkv * g, values.shape[-1]).to(out_dtype)


def hybrid_attention(query, store: Store, recent_k, recent_v, num_query_heads, scale=None,
                     query_positions: Optional[torch.Tensor] = None):
    """smaq/score.py:23-72 -- one softmax over [history; recent] logits, each
    part cast to the query dtype before the sum.

    ``query_positions`` (int64 [T]) is the build's causal extension (the
    reference has no mask): key j (history positions 0..N-1 then recent
    N..N+R-1) is visible to query t iff j <= query_positions[t].
    """
    D, hkv = store.head_dim, store.num_kv_heads
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    flat = store.get_flat_cache()
    has_hist = flat is not None and flat.num_tokens >= MIN_HISTORY_FOR_SMAQ
    has_recent = recent_k is not None and recent_k.shape[0] > 0
    if not has_hist and not has_recent:
        return torch.zeros(query.shape[0], num_query_heads, D, dtype=query.dtype)
    g = num_query_heads // hkv
    parts = []
    if has_hist:
        parts.append(_hist_scores(query, flat, store.codec, g, hkv, scale))
    if has_recent:
        parts.append(_exact_scores(query, recent_k, g, hkv, scale))
    logits = torch.cat(parts, dim=-1)
    if query_positions is not None:
        # absolute key positions: history 0..N-1, recent N..N+R-1 (N counts the
        # whole store even when it is too short to be attended)
        n_all = flat.num_tokens if flat is not None else 0
        pos_h = torch.arange(n_all) if has_hist else torch.zeros(0, dtype=torch.long)
        pos_r = n_all + torch.arange(recent_k.shape[0]) if has_recent else torch.zeros(0, dtype=torch.long)
        pos = torch.cat([pos_h, pos_r])
        mask = pos[None, :] > query_positions[:, None]
        logits = logits.masked_fill(mask[:, None, :], float("-inf"))
    w = F.softmax(logits, dim=-1)
    if has_hist and not has_recent:
        return _apply(w, dequantize_values(flat.value_q, store.value_group_size), g, hkv, query.dtype)
    if has_recent and not has_hist:
        return _apply(w, recent_v.transpose(0, 1), g, hkv, query.dtype)
    n = flat.num_tokens
    o_h = _apply(w[..., :n], dequantize_values(flat.value_q, store.value_group_size), g, hkv, query.dtype)
    o_r = _apply(w[..., n:], recent_v.transpose(0, 1), g, hkv, query.dtype)
    return o_h + o_r


# ---------------------------------------------------------------------------
# Recent window                                        smaq/capture.py:18-110
# ---------------------------------------------------------------------------

class Ring:
    """RingBuffer restated: write() returns the whole ring as overflow once it
    is full and more tokens arrive (smaq/capture.py:60-91)."""

    def __init__(self, capacity, hkv, d, dtype=torch.bfloat16):
        self.capacity = capacity
        self.k = torch.zeros(capacity, hkv, d, dtype=dtype)
        self.v = torch.zeros(capacity, hkv, d, dtype=dtype)
        self.pos = 0
        self.total = 0

    def write(self, key, value, n):
        ok, ov = [], []
        off = 0
        while n - off > 0:
            if self.capacity - self.pos <= 0:
                ok.append(self.k[:self.pos].clone())
                ov.append(self.v[:self.pos].clone())
                self.pos = 0
            w = min(n - off, self.capacity - self.pos)
            self.k[self.pos:self.pos + w] = key[off:off + w]
            self.v[self.pos:self.pos + w] = value[off:off + w]
            self.pos += w
            off += w
        self.total += n
        return (torch.cat(ok), torch.cat(ov)) if ok else None

    def peek(self):
        return None if self.pos == 0 else (self.k[:self.pos], self.v[:self.pos])
