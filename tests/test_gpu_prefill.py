"""GPU parity of the matrix-core chunked-prefill kernel (impl=3).

At sizes the oracle finishes in seconds the kernel is checked against the
CPU oracle (the paged layout included, its history gathered through the
block table); at larger and batched shapes against the generic GPU kernels
(impl=1), which are themselves oracle-checked in test_gpu_attention.py.  Tolerance as there: 2e-3 absolute + 1e-3 relative
(+ one output ulp for bf16/fp16 outputs).  Shapes exercise partial 64-key
tiles, partial 128-query blocks, GQA groups, causal masks that cut tiles, and
the history/recent split of one softmax."""

from __future__ import annotations

import pytest
import torch

import smaq_amd as S
from smaq_amd.batch import PagedQuantizedKV, QuantizedKVBatch
from oracle import smaq_ref as R
from tests.conftest import sample_keys
from tests.test_gpu_attention import _pair_scalar, assert_attn_close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_scalar_vs_oracle(dev, causal):
    """4-bit SMAQ keys, GQA 8/2, 1000 history + 45 bf16 recent tokens,
    150 bf16 queries (one full and one partial 128-query block)."""
    hkv, hq, N, Rn, T = 2, 8, 1000, 45, 150
    st, ref = _pair_scalar(dev, bits=4, hkv=hkv)
    keys = sample_keys(N * hkv, seed=201).reshape(N, hkv, 128).bfloat16()
    vals = torch.randn(N, hkv, 128, generator=torch.Generator().manual_seed(202)).bfloat16()
    st.append_chunk(keys.to(dev), vals.to(dev))
    ref.append_chunk(keys, vals)
    q = sample_keys(T * hq, seed=203).reshape(T, hq, 128).bfloat16()
    kr = sample_keys(Rn * hkv, seed=204).reshape(Rn, hkv, 128).bfloat16()
    vr = torch.randn(Rn, hkv, 128, generator=torch.Generator().manual_seed(205)).bfloat16()
    # queries spread over the history so the mask cuts many tiles
    pos = torch.linspace(300, N + Rn - 1, T).long() if causal else None
    out = S.compute_hybrid_attention(q.to(dev), st, kr.to(dev), vr.to(dev), hq,
                                     query_positions=None if pos is None else pos.to(dev), impl=3)
    assert_attn_close(out, R.hybrid_attention(q, ref, kr, vr, hq, query_positions=pos), f"prefill causal={causal}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_single_tile_parts(dev, causal, dtype):
    """History and recent window of one 64-key tile each (40 + 20 tokens),
    24 queries: each workgroup's loop runs once, so the waves that take
    their PV one tile late do it after the loop (fp16: every part in the
    cheap form; fp32: the recent window's values are not exact in f16 and
    may take the precise form)."""
    hkv, hq, N, Rn, T = 2, 8, 40, 20, 24
    st, ref = _pair_scalar(dev, bits=4, hkv=hkv)
    keys = sample_keys(N * hkv, seed=251).reshape(N, hkv, 128)
    vals = torch.randn(N, hkv, 128, generator=torch.Generator().manual_seed(252))
    st.append_chunk(keys.to(dev), vals.to(dev))
    ref.append_chunk(keys, vals)
    q = sample_keys(T * hq, seed=253).reshape(T, hq, 128).to(dtype)
    kr = sample_keys(Rn * hkv, seed=254).reshape(Rn, hkv, 128).to(dtype)
    vr = torch.randn(Rn, hkv, 128, generator=torch.Generator().manual_seed(255)).to(dtype)
    pos = torch.arange(N + Rn - T, N + Rn) if causal else None
    out = S.compute_hybrid_attention(q.to(dev), st, kr.to(dev), vr.to(dev), hq,
                                     query_positions=None if pos is None else pos.to(dev), impl=3)
    assert_attn_close(out, R.hybrid_attention(q, ref, kr, vr, hq, query_positions=pos),
                      f"prefill one tile causal={causal} {dtype}")


@pytest.mark.parametrize("qdtype", [torch.float32, torch.float16, torch.bfloat16])
def test_prefill_large_values_default_tolerance(dev, qdtype):
    """Values of scale 8 (|v| up to ~35), whose f16 rounding alone (2^-11 |v|)
    would exceed the 2e-3 budget: the key ranges holding them take the
    precise form (value lo plane, hi/lo weights), so every output dtype
    meets the default tolerance of the fp32 path."""
    hkv, hq, N, T = 2, 8, 900, 64
    st, ref = _pair_scalar(dev, bits=4, hkv=hkv)
    keys = sample_keys(N * hkv, seed=231).reshape(N, hkv, 128)
    vals = 8 * torch.randn(N, hkv, 128, generator=torch.Generator().manual_seed(232))
    st.append_chunk(keys.to(dev), vals.to(dev))
    ref.append_chunk(keys, vals)
    q = sample_keys(T * hq, seed=233).reshape(T, hq, 128).to(qdtype)
    out = S.compute_hybrid_attention(q.to(dev), st, None, None, hq, impl=3)
    assert out.dtype == qdtype
    vmax = R.dequantize_values(ref.get_flat_cache().value_q).abs().max().item()
    assert vmax > 16
    assert_attn_close(out, R.hybrid_attention(q, ref, None, None, hq), f"prefill |v|<={vmax:.1f} {qdtype}")
    # the automatic choice serves this shape with the same kernel
    assert torch.equal(S.compute_hybrid_attention(q.to(dev), st, None, None, hq), out)


def test_prefill_cancelling_values_near_budget(dev):
    """Values just under 8 in magnitude with alternating signs (outputs near
    zero while sum w|v| ~ 7.9): the largest values the cheap form accepts,
    in the case where its error bound is tightest against the absolute
    tolerance."""
    hkv, hq, N, T = 1, 4, 640, 48
    st, ref = _pair_scalar(dev, bits=4, hkv=hkv)
    keys = sample_keys(N * hkv, seed=261).reshape(N, hkv, 128)
    g = torch.Generator().manual_seed(262)
    sign = torch.where(torch.rand(N, hkv, 128, generator=g) < 0.5, -1.0, 1.0)
    vals = sign * (7.0 + 0.9 * torch.rand(N, hkv, 128, generator=g))
    st.append_chunk(keys.to(dev), vals.to(dev))
    ref.append_chunk(keys, vals)
    q = sample_keys(T * hq, seed=263).reshape(T, hq, 128)
    out = S.compute_hybrid_attention(q.to(dev), st, None, None, hq, impl=3)
    assert_attn_close(out, R.hybrid_attention(q, ref, None, None, hq), "prefill cancelling |v|<8")


@pytest.mark.parametrize("rdtype", [torch.float32, torch.bfloat16])
def test_prefill_recent_window_precision(dev, rdtype):
    """Recent window of fp32 values (not exact in f16) and of bf16 values
    beyond f16's range (up to ~4e5, exact after the 2^-8 scaling), scale-8
    history values, 70 causal queries of the same dtype."""
    hkv, hq, N, Rn, T = 2, 8, 300, 90, 70
    st, ref = _pair_scalar(dev, bits=4, hkv=hkv)
    keys = sample_keys(N * hkv, seed=271).reshape(N, hkv, 128)
    vals = 8 * torch.randn(N, hkv, 128, generator=torch.Generator().manual_seed(272))
    st.append_chunk(keys.to(dev), vals.to(dev))
    ref.append_chunk(keys, vals)
    g = torch.Generator().manual_seed(273)
    q = sample_keys(T * hq, seed=274).reshape(T, hq, 128).to(rdtype)
    kr = sample_keys(Rn * hkv, seed=275).reshape(Rn, hkv, 128).to(rdtype)
    vscale = 12.0 if rdtype == torch.float32 else 1e5
    vr = (vscale * torch.randn(Rn, hkv, 128, generator=g)).to(rdtype)
    pos = torch.arange(N + Rn - T, N + Rn)
    out = S.compute_hybrid_attention(q.to(dev), st, kr.to(dev), vr.to(dev), hq, query_positions=pos.to(dev), impl=3)
    assert_attn_close(out, R.hybrid_attention(q, ref, kr, vr, hq, query_positions=pos), f"prefill recent {rdtype}")


def test_prefill_blockvq_vs_oracle(dev):
    """c4 format: block-VQ keys (block_dim 2, 256 centroids) with outlier
    channels, fp16 recent window, 130 causal fp16 queries at the end."""
    hkv, hq, N, Rn, T = 1, 7, 777, 128, 130
    keys = sample_keys(N * hkv, seed=211).reshape(N, hkv, 128)
    outl = torch.tensor([5, 44, 90, 127])
    keys[..., outl] *= 20
    vals = torch.randn(N, hkv, 128, generator=torch.Generator().manual_seed(212))
    calib_q = sample_keys(2048, seed=213)
    calib_k = sample_keys(2048, seed=214)
    calib_k[:, outl] *= 20
    strat = S.SMAQBlockVQStrategy(128, block_dim=2, n_centroids=256, device=dev)
    strat.quantizer.fit(calib_k, calib_q, kmeans_iters=3)
    qz = strat.quantizer
    codec = R.BlockVQCodec(qz.E_blocks.cpu(), qz.centroids.cpu(), qz.decoded_centroids.cpu())
    st = S.CompressedKVStore(128, hkv, device=dev, key_strategy=strat)
    ref = R.Store(codec, 128, hkv)
    st.append_chunk(keys.half().to(dev), vals.half().to(dev))
    ref.append_chunk(keys.half(), vals.half())
    got_idx = st.get_flat_cache().key_q.indices.cpu().long()
    if not torch.equal(got_idx, ref.get_flat_cache().key_q.indices):
        ref.kc = [R.BlockQ(got_idx.unsqueeze(0), 64, 2)]   # score the same codes on both sides
    q = sample_keys(T * hq, seed=215).reshape(T, hq, 128).half()
    kr = sample_keys(Rn * hkv, seed=216).reshape(Rn, hkv, 128).half()
    vr = torch.randn(Rn, hkv, 128, generator=torch.Generator().manual_seed(217)).half()
    pos = torch.arange(N + Rn - T, N + Rn)
    out = S.compute_hybrid_attention(q.to(dev), st, kr.to(dev), vr.to(dev), hq, query_positions=pos.to(dev), impl=3)
    assert_attn_close(out, R.hybrid_attention(q, ref, kr, vr, hq, query_positions=pos), "prefill block-VQ")


def test_prefill_bytewise_decode_vs_oracle(dev):
    """Formats the tile pre-pass decodes byte by byte (8-dim VQ blocks, 4-bit
    values in groups of 16; the 2-dim / 2-bit formats above take its
    16-byte loads): 300 history tokens, no recent window, 70 causal queries."""
    hkv, hq, N, T = 2, 4, 300, 70
    keys = sample_keys(N * hkv, seed=218).reshape(N, hkv, 128)
    vals = torch.randn(N, hkv, 128, generator=torch.Generator().manual_seed(219))
    strat = S.SMAQBlockVQStrategy(128, block_dim=8, n_centroids=256, device=dev)
    strat.quantizer.fit(sample_keys(2048, seed=220), sample_keys(2048, seed=221), kmeans_iters=3)
    qz = strat.quantizer
    codec = R.BlockVQCodec(qz.E_blocks.cpu(), qz.centroids.cpu(), qz.decoded_centroids.cpu())
    st = S.CompressedKVStore(128, hkv, value_bits=4, value_group_size=16, device=dev, key_strategy=strat)
    ref = R.Store(codec, 128, hkv, value_bits=4, value_group_size=16)
    st.append_chunk(keys.half().to(dev), vals.half().to(dev))
    ref.append_chunk(keys.half(), vals.half())
    got_idx = st.get_flat_cache().key_q.indices.cpu().long()
    if not torch.equal(got_idx, ref.get_flat_cache().key_q.indices):
        ref.kc = [R.BlockQ(got_idx.unsqueeze(0), 16, 8)]   # score the same codes on both sides
    q = sample_keys(T * hq, seed=222).reshape(T, hq, 128).half()
    pos = torch.arange(N - T, N)
    out = S.compute_hybrid_attention(q.to(dev), st, None, None, hq, query_positions=pos.to(dev), impl=3)
    assert_attn_close(out, R.hybrid_attention(q, ref, None, None, hq, query_positions=pos), "prefill byte-wise")


def test_prefill_large_vs_generic(dev):
    """Qwen2-7B head shape (28/4) at 20000 history tokens and 300 causal
    queries: matrix-core prefill against the generic kernels."""
    hkv, hq, N, Rn, T = 4, 28, 20000, 128, 300
    g = torch.Generator().manual_seed(221)
    calib = sample_keys(4096, seed=222)
    strat = S.SMAQBlockVQStrategy(128, block_dim=2, n_centroids=256, device=dev)
    strat.quantizer.fit(calib, sample_keys(4096, seed=223), kmeans_iters=2)
    st = S.CompressedKVStore(128, hkv, device=dev, key_strategy=strat)
    keys = sample_keys(N * hkv, seed=224).reshape(N, hkv, 128).half().to(dev)
    vals = torch.randn(N, hkv, 128, generator=g).half().to(dev)
    st.append_chunk(keys, vals)
    q = sample_keys(T * hq, seed=225).reshape(T, hq, 128).half().to(dev)
    kr = sample_keys(Rn * hkv, seed=226).reshape(Rn, hkv, 128).half().to(dev)
    vr = torch.randn(Rn, hkv, 128, generator=g).half().to(dev)
    pos = torch.arange(N + Rn - T, N + Rn, device=dev)
    got = S.compute_hybrid_attention(q, st, kr, vr, hq, query_positions=pos, impl=3)
    ref = S.compute_hybrid_attention(q, st, kr, vr, hq, query_positions=pos, impl=1)
    assert_attn_close(got, ref.cpu(), "prefill 20000")
    auto = S.compute_hybrid_attention(q, st, kr, vr, hq, query_positions=pos)
    assert torch.equal(auto, got)   # the automatic choice for this shape


def test_prefill_batched_ragged_vs_generic(dev):
    """Batched contiguous history with ragged lengths (3-bit scalar keys) and a
    ragged recent window, 40 unmasked fp32 queries per sequence."""
    lens = [333, 1000, 64, 517]
    strat = S.SMAQFullMetricScalarStrategy(128, bits=3, device=dev).fit(sample_keys(64, seed=231))
    g = torch.Generator().manual_seed(232)
    keys = [sample_keys(n * 4, seed=233 + i).reshape(n, 4, 128).to(dev) for i, n in enumerate(lens)]
    vals = [torch.randn(n, 4, 128, generator=g).to(dev) for n in lens]
    kv = QuantizedKVBatch.encode(strat, keys, vals)
    B, T = len(lens), 40
    q = torch.randn(B, T, 16, 128, generator=g).to(dev)
    rk = torch.randn(B, 50, 4, 128, generator=g).to(dev)
    rv = torch.randn(B, 50, 4, 128, generator=g).to(dev)
    rl = torch.tensor([50, 7, 0, 31], device=dev)
    got = kv.attention(q, recent_k=rk, recent_v=rv, recent_len=rl, impl=3)
    ref = kv.attention(q, recent_k=rk, recent_v=rv, recent_len=rl, impl=1)
    assert_attn_close(got, ref.cpu(), "prefill batched ragged")


def test_prefill_paged_vs_generic(dev):
    """Paged history (block size 32, shuffled physical blocks), bf16, causal
    queries over the last 96 positions of each sequence."""
    lens = [700, 96, 1500]
    bs = 32
    nblk = [(n + bs - 1) // bs for n in lens]
    g = torch.Generator().manual_seed(241)
    perm = torch.randperm(sum(nblk) + 5, generator=g)
    table = torch.zeros(len(lens), max(nblk), dtype=torch.int32)
    o = 0
    for b, nb in enumerate(nblk):
        table[b, :nb] = perm[o:o + nb].to(torch.int32)
        o += nb
    strat = S.SMAQFullMetricScalarStrategy(128, bits=4, device=dev).fit(sample_keys(64, seed=242))
    keys = [sample_keys(n * 2, seed=243 + i).reshape(n, 2, 128).bfloat16().to(dev) for i, n in enumerate(lens)]
    vals = [torch.randn(n, 2, 128, generator=g).bfloat16().to(dev) for n in lens]
    pk = PagedQuantizedKV.encode(strat, keys, vals, table.to(dev), num_blocks=sum(nblk) + 5, block_size=bs)
    T = 96
    q = torch.randn(len(lens), T, 8, 128, generator=g).bfloat16().to(dev)
    pos = torch.stack([torch.arange(n - T, n) for n in lens]).to(dev)
    got = pk.attention(q, impl=3, query_positions=pos)
    ref = pk.attention(q, impl=1, query_positions=pos)
    assert_attn_close(got, ref.cpu(), "prefill paged")
    # and against the oracle: each sequence's history gathered from the GPU
    # pool through its block table, scored by the oracle's hybrid attention
    qz = strat.quantizer
    codec = R.ScalarCodec(128, 4, E=qz.E.cpu(), E_inv=qz.E_inv.cpu())
    for b, n in enumerate(lens):
        blocks = table[b, :nblk[b]].long().to(dev)

        def gather(x):  # pool [blocks, Hkv, bs, ...] -> [Hkv, n, ...]
            return x[blocks].transpose(0, 1).reshape(2, nblk[b] * bs, *x.shape[3:])[:, :n].cpu().contiguous()

        flat = R.FlatCache(R.ScalarQ(gather(pk.codes), gather(pk.norms), 4),
                           R.ValueQ(gather(pk.v_data), gather(pk.v_scales), gather(pk.v_zeros), 2), n)
        ost = _OracleFlatStore(flat, codec, 128, 2)
        ref_o = R.hybrid_attention(q[b].cpu(), ost, None, None, 8, query_positions=pos[b].cpu())
        assert_attn_close(got[b], ref_o, f"prefill paged vs oracle, sequence {b} ({n} tokens)")


class _OracleFlatStore:
    """The oracle store interface over a flat cache built from GPU codes."""

    def __init__(self, flat, codec, head_dim, num_kv_heads):
        self.flat, self.codec = flat, codec
        self.head_dim, self.num_kv_heads, self.value_group_size = head_dim, num_kv_heads, 32

    def get_flat_cache(self):
        return self.flat
