"""Encode-on-flush on the GPU: the capture engine's ring spills and the store's
append-only columns against the CPU oracle's Ring / Store replay.

At c3 head shape (8 KV heads, head_dim 128, bf16, 3-bit scalar keys, 2-bit
values) a prefill and a few hundred decode writes of mixed sizes drive the
ring through several spills; each spill is encoded by the HIP kernels straight
into the columns' tail rows, growing the columns on the way.  The oracle
replays the same writes through its slot-by-slot Ring and chunk-list Store.
Checked: chunk count and lengths, every column field bit for bit (codes up to
counted boundary ties, at most 2), the flat cache as head-strided views with
nothing copied, the ring contents, and hybrid decode attention over store +
ring within 2e-3 abs + 1e-3 rel (+1 bf16 ulp).  Block-VQ keys (c4 format) take
the same path; SMAQKVCache's flushes land in its columns the same way."""

from __future__ import annotations

import pytest
import torch

import smaq_amd as S
from oracle import smaq_ref as R
from tests.conftest import sample_keys
from tests.test_gpu_attention import assert_attn_close
from tests.test_gpu_codecs import _ties_ok

pytestmark = pytest.mark.gpu


def _replay(store, engine, ref_store, ref_ring, writes, dev):
    """Feed (kind, k, v) writes to the engine and the oracle replay."""
    for kind, k, v in writes:
        n = k.shape[0]
        if kind == "prefill":
            engine.ingest_prefill(k.to(dev), v.to(dev), n)
            C = ref_ring.capacity
            if n > C:
                ref_store.append_chunk(k[:n - C], v[:n - C])
            ref_ring.write(k[max(0, n - C):], v[max(0, n - C):], min(n, C))
        else:
            engine.ingest_decode(k.to(dev), v.to(dev), n)
            spill = ref_ring.write(k, v, n)
            if spill is not None:
                ref_store.append_chunk(*spill)


def _writes(hkv, seed, n_prefill, sizes):
    g = torch.Generator().manual_seed(seed)
    out = []
    total = n_prefill + sum(sizes)
    ks = sample_keys(total * hkv, seed=seed).reshape(total, hkv, 128).bfloat16()
    vs = torch.randn(total, hkv, 128, generator=g).bfloat16()
    out.append(("prefill", ks[:n_prefill], vs[:n_prefill]))
    o = n_prefill
    for n in sizes:
        out.append(("decode", ks[o:o + n], vs[o:o + n]))
        o += n
    return out


def test_ring_spills_encode_into_columns_c3_heads(dev):
    hkv, hq, bits = 8, 32, 3
    calib = sample_keys(64, seed=250)
    strat = S.SMAQFullMetricScalarStrategy(128, bits=bits, device=dev).fit(calib)
    E, Ei = R.build_metric(R.fit_sigma_centered(calib))
    codec = R.ScalarCodec(128, bits, E=E, E_inv=Ei)
    store = S.CompressedKVStore(128, hkv, key_bits=bits, device=dev, key_strategy=strat)
    engine = S.KVCaptureEngine(store, ring_capacity=128)
    ref_store, ref_ring = R.Store(codec, 128, hkv), R.Ring(128, hkv, 128)
    # prefill of 1000 tokens (872 to the store), 300 one-token decode steps,
    # then writes of 5, 200 (two windows at once), 128 and 3 tokens: several
    # spills, and the columns grow (872 -> 1744 rows)
    sizes = [1] * 300 + [5, 200, 128, 3]
    _replay(store, engine, ref_store, ref_ring, _writes(hkv, 251, 1000, sizes), dev)

    assert store.num_chunks == len(ref_store.lens) and store.num_tokens == ref_store.num_tokens
    assert engine.ring.size == ref_ring.pos
    assert torch.equal(engine.ring.peek()[0].cpu(), ref_ring.peek()[0])
    flat, rflat = store.get_flat_cache(), ref_store.get_flat_cache()
    n = flat.num_tokens
    # the flat cache is head-strided views of the columns, nothing copied
    cols = store._hist
    assert cols.capacity > n and flat.key_q.indices.stride(0) == cols.capacity * 64
    assert flat.key_q.indices.data_ptr() == cols.filled()["k_codes"].data_ptr()
    got = R.unpack_codes(flat.key_q.indices.cpu(), bits, 128)
    want = R.unpack_codes(rflat.key_q.indices, bits, 128)
    k_all = torch.cat([w[1] for w in _writes(hkv, 251, 1000, sizes)])[:n].transpose(0, 1)
    assert _ties_ok(got, want, R.scalar_y(k_all, E), R.scalar_tables(bits)[2]) <= 2
    assert torch.equal(flat.key_q.norms.cpu(), rflat.key_q.norms)
    for a, b in zip(flat.value_q[:3], rflat.value_q[:3]):
        assert torch.equal(a.cpu(), b)
    assert store.memory_bytes() == sum(
        c.indices.numel() + 2 * c.norms.numel() for c in ref_store.kc) + sum(
        v.data.numel() + 2 * v.scales.numel() + 2 * v.zeros.numel() for v in ref_store.vc)

    q = sample_keys(hq, seed=252).reshape(1, hq, 128).bfloat16()
    rk, rv = engine.ring.peek()
    out = S.compute_hybrid_attention(q.to(dev), store, rk, rv, hq)
    ref = R.hybrid_attention(q, ref_store, *ref_ring.peek(), hq)
    assert_attn_close(out, ref, "encode-on-flush hybrid decode")
    # a forced flush appends the ring as one more chunk
    engine.flush()
    spilled = ref_ring.peek()
    ref_store.append_chunk(*spilled)
    assert store.num_tokens == ref_store.num_tokens and engine.ring.size == 0
    assert torch.equal(store.get_flat_cache().value_q.data.cpu(), ref_store.get_flat_cache().value_q.data)


def test_ring_spills_blockvq_columns(dev):
    hkv, hq = 2, 8
    strat = S.SMAQBlockVQStrategy(128, block_dim=2, n_centroids=256, device=dev)
    strat.quantizer.fit(sample_keys(2048, seed=260), sample_keys(2048, seed=261), kmeans_iters=2, on_device=True)
    qz = strat.quantizer
    codec = R.BlockVQCodec(qz.E_blocks.cpu(), qz.centroids.cpu(), qz.decoded_centroids.cpu())
    store = S.CompressedKVStore(128, hkv, device=dev, key_strategy=strat)
    engine = S.KVCaptureEngine(store, ring_capacity=64)
    ref_store, ref_ring = R.Store(codec, 128, hkv), R.Ring(64, hkv, 128)
    _replay(store, engine, ref_store, ref_ring, _writes(hkv, 262, 300, [1] * 70 + [90, 7]), dev)
    flat, rflat = store.get_flat_cache(), ref_store.get_flat_cache()
    assert flat.num_tokens == rflat.num_tokens
    mism = int((flat.key_q.indices.cpu().long() != rflat.key_q.indices).sum())
    assert mism <= 2, f"{mism} block-VQ index mismatches"
    for a, b in zip(flat.value_q[:3], rflat.value_q[:3]):
        assert torch.equal(a.cpu(), b)


def test_kv_cache_flushes_into_columns(dev):
    """SMAQKVCache: one-token appends past the exact window land in the column
    history; the exact window slides without re-concatenation."""
    calib = sample_keys(64, seed=270)
    strat = S.SMAQFullMetricScalarStrategy(128, bits=4, device=dev).fit(calib)
    E, _ = R.build_metric(R.fit_sigma_centered(calib))
    _, _, db = R.scalar_tables(4)
    cache = S.SMAQKVCache(128, buffer_size=16, device=dev, key_strategy=strat)
    B, H, T0, T1 = 2, 4, 40, 300
    keys = sample_keys(B * H * (T0 + T1), seed=271).reshape(B, H, T0 + T1, 128).bfloat16()
    vals = torch.randn(B, H, T0 + T1, 128, generator=torch.Generator().manual_seed(272)).bfloat16()
    cache.prefill(keys[:, :, :T0].to(dev), vals[:, :, :T0].to(dev))
    for t in range(T0, T0 + T1):
        cache.append(keys[:, :, t:t + 1].to(dev), vals[:, :, t:t + 1].to(dev))
    nq = T0 + T1 - 16
    kq = cache.key_quantized
    assert kq.indices.shape == (B, H, nq, 64)
    ref = R.scalar_encode(keys[:, :, :nq], E, db, 4)
    assert _ties_ok(R.unpack_codes(kq.indices.cpu(), 4, 128), R.unpack_codes(ref.indices, 4, 128),
                    R.scalar_y(keys[:, :, :nq], E), db) <= 2
    assert torch.equal(kq.norms.cpu(), ref.norms)
    rv = R.quantize_values(vals[:, :, :nq], bits=2, group_size=32)
    assert torch.equal(cache.value_quantized.data.cpu(), rv.data)
    assert torch.equal(cache.key_buffer.cpu(), keys[:, :, nq:])
    assert torch.equal(cache.value_buffer.cpu(), vals[:, :, nq:])
