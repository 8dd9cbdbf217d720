"""GPU parity of the fused attention against the CPU oracle on identical
seeded inputs, at the BASELINE configs' shapes scaled down to what the oracle
finishes in seconds.  Tolerance: every output element
within 2e-3 absolute + 1e-3 relative of the oracle; for bf16/fp16 outputs one
unit in the last place of the output dtype (at |ref|) is added, since the
oracle and the kernel each round their fp32 result to that dtype.""" 

from __future__ import annotations

import math

import pytest
import torch

import smaq_amd as S
from smaq_amd.batch import PagedQuantizedKV, QuantizedKVBatch
from oracle import smaq_ref as R
from tests.conftest import sample_keys

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-3


def assert_attn_close(got: torch.Tensor, ref: torch.Tensor, what: str = ""):
    got = got.detach().float().cpu()
    ref_f = ref.detach().float()
    tol = ATOL + RTOL * ref_f.abs()
    if ref.dtype in (torch.bfloat16, torch.float16):
        # one unit in the last place of the output dtype at |ref|
        mant = 7 if ref.dtype == torch.bfloat16 else 10
        e = torch.floor(torch.log2(ref_f.abs().clamp_min(2.0 ** -14)))
        tol = tol + torch.exp2(e - mant)
    err = (got - ref_f).abs()
    worst = float((err - tol).max())
    print(f"\n[{what}] max|err|={float(err.max()):.3e} worst margin={worst:.3e}")
    assert worst <= 0, f"{what}: {int((err > tol).sum())} elements outside tolerance, max err {float(err.max()):.3e}"


def _pair_scalar(dev, bits, calib_seed=0, hkv=8):
    """(product store, oracle store) with the same calibrated SMAQ metric."""
    calib = sample_keys(64, seed=calib_seed + 60)
    strat = S.SMAQFullMetricScalarStrategy(128, bits=bits, device=dev).fit(calib)
    E, Ei = R.build_metric(R.fit_sigma_centered(calib))
    codec = R.ScalarCodec(128, bits, E=E, E_inv=Ei)
    return (S.CompressedKVStore(128, hkv, key_bits=bits, device=dev, key_strategy=strat),
            R.Store(codec, 128, hkv))


def test_config1_parity(dev):
    """c1: 1 seq, 8 KV heads, D=128, 4096 tokens, fp32, 4-bit SMAQ keys, 2-bit
    values, one decode query per head."""
    st, ref = _pair_scalar(dev, bits=4)
    keys = sample_keys(4096 * 8, seed=101).reshape(4096, 8, 128)
    vals = torch.randn(4096, 8, 128, generator=torch.Generator().manual_seed(102))
    st.append_chunk(keys.to(dev), vals.to(dev))
    ref.append_chunk(keys, vals)
    fg, fr = st.get_flat_cache(), ref.get_flat_cache()
    assert torch.equal(fg.key_q.indices.cpu(), fr.key_q.indices)
    assert torch.equal(fg.key_q.norms.cpu(), fr.key_q.norms)
    assert torch.equal(fg.value_q.data.cpu(), fr.value_q.data)
    q = sample_keys(8, seed=103).reshape(1, 8, 128)
    out = S.compute_hybrid_attention(q.to(dev), st, None, None, 8)
    assert_attn_close(out, R.hybrid_attention(q, ref, None, None, 8), "c1")
    # the score API (SMAQQuantizer.attention_score via the strategy)
    h = 3
    s_got = st.quantizer.attention_score(q[:, h].to(dev), st.quantizer.select_head(fg.key_q, h),
                                         scale=1 / math.sqrt(128), use_kernel=True)
    s_ref = ref.codec.scores(q[:, h], ref.codec.select_head(fr.key_q, h), 1 / math.sqrt(128))
    torch.testing.assert_close(s_got.cpu(), s_ref, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("q_dtype", [torch.bfloat16, torch.float32])
def test_hybrid_recent_window_gqa(dev, q_dtype):
    """GQA 4:1, chunked appends, bf16 recent ring, multi-token query."""
    st, ref = _pair_scalar(dev, bits=3, hkv=2)
    keys = sample_keys(700 * 2, seed=111).reshape(700, 2, 128).to(q_dtype)
    vals = torch.randn(700, 2, 128, generator=torch.Generator().manual_seed(112)).to(q_dtype)
    for a, b in ((0, 128), (128, 256), (256, 700)):
        st.append_chunk(keys[a:b].to(dev), vals[a:b].to(dev))
        ref.append_chunk(keys[a:b], vals[a:b])
    q = sample_keys(3 * 8, seed=113).reshape(3, 8, 128).to(q_dtype)
    kr = sample_keys(37 * 2, seed=114).reshape(37, 2, 128).bfloat16()
    vr = torch.randn(37, 2, 128, generator=torch.Generator().manual_seed(115)).bfloat16()
    out = S.compute_hybrid_attention(q.to(dev), st, kr.to(dev), vr.to(dev), 8)
    assert out.dtype == q_dtype
    assert_attn_close(out, R.hybrid_attention(q, ref, kr, vr, 8), f"recent {q_dtype}")
    # recent-only (history below MIN_HISTORY) and empty
    st2, ref2 = _pair_scalar(dev, bits=3, hkv=2)
    st2.append_chunk(keys[:10].to(dev), vals[:10].to(dev))
    ref2.append_chunk(keys[:10], vals[:10])
    out2 = S.compute_hybrid_attention(q.to(dev), st2, kr.to(dev), vr.to(dev), 8)
    assert_attn_close(out2, R.hybrid_attention(q, ref2, kr, vr, 8), "recent-only")
    z = S.compute_hybrid_attention(q.to(dev), st2, None, None, 8)
    assert torch.equal(z.cpu(), torch.zeros_like(q))


def test_blockvq_hybrid_causal(dev):
    """c4-style: block-VQ keys (block_dim 2, 256 centroids = 4 bits/dim),
    fp16 recent window, outlier channels, causal chunked-prefill queries."""
    hkv, hq, N, Rn, T = 1, 7, 900, 128, 24
    keys = sample_keys(N * hkv, seed=121).reshape(N, hkv, 128)
    outl = torch.tensor([3, 40, 77, 120])
    keys[..., outl] *= 20
    vals = torch.randn(N, hkv, 128, generator=torch.Generator().manual_seed(122))
    calib_q = sample_keys(2048, seed=123)
    calib_k = sample_keys(2048, seed=124)
    calib_k[:, outl] *= 20
    strat = S.SMAQBlockVQStrategy(128, block_dim=2, n_centroids=256, device=dev)
    strat.quantizer.fit(calib_k, calib_q, kmeans_iters=3)
    qz = strat.quantizer
    codec = R.BlockVQCodec(qz.E_blocks.cpu(), qz.centroids.cpu(), qz.decoded_centroids.cpu())
    st = S.CompressedKVStore(128, hkv, device=dev, key_strategy=strat)
    ref = R.Store(codec, 128, hkv)
    st.append_chunk(keys.to(dev), vals.to(dev))
    ref.append_chunk(keys, vals)
    got_idx = st.get_flat_cache().key_q.indices.cpu().long()
    ref_idx = ref.get_flat_cache().key_q.indices
    mism = int((got_idx != ref_idx).sum())
    assert mism <= 2, f"{mism} block-VQ index mismatches"
    if mism:   # score the same codes on both sides
        ref.kc = [R.BlockQ(got_idx.unsqueeze(0), 64, 2)]
    q = sample_keys(T * hq, seed=125).reshape(T, hq, 128)
    kr = sample_keys(Rn * hkv, seed=126).reshape(Rn, hkv, 128).half()
    vr = torch.randn(Rn, hkv, 128, generator=torch.Generator().manual_seed(127)).half()
    pos = torch.arange(N + Rn - T, N + Rn)
    out = S.compute_hybrid_attention(q.to(dev), st, kr.to(dev), vr.to(dev), hq, query_positions=pos.to(dev))
    assert_attn_close(out, R.hybrid_attention(q, ref, kr, vr, hq, query_positions=pos), "blockvq causal")
    out_nc = S.compute_hybrid_attention(q.to(dev), st, kr.to(dev), vr.to(dev), hq)
    assert_attn_close(out_nc, R.hybrid_attention(q, ref, kr, vr, hq), "blockvq no mask")


def _oracle_single(codec, keys, vals, q, hq, hkv):
    st = R.Store(codec, 128, hkv)
    st.append_chunk(keys, vals)
    return R.hybrid_attention(q, st, None, None, hq)


def test_batched_decode_contiguous(dev):
    """c3-style: GQA 32/8, bf16, 3-bit keys, ragged per-sequence lengths."""
    calib = sample_keys(64, seed=130)
    strat = S.SMAQFullMetricScalarStrategy(128, bits=3, device=dev).fit(calib)
    E, Ei = R.build_metric(R.fit_sigma_centered(calib))
    codec = R.ScalarCodec(128, 3, E=E, E_inv=Ei)
    lens = [300, 1000, 64, 517]
    keys = [sample_keys(n * 8, seed=131 + i).reshape(n, 8, 128).bfloat16() for i, n in enumerate(lens)]
    vals = [torch.randn(n, 8, 128, generator=torch.Generator().manual_seed(140 + i)).bfloat16()
            for i, n in enumerate(lens)]
    kvb = QuantizedKVBatch.encode(strat, [k.to(dev) for k in keys], [v.to(dev) for v in vals])
    q = torch.randn(len(lens), 32, 128, generator=torch.Generator().manual_seed(150)).bfloat16()
    out = kvb.attention(q.to(dev))
    for b in range(len(lens)):
        ref = _oracle_single(codec, keys[b], vals[b], q[b:b + 1], 32, 8)
        assert_attn_close(out[b:b + 1], ref, f"batch seq {b}")
    # uniform lengths take the no-table addressing path
    kvu = QuantizedKVBatch.encode(strat, torch.stack([k[:64] for k in keys]).to(dev),
                                  torch.stack([v[:64] for v in vals]).to(dev))
    out_u = kvu.attention(q.to(dev))
    for b in range(len(lens)):
        assert_attn_close(out_u[b:b + 1], _oracle_single(codec, keys[b][:64], vals[b][:64], q[b:b + 1], 32, 8),
                          f"uniform seq {b}")


def test_paged_decode(dev):
    """c5-style: block size 16, shuffled block tables, Student-t keys."""
    calib = sample_keys(64, seed=160)
    strat = S.SMAQFullMetricScalarStrategy(128, bits=3, device=dev).fit(calib)
    E, Ei = R.build_metric(R.fit_sigma_centered(calib))
    codec = R.ScalarCodec(128, 3, E=E, E_inv=Ei)
    g = torch.Generator().manual_seed(161)
    lens = [int(x) for x in torch.randint(20, 400, (5,), generator=g)]
    bs = 16
    nblk = [(n + bs - 1) // bs for n in lens]
    perm = torch.randperm(sum(nblk) + 7, generator=g)
    table = torch.zeros(len(lens), max(nblk), dtype=torch.int32)
    o = 0
    for b, nb in enumerate(nblk):
        table[b, :nb] = perm[o:o + nb].to(torch.int32)
        o += nb
    tdist = torch.distributions.StudentT(3.0)
    torch.manual_seed(162)
    keys = [tdist.sample((n, 8, 128)).bfloat16() for n in lens]
    vals = [torch.randn(n, 8, 128, generator=g).bfloat16() for n in lens]
    pk = PagedQuantizedKV.encode(strat, [k.to(dev) for k in keys], [v.to(dev) for v in vals], table.to(dev),
                                 num_blocks=sum(nblk) + 7, block_size=bs)
    q = torch.randn(len(lens), 32, 128, generator=g).bfloat16()
    out = pk.attention(q.to(dev))
    for b in range(len(lens)):
        assert_attn_close(out[b:b + 1], _oracle_single(codec, keys[b], vals[b], q[b:b + 1], 32, 8), f"paged {b}")


def test_length_tensors_any_integer_dtype_or_device(dev):
    """Per-sequence lengths reach the kernels as int64 on the device whatever
    the caller hands in: int32 (vLLM's seq_lens) and host tensors give the
    same output as device int64, bit for bit."""
    calib = sample_keys(64, seed=170)
    strat = S.SMAQFullMetricScalarStrategy(128, bits=3, device=dev).fit(calib)
    lens = [200, 90, 333]
    keys = [sample_keys(n * 8, seed=171 + i).reshape(n, 8, 128).bfloat16().to(dev) for i, n in enumerate(lens)]
    vals = [torch.randn(n, 8, 128, generator=torch.Generator().manual_seed(175 + i)).bfloat16().to(dev)
            for i, n in enumerate(lens)]
    kvb = QuantizedKVBatch.encode(strat, keys, vals)
    g = torch.Generator().manual_seed(178)
    q = torch.randn(3, 32, 128, generator=g).bfloat16().to(dev)
    rk = torch.randn(3, 16, 8, 128, generator=g).bfloat16().to(dev)
    rv = torch.randn(3, 16, 8, 128, generator=g).bfloat16().to(dev)
    base = kvb.attention(q, recent_k=rk, recent_v=rv, recent_len=torch.tensor([16, 3, 9], device=dev))
    for rl in (torch.tensor([16, 3, 9], dtype=torch.int32, device=dev), torch.tensor([16, 3, 9], dtype=torch.int32),
               torch.tensor([16, 3, 9])):
        got = kvb.attention(q, recent_k=rk, recent_v=rv, recent_len=rl)
        assert torch.equal(got, base), f"recent_len {rl.dtype} on {rl.device}"
    kvb.hist_len = kvb.hist_len.to(torch.int32).cpu()
    kvb.seq_start = kvb.seq_start.to(torch.int32)
    got = kvb.attention(q, recent_k=rk, recent_v=rv, recent_len=torch.tensor([16, 3, 9], device=dev))
    assert torch.equal(got, base), "int32 host hist_len / int32 seq_start"
    with pytest.raises(ValueError):
        kvb.attention(q, recent_k=rk, recent_v=rv, recent_len=torch.tensor([16.0, 3.0, 9.0], device=dev))


def test_store_mixed_dtype_appends(dev):
    """Chunks of bf16, then fp16, then fp32 keys/values appended to one store:
    the columns widen to the promoted dtype (bf16 + fp16 -> fp32) as the
    reference's torch.cat of its quantised chunks does (smaq/store.py:97-114),
    so the flat cache equals the oracle's -- dtypes included, value bytes,
    norms and value metadata bit for bit, key codes apart from at most two
    boundary ties -- and the attention output matches."""
    st, ref = _pair_scalar(dev, bits=3, hkv=2)
    n = [100, 60, 50]
    keys = sample_keys(sum(n) * 2, seed=131).reshape(sum(n), 2, 128)
    vals = torch.randn(sum(n), 2, 128, generator=torch.Generator().manual_seed(132))
    a = 0
    for cnt, dt in zip(n, (torch.bfloat16, torch.float16, torch.float32)):
        k, v = keys[a:a + cnt].to(dt), vals[a:a + cnt].to(dt)
        st.append_chunk(k.to(dev), v.to(dev))
        ref.append_chunk(k, v)
        a += cnt
    fg, fr = st.get_flat_cache(), ref.get_flat_cache()
    assert fg.key_q.norms.dtype == fr.key_q.norms.dtype == torch.float32
    assert fg.value_q.scales.dtype == fr.value_q.scales.dtype == torch.float32
    # (a code byte may differ only at a boundary tie; none is expected here)
    assert int((fg.key_q.indices.cpu() != fr.key_q.indices).sum()) <= 2
    assert torch.equal(fg.key_q.norms.cpu(), fr.key_q.norms)
    assert torch.equal(fg.value_q.data.cpu(), fr.value_q.data)
    assert torch.equal(fg.value_q.scales.cpu(), fr.value_q.scales)
    assert torch.equal(fg.value_q.zeros.cpu(), fr.value_q.zeros)
    q = sample_keys(8, seed=133).reshape(1, 8, 128)
    out = S.compute_hybrid_attention(q.to(dev), st, None, None, 8)
    assert_attn_close(out, R.hybrid_attention(q, ref, None, None, 8), "mixed-dtype store")


def test_compute_hybrid_attention_keeps_its_plan(dev):
    """Repeated compute_hybrid_attention calls over an unchanged store re-use
    the launch kept on the store (a new recent window of the same shape is
    rebound, not rebuilt), each call returns its own output tensor, and an
    append replaces the plan; every result equals the oracle's."""
    st, ref = _pair_scalar(dev, bits=3, hkv=2)
    keys = sample_keys(400 * 2, seed=151).reshape(400, 2, 128)
    vals = torch.randn(400, 2, 128, generator=torch.Generator().manual_seed(152))
    st.append_chunk(keys[:300].to(dev), vals[:300].to(dev))
    ref.append_chunk(keys[:300], vals[:300])
    g = torch.Generator().manual_seed(153)
    outs, plans = [], []
    for step in range(3):
        q = sample_keys(8, seed=160 + step).reshape(1, 8, 128)
        kr = torch.randn(5, 2, 128, generator=g).bfloat16()
        vr = torch.randn(5, 2, 128, generator=g).bfloat16()
        out = S.compute_hybrid_attention(q.to(dev), st, kr.to(dev), vr.to(dev), 8)
        assert_attn_close(out, R.hybrid_attention(q, ref, kr, vr, 8), f"kept plan step {step}")
        outs.append(out)
        plans.append(st._fused_plan[1])
    assert plans[0] is plans[1] is plans[2]
    assert outs[0].data_ptr() != outs[1].data_ptr()
    st.append_chunk(keys[300:].to(dev), vals[300:].to(dev))
    ref.append_chunk(keys[300:], vals[300:])
    q = sample_keys(8, seed=170).reshape(1, 8, 128)
    out = S.compute_hybrid_attention(q.to(dev), st, None, None, 8)
    assert st._fused_plan[1] is not plans[0]
    assert_attn_close(out, R.hybrid_attention(q, ref, None, None, 8), "after append")
