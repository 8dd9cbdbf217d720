"""SMAQKVCache (smaq/kv_cache.py:106-290) on the GPU against the CPU oracle.

The cache keeps the newest ``buffer_size`` tokens exact and compresses the
rest through the GPU key codec and value packer; its scores are
[compressed, exact] along the key axis without a softmax, and ``attend``
applies weights to the dequantised and exact values.  The oracle encodes the
same flushed tokens in one pass (codes are per row, so chunking does not
change them).  Codes bit-exact apart from counted boundary ties (each within
1e-6 relative of a decision boundary, at most 2), norms and value bytes
bit-exact; scores within 2e-4 abs +
1e-4 rel (as the scalar codec's score test); attended outputs within 2e-3 abs
+ 1e-3 rel.
"""

from __future__ import annotations

import pytest
import torch

import smaq_amd as S
from oracle import smaq_ref as R
from tests.conftest import sample_keys
from tests.test_gpu_codecs import _ties_ok

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits,dtype", [(3, torch.float32), (4, torch.bfloat16)])
def test_kv_cache_prefill_append_scores_attend(dev, bits, dtype):
    calib = sample_keys(64, seed=110)
    strat = S.SMAQFullMetricScalarStrategy(128, bits=bits, device=dev).fit(calib)
    E, Ei = R.build_metric(R.fit_sigma_centered(calib))
    c, _, db = R.scalar_tables(bits)
    buf = 32
    cache = S.SMAQKVCache(128, buffer_size=buf, device=dev, key_strategy=strat)
    B, H, T0, T1 = 1, 4, 100, 45
    keys = sample_keys(B * H * (T0 + T1), seed=111).reshape(B, H, T0 + T1, 128).to(dtype)
    vals = torch.randn(B, H, T0 + T1, 128, generator=torch.Generator().manual_seed(112)).to(dtype)
    cache.prefill(keys[:, :, :T0].to(dev), vals[:, :, :T0].to(dev))
    assert cache.key_quantized.indices.shape[-2] == T0 - buf
    for t in range(T0, T0 + T1, 5):   # decode-sized appends, each flushing past the buffer
        cache.append(keys[:, :, t:t + 5].to(dev), vals[:, :, t:t + 5].to(dev))
    n = T0 + T1
    nq = n - buf
    assert cache.get_seq_length() == n
    assert cache.key_buffer.shape[-2] == buf and cache.key_quantized.indices.shape[-2] == nq

    ref_k = R.scalar_encode(keys[:, :, :nq], E, db, bits)
    ref_v = R.quantize_values(vals[:, :, :nq], bits=2, group_size=32)
    got_codes = R.unpack_codes(cache.key_quantized.indices.cpu(), bits, 128)
    assert _ties_ok(got_codes, R.unpack_codes(ref_k.indices, bits, 128),
                    R.scalar_y(keys[:, :, :nq], E), db) <= 2
    assert torch.equal(cache.key_quantized.norms.cpu(), ref_k.norms)
    assert torch.equal(cache.value_quantized.data.cpu(), ref_v.data)
    assert torch.equal(cache.value_quantized.scales.cpu(), ref_v.scales)
    assert torch.equal(cache.value_quantized.zeros.cpu(), ref_v.zeros)

    query = sample_keys(B * H * 2, seed=113).reshape(B, H, 2, 128).to(dtype)
    scale = 0.09
    s = cache.attention_scores(query.to(dev), scale=scale).cpu().float()
    s_ref = torch.cat([R.smaq_scores(query, ref_k, c, Ei, 128, scale=scale).float(),
                       (torch.matmul(query.float(), keys[:, :, nq:].float().transpose(-2, -1)) * scale)], dim=-1)
    assert s.shape == (B, H, 2, n)
    torch.testing.assert_close(s, s_ref, atol=2e-4 if dtype == torch.float32 else 2e-2,
                               rtol=1e-4 if dtype == torch.float32 else 1e-2)

    if dtype == torch.float32:
        # (like the reference, attend multiplies the weights with fp32
        # dequantised values, so it is exercised with fp32 weights)
        w = torch.softmax(s_ref, dim=-1)
        out = cache.attend(w.to(dev)).cpu()
        v_hat = R.dequantize_values(ref_v, 32)
        ref = torch.matmul(w[..., :nq], v_hat) + torch.matmul(w[..., nq:], vals[:, :, nq:])
        assert bool(((out - ref).abs() <= 2e-3 + 1e-3 * ref.abs()).all()), float((out - ref).abs().max())

    mem = cache.memory_bytes()
    assert mem["quantized_keys"] == strat.memory_bytes(cache.key_quantized)
    assert mem["quantized_values"] == ref_v.data.numel() + 2 * ref_v.scales.numel() + 2 * ref_v.zeros.numel()
    assert mem["buffer"] == 2 * 2 * B * H * buf * 128
    assert mem["total"] == mem["quantized_keys"] + mem["quantized_values"] + mem["buffer"]


def test_kv_cache_short_prefill_stays_exact(dev):
    cache = S.SMAQKVCache(128, buffer_size=64, device=dev)
    k = torch.randn(1, 2, 40, 128, device=dev)
    cache.prefill(k, k)
    assert cache.key_quantized is None and cache.key_buffer.shape[-2] == 40
    q = torch.randn(1, 2, 1, 128, device=dev)
    s = cache.attention_scores(q)
    torch.testing.assert_close(s, torch.matmul(q, k.transpose(-2, -1).contiguous()) / 128 ** 0.5)
    w = torch.softmax(s, dim=-1)
    torch.testing.assert_close(cache.attend(w), torch.matmul(w, k))


def test_allocated_bytes_reports_capacity(dev):
    """allocated_bytes (not in the reference) counts what the device holds:
    the compressed columns at their capacity (doubling growth, so between the
    reference's logical bytes and twice them plus the minimum allocation) and
    the exact window's double-size buffers; memory_bytes keeps the
    reference's logical count."""
    calib = sample_keys(64, seed=140)
    strat = S.SMAQFullMetricScalarStrategy(128, bits=3, device=dev).fit(calib)
    st = S.CompressedKVStore(128, 2, key_bits=3, device=dev, key_strategy=strat)
    keys = sample_keys(700 * 2, seed=141).reshape(700, 2, 128).bfloat16()
    vals = torch.randn(700, 2, 128, generator=torch.Generator().manual_seed(142)).bfloat16()
    for a, b in ((0, 300), (300, 301), (301, 700)):
        st.append_chunk(keys[a:b].to(dev), vals[a:b].to(dev))
    fc = st.get_flat_cache()
    filled = sum(t.nelement() * t.element_size() for t in (fc.key_q.indices, fc.key_q.norms, fc.value_q.data,
                                                          fc.value_q.scales, fc.value_q.zeros))
    per_row = filled // (700 * 2)
    alloc = st.allocated_bytes()
    assert filled <= alloc <= 2 * filled + 256 * 2 * per_row, (filled, alloc)
    assert st.memory_bytes() <= filled
    cache = S.SMAQKVCache(128, buffer_size=32, device=dev, key_strategy=strat)
    cache.prefill(keys[:200].transpose(0, 1).unsqueeze(0).to(dev), vals[:200].transpose(0, 1).unsqueeze(0).to(dev))
    exact = 2 * (2 * 32 * 2 * 128 * 2)                      # keys + values, twice the window, bf16
    assert cache.allocated_bytes() >= exact + cache.memory_bytes()["quantized_keys"]


@pytest.mark.parametrize("bits,group", [(2, 32), (4, 32), (8, 32), (2, 16)])
@pytest.mark.parametrize("sdtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("N", [0, 1, 37, 3000])
def test_apply_values_matches_dequantized_matmul(dev, bits, group, sdtype, N):
    """smaq_apply_values (the compressed term of SMAQKVCache.attend,
    smaq/kv_cache.py:247-252) against the oracle's fp32 dequantised values
    (smaq/kv_cache.py:94-103) times the weights in float64: within 2e-3 abs +
    1e-3 rel, and within 1e-5 of the float64 sum (fp32 accumulation); 6 query
    rows (more than one 4-row pass), several token splits at N = 3000, and a
    weight view sliced out of a wider matrix as attend passes it."""
    from smaq_amd import _native
    B, H, nq = 2, 3, 6
    g = torch.Generator().manual_seed(150 + bits + N)
    vals = (torch.randn(B, H, N, 128, generator=g) * 3.0).to(sdtype)
    ref_v = R.quantize_values(vals, bits=bits, group_size=group)
    w_all = torch.softmax(torch.randn(B, H, nq, N + 9, generator=g) * 2.0, dim=-1)
    w = w_all[..., 4:4 + N]
    v_hat = R.dequantize_values(ref_v, group)
    ref = torch.matmul(w.double(), v_hat.double())
    got = _native.apply_values(w_all.to(dev)[..., 4:4 + N], ref_v.data.to(dev), ref_v.scales.to(dev),
                               ref_v.zeros.to(dev), bits, group).cpu()
    assert got.shape == (B, H, nq, 128) and got.dtype == torch.float32
    err = (got.double() - ref).abs()
    assert bool((err <= 2e-3 + 1e-3 * ref.abs()).all()), float(err.max())
    assert float(err.max()) <= 1e-5 * max(1.0, float(ref.abs().max())), float(err.max())
