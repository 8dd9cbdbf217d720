"""Pins the oracle's hybrid attention (smaq/score.py semantics) against the
float64 closed form softmax(q [K_hat; K_rec]^T * scale) [V_hat; V_rec] on
the dequantised tensors, plus the special cases the reference encodes.  CPU."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import smaq_ref as R
from tests.conftest import sample_keys, spectral_sigma


def _codec(bits=3, seed=0):
    sigma, _, _ = spectral_sigma(128, seed)
    E, Ei = R.build_metric(R.fit_sigma_centered(sample_keys(64, seed=seed + 50)))
    return R.ScalarCodec(128, bits, E=E, E_inv=Ei)


def _closed_form(query, khat, vhat, kr, vr, g, scale, positions=None, n_all=None):
    """float64 softmax attention per query head; khat/vhat [Hkv, N, D]."""
    T, Hq, D = query.shape
    hkv = khat.shape[0] if khat is not None else kr.shape[1]
    out = np.zeros((T, Hq, D))
    for hq in range(Hq):
        h = hq // g
        ks, vs = [], []
        if khat is not None:
            ks.append(khat[h].double().numpy())
            vs.append(vhat[h].double().numpy())
        if kr is not None:
            ks.append(kr[:, h].double().numpy())
            vs.append(vr[:, h].double().numpy())
        K, V = np.concatenate(ks), np.concatenate(vs)
        for t in range(T):
            s = K @ query[t, hq].double().numpy() * scale
            if positions is not None:
                pos = np.arange(len(s)) if khat is not None else n_all + np.arange(len(s))
                s = np.where(pos > positions[t], -np.inf, s)
            w = np.exp(s - s.max())
            w /= w.sum()
            out[t, hq] = w @ V
    return out


@pytest.mark.parametrize("with_recent", [False, True])
def test_hybrid_matches_closed_form(with_recent):
    codec = _codec()
    hkv, hq, T, N, R_ = 2, 6, 3, 200, 17
    st = R.Store(codec, 128, hkv)
    keys = sample_keys(N * hkv, seed=3).reshape(N, hkv, 128)
    vals = torch.randn(N, hkv, 128, generator=torch.Generator().manual_seed(4))
    st.append_chunk(keys[:120], vals[:120])
    st.append_chunk(keys[120:], vals[120:])
    q = sample_keys(T * hq, seed=5).reshape(T, hq, 128)
    kr = sample_keys(R_ * hkv, seed=6).reshape(R_, hkv, 128) if with_recent else None
    vr = torch.randn(R_, hkv, 128, generator=torch.Generator().manual_seed(7)) if with_recent else None
    out = R.hybrid_attention(q, st, kr, vr, hq)
    flat = st.get_flat_cache()
    khat = codec.dequantize(flat.key_q)
    vhat = R.dequantize_values(flat.value_q, 32)
    want = _closed_form(q, khat, vhat, kr, vr, hq // hkv, 1 / math.sqrt(128))
    np.testing.assert_allclose(out.double().numpy(), want, atol=2e-5, rtol=1e-4)


def test_min_history_rule_and_empty():
    codec = _codec()
    st = R.Store(codec, 128, 1)
    q = sample_keys(2, seed=8).reshape(1, 2, 128)
    assert torch.equal(R.hybrid_attention(q, st, None, None, 2), torch.zeros(1, 2, 128))
    st.append_chunk(sample_keys(15, seed=9).reshape(15, 1, 128), torch.randn(15, 1, 128))
    assert torch.equal(R.hybrid_attention(q, st, None, None, 2), torch.zeros(1, 2, 128))   # 15 < 16
    kr = sample_keys(4, seed=10).reshape(4, 1, 128)
    vr = torch.randn(4, 1, 128)
    out = R.hybrid_attention(q, st, kr, vr, 2)
    want = _closed_form(q, None, None, kr, vr, 2, 1 / math.sqrt(128))
    np.testing.assert_allclose(out.double().numpy(), want, atol=1e-5)


def test_causal_extension_closed_form():
    codec = _codec()
    hkv, hq, N, R_ = 1, 2, 40, 8
    st = R.Store(codec, 128, hkv)
    st.append_chunk(sample_keys(N, seed=11).reshape(N, 1, 128), torch.randn(N, 1, 128))
    q = sample_keys(3 * hq, seed=12).reshape(3, hq, 128)
    kr = sample_keys(R_, seed=13).reshape(R_, 1, 128)
    vr = torch.randn(R_, 1, 128)
    pos = torch.tensor([5, 41, 47])
    out = R.hybrid_attention(q, st, kr, vr, hq, query_positions=pos)
    flat = st.get_flat_cache()
    want = _closed_form(q, codec.dequantize(flat.key_q), R.dequantize_values(flat.value_q, 32), kr, vr, hq,
                        1 / math.sqrt(128), positions=pos.numpy())
    np.testing.assert_allclose(out.double().numpy(), want, atol=2e-5, rtol=1e-4)


def test_bf16_output_casts_each_part():
    """out = bf16(bf16(o_hist) + bf16(o_recent)) (smaq/score.py:70-72)."""
    codec = _codec()
    st = R.Store(codec, 128, 1)
    st.append_chunk(sample_keys(64, seed=14).reshape(64, 1, 128).bfloat16(), torch.randn(64, 1, 128).bfloat16())
    q = sample_keys(4, seed=15).reshape(1, 4, 128).bfloat16()
    kr = sample_keys(5, seed=16).reshape(5, 1, 128).bfloat16()
    vr = torch.randn(5, 1, 128).bfloat16()
    out = R.hybrid_attention(q, st, kr, vr, 4)
    assert out.dtype == torch.bfloat16
    flat = st.get_flat_cache()
    want = _closed_form(q.float(), codec.dequantize(flat.key_q), R.dequantize_values(flat.value_q, 32),
                        kr.float(), vr.float(), 4, 1 / math.sqrt(128))
    np.testing.assert_allclose(out.double().numpy(), want, atol=2e-2, rtol=2e-2)


def test_gqa_head_mapping():
    """Query head h reads KV head h // g: swapping KV heads permutes outputs."""
    codec = _codec()
    keys = sample_keys(2 * 50, seed=17).reshape(50, 2, 128)
    vals = torch.randn(50, 2, 128)
    q = sample_keys(4, seed=18).reshape(1, 4, 128)
    a, b = R.Store(codec, 128, 2), R.Store(codec, 128, 2)
    a.append_chunk(keys, vals)
    b.append_chunk(keys.flip(1), vals.flip(1))
    oa = R.hybrid_attention(q, a, None, None, 4)
    ob = R.hybrid_attention(q[:, [2, 3, 0, 1]], b, None, None, 4)
    assert torch.allclose(oa[:, [2, 3, 0, 1]], ob, atol=1e-6)


def test_ring_overflow_semantics():
    ring = R.Ring(4, 1, 2, dtype=torch.float32)
    x = torch.arange(20, dtype=torch.float32).reshape(10, 1, 2)
    assert ring.write(x[:3], x[:3], 3) is None
    ov = ring.write(x[3:6], x[3:6], 3)      # fills to 4, then spills all 4, keeps 2
    assert ov is not None and torch.equal(ov[0], x[:4]) and ring.pos == 2
    assert torch.equal(ring.peek()[0], x[4:6])
