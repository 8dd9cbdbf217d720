"""GPU parity of the matrix-core decode kernel (attention_mfma.hip) against
the CPU oracle, and against the generic kernels, over the decode shapes it
serves: 3/4-bit scalar keys, 2-bit values, GQA 1..4, contiguous and paged
histories, ragged lengths that are not multiples of the 32-token tile.
Tolerance as tests/test_gpu_attention.py (2e-3 abs + 1e-3 rel, + 1 output ulp
for 16-bit outputs)."""

from __future__ import annotations

import pytest
import torch

import smaq_amd as S
from smaq_amd.batch import PagedQuantizedKV, QuantizedKVBatch
from oracle import smaq_ref as R
from tests.conftest import sample_keys
from tests.test_gpu_attention import assert_attn_close

pytestmark = pytest.mark.gpu


def _codec_pair(dev, bits, seed):
    calib = sample_keys(64, seed=seed)
    strat = S.SMAQFullMetricScalarStrategy(128, bits=bits, device=dev).fit(calib)
    E, Ei = R.build_metric(R.fit_sigma_centered(calib))
    return strat, R.ScalarCodec(128, bits, E=E, E_inv=Ei)


def _oracle(codec, k, v, q, hq, hkv):
    st = R.Store(codec, 128, hkv)
    st.append_chunk(k, v)
    return R.hybrid_attention(q, st, None, None, hq)


@pytest.mark.parametrize("bits,g,dtype", [(3, 4, torch.bfloat16), (4, 1, torch.float32), (3, 2, torch.float16),
                                          (4, 3, torch.bfloat16)])
def test_mfma_decode_contiguous(dev, bits, g, dtype):
    strat, codec = _codec_pair(dev, bits, 200 + bits * 10 + g)
    hkv = 4
    lens = [300, 1000, 64, 517, 17, 2049]
    gen = torch.Generator().manual_seed(bits * 7 + g)
    keys = [sample_keys(n * hkv, seed=210 + i).reshape(n, hkv, 128).to(dtype) for i, n in enumerate(lens)]
    vals = [torch.randn(n, hkv, 128, generator=gen).to(dtype) for n in lens]
    kvb = QuantizedKVBatch.encode(strat, [k.to(dev) for k in keys], [v.to(dev) for v in vals])
    q = torch.randn(len(lens), hkv * g, 128, generator=gen).to(dtype)
    out_m = kvb.attention(q.to(dev), impl=2)
    out_g = kvb.attention(q.to(dev), impl=1)
    for b in range(len(lens)):
        ref = _oracle(codec, keys[b], vals[b], q[b:b + 1], hkv * g, hkv)
        assert_attn_close(out_m[b:b + 1], ref, f"mfma {bits}b g={g} seq {b} len {lens[b]}")
        assert_attn_close(out_g[b:b + 1], ref, f"generic {bits}b g={g} seq {b}")


def test_mfma_decode_paged(dev):
    strat, codec = _codec_pair(dev, 3, 260)
    gen = torch.Generator().manual_seed(261)
    lens = [int(x) for x in torch.randint(1, 700, (6,), generator=gen)]
    bs = 16
    nblk = [(n + bs - 1) // bs for n in lens]
    nphys = sum(nblk) + 11
    perm = torch.randperm(nphys, generator=gen)
    table = torch.zeros(len(lens), max(nblk), dtype=torch.int32)
    o = 0
    for b, nb in enumerate(nblk):
        table[b, :nb] = perm[o:o + nb].to(torch.int32)
        o += nb
    keys = [sample_keys(n * 8, seed=270 + b).reshape(n, 8, 128).bfloat16() for b, n in enumerate(lens)]
    vals = [torch.randn(n, 8, 128, generator=gen).bfloat16() for n in lens]
    pk = PagedQuantizedKV.encode(strat, [k.to(dev) for k in keys], [v.to(dev) for v in vals], table.to(dev),
                                 num_blocks=nphys, block_size=bs)
    q = torch.randn(len(lens), 32, 128, generator=gen).bfloat16()
    out = pk.attention(q.to(dev), impl=2)
    for b in range(len(lens)):
        assert_attn_close(out[b:b + 1], _oracle(codec, keys[b], vals[b], q[b:b + 1], 32, 8), f"paged mfma {b}")


def test_mfma_decode_peaked_scores(dev):
    """Large query norms (sharp softmax): the hi/lo splits keep scores exact
    enough that the winning tokens' weights match."""
    strat, codec = _codec_pair(dev, 4, 280)
    n = 1500
    keys = sample_keys(n * 2, seed=281).reshape(n, 2, 128)
    vals = torch.randn(n, 2, 128, generator=torch.Generator().manual_seed(282))
    q = sample_keys(8, seed=283).reshape(1, 8, 128) * 40.0
    kvb = QuantizedKVBatch.encode(strat, [keys.to(dev)], [vals.to(dev)])
    out = kvb.attention(q.to(dev), impl=2)
    assert_attn_close(out, _oracle(codec, keys, vals, q, 8, 2), "peaked")


def test_mfma_unsupported_shape_raises(dev):
    strat, _ = _codec_pair(dev, 3, 290)
    keys = sample_keys(64 * 2, seed=291).reshape(64, 2, 128)
    kvb = QuantizedKVBatch.encode(strat, [keys.to(dev)], [keys.to(dev)])
    q = torch.randn(1, 2, 16, 128)         # 2 query tokens: not a decode shape
    with pytest.raises(RuntimeError, match="matrix-core"):
        kvb.attention(q.to(dev), impl=2)
