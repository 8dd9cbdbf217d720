"""BASELINE configs at their full sizes on the GPU, checked through
properties that do not depend on size (the oracle cannot run whole
workloads in seconds):

* rows are encoded independently, so a random sample of the encoded rows
  must equal the oracle's encoding of those rows (codes up to counted
  boundary / argmin ties, value bytes bit for bit);
* sequences attend independently, so sampled sequences of the full batch
  must match the oracle run on that sequence alone (same tolerance as
  tests/test_gpu_attention.py).

c3: 32 sequences x 32768 tokens x 8 KV heads (3-bit scalar keys, bf16).
c2: 16 x 32768 x 8 token-heads, block-VQ (8-dim blocks, 256 centroids).
c5: 256 paged sequences, lengths U[1024, 16384], 16-token blocks,
    Student-t(3) keys.
c2: codebook fitted on 65536 samples with 20 Lloyd iterations.
c4: 2048 causal queries (28 heads) over 65408 block-VQ history tokens
    (block_dim 2) + 128 fp16 recent tokens; 8 query tokens from each of the
    8 256-token query blocks against the oracle run on those queries alone.
"""

from __future__ import annotations

import pytest
import torch

import smaq_amd as S
from smaq_amd import _native
from smaq_amd.batch import PagedQuantizedKV, QuantizedKVBatch, _encode_rows
from smaq_amd.synthetic import sample_keys as dev_sample_keys
from smaq_amd.synthetic import paged_lengths_and_table, student_t
from smaq_amd.synthetic import sample_values as dev_sample_values
from oracle import smaq_ref as R
from tests.conftest import sample_keys
from tests.test_gpu_attention import assert_attn_close
from tests.test_gpu_codecs import _check_vq_against_oracle, _ties_ok

pytestmark = pytest.mark.gpu


class _FlatStore:
    """The oracle store interface over a flat cache built from GPU codes."""

    def __init__(self, flat, codec, head_dim, num_kv_heads):
        self.flat, self.codec = flat, codec
        self.head_dim, self.num_kv_heads, self.value_group_size = head_dim, num_kv_heads, 32

    def get_flat_cache(self):
        return self.flat


def test_c3_full_size_decode(dev):
    B, N, Hq, Hkv, D, bits = 32, 32768, 32, 8, 128, 3
    calib = sample_keys(64, seed=3)
    strat = S.SMAQFullMetricScalarStrategy(D, bits=bits, device=dev).fit(calib)
    keys = dev_sample_keys(B * N * Hkv, seed=11, device=dev, dtype=torch.bfloat16).view(B, N, Hkv, D)
    vals = dev_sample_values(B * N * Hkv, seed=12, device=dev, dtype=torch.bfloat16).view(B, N, Hkv, D)
    kvb = QuantizedKVBatch.encode(strat, keys, vals, value_bits=2, value_group=32)
    q = torch.randn(B, Hq, D, generator=torch.Generator(device=dev).manual_seed(13), device=dev).bfloat16()
    out = kvb.attention(q, impl=2).cpu()
    E, Ei = R.build_metric(R.fit_sigma_centered(calib))
    c, _, db = R.scalar_tables(bits)
    # sampled rows: codes and value bytes against the oracle
    g = torch.Generator().manual_seed(160)
    n = 4096
    bs_, ts_, hs_ = (torch.randint(0, B, (n,), generator=g), torch.randint(0, N, (n,), generator=g),
                     torch.randint(0, Hkv, (n,), generator=g))
    k_s = keys[bs_.to(dev), ts_.to(dev), hs_.to(dev)].cpu()
    v_s = vals[bs_.to(dev), ts_.to(dev), hs_.to(dev)].cpu()
    flat_rows = (bs_ * N + ts_).to(dev)
    got_codes = kvb.codes[hs_.to(dev), flat_rows].cpu()
    ref = R.scalar_encode(k_s, E, db, bits)
    assert _ties_ok(R.unpack_codes(got_codes, bits, D), R.unpack_codes(ref.indices, bits, D),
                    R.scalar_y(k_s, E), db) <= 2
    assert torch.equal(kvb.norms[hs_.to(dev), flat_rows].cpu(), ref.norms)
    ref_v = R.quantize_values(v_s, bits=2, group_size=32)
    assert torch.equal(kvb.v_data[hs_.to(dev), flat_rows].cpu(), ref_v.data)
    assert torch.equal(kvb.v_scales[hs_.to(dev), flat_rows].cpu(), ref_v.scales)
    # whole sequences against the oracle on that sequence alone
    codec = R.ScalarCodec(D, bits, E=E, E_inv=Ei)
    for b in (0, B - 1):
        st = R.Store(codec, D, Hkv)
        st.append_chunk(keys[b].cpu(), vals[b].cpu())
        ref_o = R.hybrid_attention(q[b:b + 1].cpu(), st, None, None, Hq)
        assert_attn_close(out[b:b + 1], ref_o, f"c3 full size, sequence {b}")


def test_c2_full_size_encode(dev):
    seqs, toks, Hkv, D = 16, 32768, 8, 128
    rows = seqs * toks * Hkv
    # the bench's codebook: k-means++ on 65536 seeded samples, 20 Lloyd
    # iterations (device fit; the encoder is checked against the oracle for
    # whatever codebook it is given)
    vq = S.SMAQBlockVQ(D, block_dim=8, device=dev)
    vq.fit(sample_keys(65536, seed=21), sample_keys(65536, seed=22), kmeans_iters=20, on_device=True)
    Eb, C = vq.E_blocks.cpu(), vq.centroids.cpu()
    keys = dev_sample_keys(rows, seed=23, device=dev, dtype=torch.bfloat16).view(seqs, toks, Hkv, D)
    vals = dev_sample_values(rows, seed=24, device=dev, dtype=torch.bfloat16).view(seqs, toks, Hkv, D)
    vq.tie_counter = _native.TieCounter(dev)
    idx = vq.quantize(keys).indices.reshape(rows, 16)
    ties = vq.tie_counter.value()
    pv = S.quantize_values(vals, bits=2, group_size=32)
    g = torch.Generator().manual_seed(161)
    sel = torch.randint(0, rows, (8192,), generator=g)
    k_s = keys.reshape(rows, D)[sel.to(dev)].cpu()
    ref = R.blockvq_encode(k_s, Eb, C).indices
    # every tie of the whole launch is counted; the sample's mismatches must be ties
    _check_vq_against_oracle(idx[sel.to(dev)].cpu().long(), ref, k_s, Eb, C, ties, "c2 full size, 8192 sampled rows")
    assert ties < rows * 16 * 1e-3
    ref_v = R.quantize_values(vals.reshape(rows, D)[sel.to(dev)].cpu(), bits=2, group_size=32)
    assert torch.equal(pv.data.reshape(rows, 32)[sel.to(dev)].cpu(), ref_v.data)
    assert torch.equal(pv.scales.reshape(rows, 4)[sel.to(dev)].cpu(), ref_v.scales)
    assert torch.equal(pv.zeros.reshape(rows, 4)[sel.to(dev)].cpu(), ref_v.zeros)


def test_c5_full_size_paged(dev):
    B, Hq, Hkv, D, bs = 256, 32, 8, 128, 16
    lens, table, total = paged_lengths_and_table(B, bs, seed=4)
    calib = sample_keys(64, seed=3)
    strat = S.SMAQFullMetricScalarStrategy(D, bits=3, device=dev).fit(calib)
    # BASELINE c5: Student-t(3) keys per channel (the bench's draw)
    gd = torch.Generator(device=dev).manual_seed(41)
    kp = torch.empty(total, bs, Hkv, D, dtype=torch.bfloat16, device=dev)
    vp = torch.empty_like(kp)
    for i in range(0, total, 8192):
        j = min(total, i + 8192)
        kp[i:j] = student_t((j - i, bs, Hkv, D), gd, dev)
        vp[i:j] = torch.randn((j - i, bs, Hkv, D), generator=gd, device=dev).to(torch.bfloat16)
    codes, norms, vd, vsc, vz = _encode_rows(strat, kp.permute(0, 2, 1, 3), vp.permute(0, 2, 1, 3), 2, 32)
    del kp, vp
    pk = PagedQuantizedKV(strat, codes, norms, vd, vsc, vz, table.to(dev), lens.tolist(), bs, 2, 32)
    q = torch.randn(B, Hq, D, generator=torch.Generator(device=dev).manual_seed(43), device=dev).bfloat16()
    out = pk.attention(q, impl=2).cpu()
    E, Ei = R.build_metric(R.fit_sigma_centered(calib))
    codec = R.ScalarCodec(D, 3, E=E, E_inv=Ei)
    order = torch.argsort(lens)
    for b in (int(order[0]), int(order[B // 2]), int(order[-1])):
        L = int(lens[b])
        nb = (L + bs - 1) // bs
        blocks = table[b, :nb].long().to(dev)

        def gather(x):  # pool [blocks, Hkv, bs, ...] -> [Hkv, L, ...]
            return x[blocks].transpose(0, 1).reshape(Hkv, nb * bs, *x.shape[3:])[:, :L].cpu().contiguous()

        flat = R.FlatCache(R.ScalarQ(gather(codes), gather(norms), 3),
                           R.ValueQ(gather(vd), gather(vsc), gather(vz), 2), L)
        ref_o = R.hybrid_attention(q[b:b + 1].cpu(), _FlatStore(flat, codec, D, Hkv), None, None, Hq)
        assert_attn_close(out[b:b + 1], ref_o, f"c5 full size, sequence {b} ({L} tokens)")


def test_c4_full_size_prefill(dev):
    Hq, Hkv, D = 28, 4, 128
    N, Rn, T = 65536 - 128, 128, 2048
    g = torch.Generator().manual_seed(3)
    outl = torch.randperm(D, generator=g)[:4]
    calib_k = sample_keys(4096, seed=31)
    calib_k[:, outl] *= 20
    calib_q = sample_keys(4096, seed=32)
    strat = S.SMAQBlockVQStrategy(D, block_dim=2, n_centroids=256, device=dev)
    strat.quantizer.fit(calib_k.to(dev), calib_q.to(dev), kmeans_iters=3, on_device=True)
    keys = dev_sample_keys(N * Hkv, seed=33, device=dev, dtype=torch.float16).view(N, Hkv, D)
    keys[..., outl.to(dev)] *= 20
    vals = dev_sample_values(N * Hkv, seed=34, device=dev, dtype=torch.float16).view(N, Hkv, D)
    st = S.CompressedKVStore(D, Hkv, device=dev, key_strategy=strat)
    st.append_chunk(keys, vals)
    kr = dev_sample_keys(Rn * Hkv, seed=35, device=dev, dtype=torch.float16).view(Rn, Hkv, D)
    kr[..., outl.to(dev)] *= 20
    vr = dev_sample_values(Rn * Hkv, seed=36, device=dev, dtype=torch.float16).view(Rn, Hkv, D)
    q = dev_sample_keys(T * Hq, seed=37, device=dev, dtype=torch.float16).view(T, Hq, D)
    pos = torch.arange(N + Rn - T, N + Rn, device=dev)
    out = S.compute_hybrid_attention(q, st, kr, vr, Hq, query_positions=pos).cpu()
    qz = strat.quantizer
    codec = R.BlockVQCodec(qz.E_blocks.cpu(), qz.centroids.cpu(), qz.decoded_centroids.cpu())
    gf = st.get_flat_cache()
    flat = R.FlatCache(R.BlockQ(gf.key_q.indices.cpu(), gf.key_q.n_blocks, gf.key_q.block_dim),
                       R.ValueQ(gf.value_q.data.cpu(), gf.value_q.scales.cpu(), gf.value_q.zeros.cpu(),
                                gf.value_q.bits), gf.num_tokens)
    ost = _FlatStore(flat, codec, D, Hkv)
    # eight query tokens from each 256-token query block (the kernel's
    # workgroup rows), first and last of every block included; each token's
    # output merges every key split of the history
    sel = torch.tensor([blk * 256 + o for blk in range(T // 256) for o in (0, 37, 74, 111, 148, 185, 222, 255)])
    ref_o = R.hybrid_attention(q[sel.to(dev)].cpu(), ost, kr.cpu(), vr.cpu(), Hq, query_positions=pos[sel.to(dev)].cpu())
    assert_attn_close(out[sel], ref_o, f"c4 full size, {sel.numel()} queries over {T // 256} query blocks")
