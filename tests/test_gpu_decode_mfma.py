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


def test_mfma_decode_many_splits(dev):
    """One sequence, 2 KV heads, 20000 tokens: the context is cut into 40
    splits of 384-512 tokens (whole 128-token steps), so the split merge runs
    five chunks of loads and rescales its sums whenever a later chunk holds a
    larger maximum."""
    strat, codec = _codec_pair(dev, 3, 280)
    hkv, g, n = 2, 4, 20000
    keys = sample_keys(n * hkv, seed=281).reshape(n, hkv, 128).bfloat16()
    vals = torch.randn(n, hkv, 128, generator=torch.Generator().manual_seed(282)).bfloat16()
    # a late token the queries align with, so the maximum moves in a late chunk
    keys[18000] = keys[18000] * 4
    kvb = QuantizedKVBatch.encode(strat, [keys.to(dev)], [vals.to(dev)])
    q = keys[18000].float().repeat_interleave(g, dim=0).unsqueeze(0).bfloat16()
    out = kvb.attention(q.to(dev), impl=2)
    assert_attn_close(out, _oracle(codec, keys, vals, q, hkv * g, hkv), "mfma 40 splits")


def test_mfma_decode_slot_weighted_splits(dev):
    """8 ragged sequences x 8 KV heads = 64 units: a one-round grid of 16
    splits per unit spans four round-slots per CU, so the splits of later
    slots are shorter (weights 64 - 10 * slot) and every boundary falls on a
    whole 128-token step of each sequence's own length."""
    strat, codec = _codec_pair(dev, 3, 300)
    hkv, g = 8, 4
    lens = [3001, 8192, 4500, 129, 7777, 5000, 2048, 6100]
    gen = torch.Generator().manual_seed(301)
    keys = [sample_keys(n * hkv, seed=310 + i).reshape(n, hkv, 128).bfloat16() for i, n in enumerate(lens)]
    vals = [torch.randn(n, hkv, 128, generator=gen).bfloat16() for n in lens]
    kvb = QuantizedKVBatch.encode(strat, [k.to(dev) for k in keys], [v.to(dev) for v in vals])
    q = torch.randn(len(lens), hkv * g, 128, generator=gen).bfloat16()
    out = kvb.attention(q.to(dev), impl=2)
    for b in (0, 1, 3, 4, 7):
        ref = _oracle(codec, keys[b], vals[b], q[b:b + 1], hkv * g, hkv)
        assert_attn_close(out[b:b + 1], ref, f"slot-weighted splits seq {b} len {lens[b]}")


@pytest.mark.parametrize("qdtype", [torch.float32, torch.float16, torch.bfloat16])
def test_mfma_decode_direct_output(dev, qdtype):
    """Contexts of at most 512 tokens give one split per (sequence, head) and
    no recent part, so the decode kernel writes the output itself (no split
    combine); a history phase followed by a separate combine phase gives the
    same bits (the rotation, phase 8, first)."""
    strat, codec = _codec_pair(dev, 3, 320)
    hkv, g = 8, 4
    lens = [300, 512, 17, 200, 64]
    gen = torch.Generator().manual_seed(321)
    keys = [sample_keys(n * hkv, seed=330 + i).reshape(n, hkv, 128).bfloat16() for i, n in enumerate(lens)]
    vals = [torch.randn(n, hkv, 128, generator=gen).bfloat16() for n in lens]
    kvb = QuantizedKVBatch.encode(strat, [k.to(dev) for k in keys], [v.to(dev) for v in vals])
    q = torch.randn(len(lens), hkv * g, 128, generator=gen).to(qdtype)
    out = kvb.attention(q.to(dev), impl=2)
    assert out.dtype == qdtype
    for b in range(len(lens)):
        ref = _oracle(codec, keys[b], vals[b], q[b:b + 1], hkv * g, hkv)
        assert_attn_close(out[b:b + 1], ref, f"direct output {qdtype} seq {b} len {lens[b]}")
    plan = kvb.plan(q.to(dev))
    full = plan.run(q.to(dev)).clone()
    plan.out.zero_()
    plan.load_query(q.to(dev))
    plan.launch(phases=8)      # query rotation
    plan.launch(phases=1)
    plan.launch(phases=4)
    torch.cuda.synchronize()
    assert torch.equal(plan.out, full)


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


def test_mfma_decode_paged_longest_first(dev):
    """256 ragged sequences x 8 KV heads = 2048 (sequence, head) units: one
    workgroup each, dispatched longest sequence first through an order the
    library writes into the plan's workspace (its size shows the path is
    taken).  Every sequence matches the generic kernels (batch order) and a
    sample, including the longest and the shortest, matches the oracle."""
    strat, codec = _codec_pair(dev, 3, 300)
    gen = torch.Generator().manual_seed(301)
    B, bs, hkv = 256, 16, 8
    lens = [int(x) for x in torch.randint(1, 160, (B,), generator=gen)]
    lens[7], lens[200] = 900, 1
    nblk = [(n + bs - 1) // bs for n in lens]
    nphys = sum(nblk) + 5
    perm = torch.randperm(nphys, generator=gen)
    table = torch.zeros(B, max(nblk), dtype=torch.int32)
    o = 0
    for b, nb in enumerate(nblk):
        table[b, :nb] = perm[o:o + nb].to(torch.int32)
        o += nb
    allk = sample_keys(sum(lens) * hkv, seed=302).reshape(sum(lens), hkv, 128).bfloat16()
    allv = torch.randn(sum(lens), hkv, 128, generator=gen).bfloat16()
    cut = [0]
    for n in lens:
        cut.append(cut[-1] + n)
    keys = [allk[cut[b]:cut[b + 1]] for b in range(B)]
    vals = [allv[cut[b]:cut[b + 1]] for b in range(B)]
    pk = PagedQuantizedKV.encode(strat, [k.to(dev) for k in keys], [v.to(dev) for v in vals], table.to(dev),
                                 num_blocks=nphys, block_size=bs)
    q = torch.randn(B, 32, 128, generator=gen).bfloat16()
    plan = pk.plan(q.to(dev), impl=2)
    partials = B * hkv * 4 * (128 + 2) * 4          # one split: (m, l, o) per query row
    assert plan.workspace.numel() == partials + B * 4, "longest-first order not planned"
    out = plan.run(q.to(dev)).squeeze(1).clone()
    again = plan.run(q.to(dev)).squeeze(1)
    assert torch.equal(out, again)
    out_g = pk.attention(q.to(dev), impl=1)
    assert_attn_close(out, out_g.cpu(), "longest first vs generic (all sequences)")
    # the oracle's store API ignores histories under MIN_HISTORY_FOR_SMAQ
    # tokens (smaq/score.py:38); the batched path attends every history, so
    # the sample is drawn from sequences of 16+ tokens ...
    for b in [7] + [b for b in range(B) if lens[b] >= 16][:4]:
        assert_attn_close(out[b:b + 1], _oracle(codec, keys[b], vals[b], q[b:b + 1], 32, hkv),
                          f"longest first seq {b} len {lens[b]}")
    # ... and the 1-token history attends its one token: the output is that
    # token's dequantised value for each query head of the group
    vq = R.quantize_values(vals[200].permute(1, 0, 2).unsqueeze(0), bits=2, group_size=32)
    v_hat = R.dequantize_values(vq, 32)[0, :, 0, :].repeat_interleave(32 // hkv, dim=0)
    assert_attn_close(out[200:201], v_hat.unsqueeze(0).bfloat16(), "longest first seq 200 len 1")


def _paged_table(lens, bs, gen, spare=7):
    nblk = [(n + bs - 1) // bs for n in lens]
    nphys = sum(nblk) + spare
    perm = torch.randperm(nphys, generator=gen)
    table = torch.zeros(len(lens), max(nblk), dtype=torch.int32)
    o = 0
    for b, nb in enumerate(nblk):
        table[b, :nb] = perm[o:o + nb].to(torch.int32)
        o += nb
    return table, nphys


def _first_round(dev, hkv, slots=4):
    """Sequences whose KV heads fill one round of decode workgroup slots (4
    per CU with 16-bit metadata, 3 with fp32)."""
    return torch.cuda.get_device_properties(dev).multi_processor_count * slots // hkv


def _item_rows(plan, B, hkv, slots=4):
    """The work items the library wrote into the plan's workspace (after the
    partials): [n_items, 4] int32 rows (sequence, first token, end token,
    count << 16 | piece)."""
    fr = _first_round(plan.device, hkv, slots)
    n_items = fr + (B - fr) * _max_pieces(plan)
    off = plan.workspace.numel() - n_items * 16
    return plan.workspace[off:].view(torch.int32).view(n_items, 4).cpu(), n_items


PIECE_TOKENS = 4096  # the library's kDecodePiece (attention.hip)


def _max_pieces(plan):
    """Pieces the plan allows per sequence: pieces of the history length over
    8, at least PIECE_TOKENS, rounded up to 128-token steps."""
    L = plan.params.max_hist_len
    piece = max(PIECE_TOKENS, -(-L // 8))
    piece = -(-piece // 128) * 128
    return -(-L // piece)


@pytest.mark.parametrize("bs,dtype", [(16, torch.bfloat16), (32, torch.bfloat16), (16, torch.float32)])
def test_mfma_decode_paged_pieces(dev, bs, dtype):
    """More ragged sequences than one round of workgroup slots holds (48 more
    than fill the 1,024 slots of 4 per CU with 16-bit metadata, or the 768 of
    3 per CU with fp32 metadata; 8 KV heads) and histories above 4,096
    tokens: the sequences that start after the first round run in pieces of
    about 4,096 tokens, merged by the decode kernel's arrival counters.  The
    library's item list covers every sequence's history exactly once, within
    the planned number of items and pieces; the output is the same bits on a
    second call (counters reset) and through separate launches, matches the
    generic kernels for every sequence, and the oracle for the longest
    sequence and pieced ones.  16- and 32-token pages (the kernel's two
    paged variants)."""
    strat, codec = _codec_pair(dev, 3, 380)
    gen = torch.Generator().manual_seed(381)
    hkv = 8
    slots = 3 if dtype == torch.float32 else 4
    fr = _first_round(dev, hkv, slots)
    B = fr + 48
    lens = [int(x) for x in torch.randint(4200, 4701, (B,), generator=gen)]
    lens[5] = 9000
    table, nphys = _paged_table(lens, bs, gen)
    allk = sample_keys(sum(lens) * hkv, seed=382).reshape(sum(lens), hkv, 128).to(dtype)
    allv = torch.randn(sum(lens), hkv, 128, generator=gen).to(dtype)
    cut = [0]
    for n in lens:
        cut.append(cut[-1] + n)
    keys = [allk[cut[b]:cut[b + 1]] for b in range(B)]
    vals = [allv[cut[b]:cut[b + 1]] for b in range(B)]
    pk = PagedQuantizedKV.encode(strat, [k.to(dev) for k in keys], [v.to(dev) for v in vals], table.to(dev),
                                 num_blocks=nphys, block_size=bs)
    del allk, allv
    q = torch.randn(B, 32, 128, generator=gen).to(dtype)
    plan = pk.plan(q.to(dev), impl=2)
    maxp = _max_pieces(plan)
    assert maxp == 3
    partials = B * hkv * 4 * maxp * (128 + 2) * 4
    n_items = fr + (B - fr) * maxp
    assert plan.workspace.numel() == ((partials + 255) // 256) * 256 + n_items * 16, "pieces not planned"
    out = plan.run(q.to(dev)).squeeze(1).clone()
    again = plan.run(q.to(dev)).squeeze(1)
    torch.cuda.synchronize()
    assert torch.equal(out, again), "second call differs"
    assert int(plan.arrivals.abs().sum()) == 0, "arrival counters not reset"
    # the full call builds the schedule inside the rotation's launch; the
    # rotation alone, then the history phase (schedule launch + decode), and
    # the decode kernel alone on that schedule (phase 16) give the same bits
    plan.load_query(q.to(dev))
    plan.out.zero_()
    plan.launch(phases=8)
    plan.launch(phases=1)
    torch.cuda.synchronize()
    assert torch.equal(plan.out.squeeze(1), out), "separate rotation and schedule launches differ"
    plan.out.zero_()
    plan.launch(phases=1 | 16)
    torch.cuda.synchronize()
    assert torch.equal(plan.out.squeeze(1), out), "decode on the kept schedule differs"
    items, _ = _item_rows(plan, B, hkv, slots)
    real = items[items[:, 0] >= 0]
    assert bool((items[len(real):, 0] < 0).all()), "empty items must follow the real ones"
    pieced = set()
    for b in range(B):
        rows = real[real[:, 0] == b]
        count = int(rows[0, 3]) >> 16
        assert 1 <= count <= maxp and len(rows) == count, f"seq {b}: {len(rows)} items, count {count}"
        rows = rows[torch.argsort(rows[:, 3] & 0xFFFF)]
        assert int(rows[0, 1]) == 0 and int(rows[-1, 2]) == lens[b], f"seq {b} range"
        assert bool((rows[1:, 1] == rows[:-1, 2]).all()), f"seq {b} pieces not contiguous"
        assert bool((rows[:-1, 2] % 128 == 0).all()), f"seq {b} boundaries off the 128-token step"
        if count > 1:
            pieced.add(b)
    assert len(pieced) >= 40, f"only {len(pieced)} sequences pieced"
    order = sorted(range(B), key=lambda b: -lens[b])
    assert not (pieced & set(order[:fr])), "a first-round sequence was pieced"
    out_g = pk.attention(q.to(dev), impl=1)
    assert_attn_close(out, out_g.cpu(), "pieces vs generic (all sequences)")
    for b in [5] + sorted(pieced)[:3]:
        assert_attn_close(out[b:b + 1], _oracle(codec, keys[b], vals[b], q[b:b + 1], 32, hkv),
                          f"pieces seq {b} len {lens[b]}")


@pytest.mark.parametrize("max_len,pieced", [(16384, True), (32768, False)])
def test_decode_pieces_plan_respects_the_grid_limit(dev, max_len, pieced):
    """The work items are the decode grid's y dimension (at most 65535): a
    paged batch of 10,000 ragged sequences takes pieces while first round +
    later sequences x most pieces fits (histories up to 16,384 tokens: 4
    pieces), and the one-split longest-first order beyond (32,768: 8 pieces
    would need 79,104 items).  Only the workspace size is asked for (the
    parameter block's pointers are placeholders the size computation does
    not read)."""
    from smaq_amd import _native
    _native.lib()  # the library on this device
    B, hkv, hq = 10000, 8, 32
    p = _native.AttnParams()
    p.batch, p.q_len, p.n_q_heads, p.n_kv_heads, p.head_dim, p.scale = B, 1, hq, hkv, 128, 128 ** -0.5
    fake = 1 << 20  # 16-byte aligned placeholders
    p.q_hist = p.q_exact = p.out = p.workspace = p.key_lut = fake
    p.has_history, p.key_format, p.key_bits, p.key_row_bytes = 1, _native.KEY_SCALAR, 3, 64
    p.key_bytes = p.key_norms = p.val_bytes = p.val_scales = p.val_zeros = fake
    p.norm_dtype = p.val_dtype = p.out_dtype = _native.dtype_code(torch.bfloat16)
    p.val_bits, p.val_group, p.val_row_bytes = 2, 32, 32
    p.hist_len = p.block_table = p.arrivals = fake
    p.block_size, p.max_blocks, p.max_hist_len = 16, max_len // 16, max_len
    fr = _first_round(dev, hkv)
    S = max_len // 4096 if pieced else 1
    partials = B * hkv * 4 * S * (128 + 2) * 4
    sched = (fr + (B - fr) * S) * 16 if pieced else B * 4
    assert (fr + (B - fr) * (max_len // 4096) <= 65535) == pieced
    assert _native.attn_workspace_bytes(p) == ((partials + 255) // 256) * 256 + sched


@pytest.mark.parametrize("odtype", [torch.bfloat16, torch.float32])
def test_mfma_decode_pieces_with_recent(dev, odtype):
    """Longest-first pieces on a contiguous ragged batch with an exact recent
    window (per-sequence lengths, some empty): the recent phase runs first,
    the decode kernel's last workgroup per (sequence, KV head) merges its
    pieces and the recent partials.  Same bits on a second call; the generic
    kernels for every sequence and the oracle on a sample."""
    strat, codec = _codec_pair(dev, 3, 390)
    gen = torch.Generator().manual_seed(391)
    B, hkv, g, RW = 160, 8, 4, 24
    lens = [int(x) for x in torch.randint(4200, 5001, (B,), generator=gen)]
    rl = [int(x) for x in torch.randint(0, RW + 1, (B,), generator=gen)]
    allk = sample_keys(sum(lens) * hkv, seed=392).reshape(sum(lens), hkv, 128).bfloat16()
    allv = torch.randn(sum(lens), hkv, 128, generator=gen).bfloat16()
    cut = [0]
    for n in lens:
        cut.append(cut[-1] + n)
    keys = [allk[cut[b]:cut[b + 1]] for b in range(B)]
    vals = [allv[cut[b]:cut[b + 1]] for b in range(B)]
    kvb = QuantizedKVBatch.encode(strat, [k.to(dev) for k in keys], [v.to(dev) for v in vals])
    del allk, allv
    rk = torch.randn(B, RW, hkv, 128, generator=gen).bfloat16()
    rv = torch.randn(B, RW, hkv, 128, generator=gen).bfloat16()
    q = torch.randn(B, hkv * g, 128, generator=gen).to(odtype)
    qd = q.to(dev)
    plan = kvb.plan(qd, recent_k=rk.to(dev), recent_v=rv.to(dev), recent_len=torch.tensor(rl), impl=2)
    maxp = _max_pieces(plan)
    assert maxp == 2
    out = plan.run(qd).squeeze(1).clone()
    again = plan.run(qd).squeeze(1).clone()
    torch.cuda.synchronize()
    assert torch.equal(out, again) and int(plan.arrivals.abs().sum()) == 0
    items, _ = _item_rows(plan, B, hkv)
    counts = items[items[:, 0] >= 0, 3] >> 16
    assert int(counts.max()) >= 2, "no sequence pieced"
    out_g = kvb.attention(qd, recent_k=rk.to(dev), recent_v=rv.to(dev), recent_len=torch.tensor(rl), impl=1)
    assert_attn_close(out, out_g.cpu(), f"pieces + recent vs generic {odtype}")
    short = sorted(range(B), key=lambda b: lens[b])
    for b in short[:2] + [short[-1]]:
        st = R.Store(codec, 128, hkv)
        st.append_chunk(keys[b], vals[b])
        n = rl[b]
        want = R.hybrid_attention(q[b:b + 1], st, rk[b, :n] if n else None, rv[b, :n] if n else None, hkv * g)
        assert_attn_close(out[b:b + 1], want, f"pieces + recent {odtype} seq {b}")


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


@pytest.mark.parametrize("qdtype", [torch.float32, torch.float16, torch.bfloat16])
def test_mfma_decode_split_merge(dev, qdtype):
    """Several splits per (sequence, KV head) and a rotated codec: the plan
    hands the raw query to the library (which rotates it into q_hist) and
    gives arrival counters, so the decode kernel's last workgroup per unit
    merges the splits.  The output is bit-identical to the separate launches
    (rotation by the caller, decode partials, combine kernel), the counters
    are zero again after every call (a second run gives the same bits), and
    sampled sequences match the oracle."""
    from smaq_amd import _native
    strat, codec = _codec_pair(dev, 3, 340)
    hkv, g = 8, 4
    lens = [6000, 4097, 5555]
    gen = torch.Generator().manual_seed(341)
    keys = [sample_keys(n * hkv, seed=342 + i).reshape(n, hkv, 128).bfloat16() for i, n in enumerate(lens)]
    vals = [torch.randn(n, hkv, 128, generator=gen).bfloat16() for n in lens]
    kvb = QuantizedKVBatch.encode(strat, [k.to(dev) for k in keys], [v.to(dev) for v in vals])
    q = torch.randn(len(lens), hkv * g, 128, generator=gen).to(qdtype)
    qd = q.to(dev)
    plan = kvb.plan(qd, impl=2)
    assert plan.rot_t is not None and plan.params.rot_mt, "codec without rotation"
    # the plan's workspace holds more than one split per unit: the merge path
    one_split = len(lens) * hkv * g * (128 + 2) * 4
    assert plan.workspace.numel() > one_split
    out1 = plan.run(qd).clone()
    out2 = plan.run(qd).clone()
    torch.cuda.synchronize()
    assert torch.equal(out1, out2), "second call differs (arrival counters not reset?)"
    assert int(plan.arrivals.abs().sum()) == 0
    # separate launches: rotation by the caller, partials, combine
    plan.params.arrivals = None
    plan.params.rot_mt = None
    plan.params.rot_scale = None
    plan.q_hist.zero_()
    _native.rotate_rows_into(qd.reshape(plan.shape).contiguous(), plan.rot_t, plan.rot_scale, plan.q_hist)
    plan.out.zero_()
    ref = plan.launch().clone()
    torch.cuda.synchronize()
    assert torch.equal(out1, ref), f"split merge differs: {(out1.float() - ref.float()).abs().max()}"
    for b in (0, 2):
        assert_attn_close(out1[b:b + 1], _oracle(codec, keys[b], vals[b], q[b:b + 1], hkv * g, hkv),
                          f"split merge {qdtype} seq {b}")


@pytest.mark.parametrize("odtype", [torch.float32, torch.bfloat16])
def test_mfma_decode_merge_with_recent(dev, odtype):
    """History in several splits plus an exact recent window (ragged lengths,
    one sequence with an empty window): the recent phase runs first and the
    decode kernel's last workgroup per unit merges history and recent
    partials, rounding each to the output dtype before adding them.  Bit for
    bit the separate launches (history, recent, combine phases), and the
    oracle on sampled sequences."""
    strat, codec = _codec_pair(dev, 3, 350)
    hkv, g, RW = 8, 4, 40
    lens = [3000, 5000, 700]
    rl = [40, 0, 17]
    gen = torch.Generator().manual_seed(351)
    keys = [sample_keys(n * hkv, seed=352 + i).reshape(n, hkv, 128).bfloat16() for i, n in enumerate(lens)]
    vals = [torch.randn(n, hkv, 128, generator=gen).bfloat16() for n in lens]
    rk = torch.randn(len(lens), RW, hkv, 128, generator=gen).bfloat16()
    rv = torch.randn(len(lens), RW, hkv, 128, generator=gen).bfloat16()
    kvb = QuantizedKVBatch.encode(strat, [k.to(dev) for k in keys], [v.to(dev) for v in vals])
    q = torch.randn(len(lens), hkv * g, 128, generator=gen).to(odtype)
    qd = q.to(dev)
    plan = kvb.plan(qd, recent_k=rk.to(dev), recent_v=rv.to(dev), recent_len=torch.tensor(rl), impl=2)
    out = plan.run(qd).clone()
    again = plan.run(qd).clone()
    torch.cuda.synchronize()
    assert torch.equal(out, again) and int(plan.arrivals.abs().sum()) == 0
    plan.out.zero_()
    plan.load_query(qd)
    for ph in (8, 1, 2, 4):
        plan.launch(phases=ph)
    torch.cuda.synchronize()
    assert torch.equal(plan.out, out), f"merge with recent differs: {(plan.out.float() - out.float()).abs().max()}"
    for b in range(len(lens)):
        st = R.Store(codec, 128, hkv)
        st.append_chunk(keys[b], vals[b])
        n = rl[b]
        want = R.hybrid_attention(q[b:b + 1], st, rk[b, :n] if n else None, rv[b, :n] if n else None, hkv * g)
        assert_attn_close(out[b:b + 1].squeeze(1), want, f"merge with recent {odtype} seq {b}")


@pytest.mark.parametrize("g,rdtype", [(1, torch.float32), (2, torch.float16), (4, torch.bfloat16)])
def test_recent_decode_kernel(dev, g, rdtype):
    """The decode-shape recent-window kernel (one query token, head_dim 128,
    1/2/4 query heads per KV head) over ragged windows of up to two 64-token
    chunks (100, 1, 64, 65 and 0 tokens): every sequence matches the oracle,
    and the generic kernels (impl 1) within the same tolerance."""
    strat, codec = _codec_pair(dev, 3, 360 + g)
    hkv, RW = 4, 100
    lens = [500, 300, 64, 1000, 129]
    rl = [100, 1, 64, 65, 0]
    gen = torch.Generator().manual_seed(361 + g)
    keys = [sample_keys(n * hkv, seed=362 + i).reshape(n, hkv, 128).bfloat16() for i, n in enumerate(lens)]
    vals = [torch.randn(n, hkv, 128, generator=gen).bfloat16() for n in lens]
    rk = (torch.randn(len(lens), RW, hkv, 128, generator=gen) * 0.5).to(rdtype)
    rv = torch.randn(len(lens), RW, hkv, 128, generator=gen).to(rdtype)
    kvb = QuantizedKVBatch.encode(strat, [k.to(dev) for k in keys], [v.to(dev) for v in vals])
    q = torch.randn(len(lens), hkv * g, 128, generator=gen).bfloat16()
    args = dict(recent_k=rk.to(dev), recent_v=rv.to(dev), recent_len=torch.tensor(rl))
    out = kvb.attention(q.to(dev), **args)
    gen_out = kvb.attention(q.to(dev), impl=1, **args)
    for b in range(len(lens)):
        st = R.Store(codec, 128, hkv)
        st.append_chunk(keys[b], vals[b])
        n = rl[b]
        want = R.hybrid_attention(q[b:b + 1], st, rk[b, :n] if n else None, rv[b, :n] if n else None, hkv * g)
        assert_attn_close(out[b:b + 1], want, f"recent kernel g={g} {rdtype} seq {b}")
        assert_attn_close(gen_out[b:b + 1], want, f"generic recent g={g} {rdtype} seq {b}")


@pytest.mark.parametrize("lens", [[3000, 2000], [400, 300]])
def test_nan_key_norm_gives_nan_rows(dev, lens):
    """A NaN key norm makes that token's scores NaN, and the reference's
    softmax (smaq/score.py:61-72) returns NaN for every query row that
    scores it.  The fused paths do the same -- matrix-core decode with the
    in-kernel split merge, with the combine launch, with one split writing
    the output directly ([400, 300]), the generic kernels and the
    matrix-core prefill -- while every other row keeps its bits (finite, for
    the prefill)."""
    strat, _ = _codec_pair(dev, 3, 370)
    hkv, g = 2, 4
    gen = torch.Generator().manual_seed(371)
    keys = [sample_keys(n * hkv, seed=372 + i).reshape(n, hkv, 128).bfloat16().to(dev) for i, n in enumerate(lens)]
    vals = [torch.randn(n, hkv, 128, generator=gen).bfloat16().to(dev) for n in lens]
    kvb = QuantizedKVBatch.encode(strat, keys, vals)
    q = torch.randn(len(lens), hkv * g, 128, generator=gen).bfloat16().to(dev)
    clean = {impl: kvb.attention(q, impl=impl).clone() for impl in (1, 2)}
    kvb.norms[1, 123] = float("nan")                 # sequence 0, KV head 1, token 123
    bad = torch.zeros(len(lens), hkv * g, dtype=torch.bool)
    bad[0, g:2 * g] = True
    for impl in (1, 2):
        for merge in ((True, False) if impl == 2 else (True,)):
            plan = kvb.plan(q, impl=impl)
            if not merge:
                plan.params.arrivals = None
            out = plan.run(q).squeeze(1).cpu()
            what = f"impl {impl} merge {merge}"
            assert bool(torch.isnan(out[bad]).all()), what
            assert bool(torch.equal(out[~bad], clean[impl].cpu()[~bad])), what
    # the matrix-core prefill (16 query tokens per sequence) and its combine
    q16 = torch.randn(len(lens), 16, hkv * g, 128, generator=gen).bfloat16().to(dev)
    out = kvb.attention(q16, impl=3).cpu()
    assert bool(torch.isnan(out[0, :, g:2 * g]).all()), "prefill"
    assert not bool(torch.isnan(out[0, :, :g]).any()) and not bool(torch.isnan(out[1:]).any()), "prefill"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_mfma_decode_paged_value_descriptor_bits(dev, dtype):
    """16-token pages: the plan records the pools' row count (hist_rows), and
    the decode kernel then reads the value pool through one range-checked
    descriptor with 32-bit lane offsets.  Same bits as the 64-bit per-lane
    addresses it takes with hist_rows = 0 (ragged lengths, one sequence of
    5,000 tokens), and the oracle's result for a sample."""
    strat, codec = _codec_pair(dev, 3, 420)
    gen = torch.Generator().manual_seed(421)
    hkv, bs = 8, 16
    B = 40
    lens = [int(x) for x in torch.randint(1, 900, (B,), generator=gen)]
    lens[3] = 5000
    table, nphys = _paged_table(lens, bs, gen)
    keys = [sample_keys(n * hkv, seed=430 + b).reshape(n, hkv, 128).to(dtype) for b, n in enumerate(lens)]
    vals = [torch.randn(n, hkv, 128, generator=gen).to(dtype) for n in lens]
    pk = PagedQuantizedKV.encode(strat, [k.to(dev) for k in keys], [v.to(dev) for v in vals], table.to(dev),
                                 num_blocks=nphys, block_size=bs)
    q = torch.randn(B, 32, 128, generator=gen).to(dtype)
    plan = pk.plan(q.to(dev), impl=2)
    assert plan.params.hist_rows == nphys * hkv * bs
    desc = plan.run(q.to(dev)).clone()
    plan.params.hist_rows = 0
    addr = plan.run(q.to(dev)).clone()
    # a row count past the 4 GB limit: the per-lane addresses again
    plan.params.hist_rows = 1 << 28
    big = plan.run(q.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(desc, addr), "value descriptor and per-lane addresses differ"
    assert torch.equal(big, addr), "a pool above 4 GB must take the per-lane addresses"
    for b in (0, 3, B - 1):
        assert_attn_close(desc[b:b + 1].squeeze(1), _oracle(codec, keys[b], vals[b], q[b:b + 1], 32, hkv),
                          f"paged value descriptor {dtype} seq {b}")
