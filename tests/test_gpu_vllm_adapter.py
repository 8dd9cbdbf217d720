"""vLLM adapter serving paths on the GPU against the CPU oracle, through fake
vLLM objects (vLLM is not installed).

* Reference layout (smaq/integration/vllm.py:113-272): K/V writes feed the
  capture engine (prefill: all but the last ring-capacity tokens compressed;
  decode: ring, whose overflow flushes to the store); a hybrid decode step is
  compute_hybrid_attention over the store plus the ring.  The oracle replays
  the same writes through its Store and Ring.
* Paged pools (the adapter's extension): each write is encoded into the rows
  its slots name; a decode step of the whole batch runs over vLLM's block
  table and sequence lengths.  The oracle encodes each sequence's tokens into
  its own Store and attends per sequence.

Tolerance: 2e-3 absolute + 1e-3 relative (+1 ulp of the bf16 output), as the
other attention parity tests."""

from __future__ import annotations

import pytest
import torch

import smaq_amd.integration as I
import smaq_amd.integration.vllm as V
from oracle import smaq_ref as R
from tests.conftest import sample_keys
from tests.test_gpu_attention import assert_attn_close
from tests.vllm_fakes import FakeFlashImpl, make_runner, meta

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _restore_mode():
    yield
    V.set_mode(V.MODE_CAPTURE_ONLY)


def _oracle_codec(state):
    qz = state.store.key_strategy.quantizer
    return R.ScalarCodec(state.config.head_dim, state.config.key_bits, E=qz.E.float().cpu(),
                         E_inv=qz.E_inv.float().cpu())


def test_reference_layout_hybrid_decode(dev):
    hq, hkv, D = 8, 2, 128
    impl = FakeFlashImpl(hq, hkv, D)
    kv = torch.zeros(2, 32, 16, hkv, D, dtype=torch.bfloat16, device=dev)
    runner = make_runner({"l0": impl}, dev, {"l0": kv})
    calib = {"l0": R.fit_sigma_centered(sample_keys(64, seed=71))}
    st = I.install_hooks(runner, calibration_covariances=calib, key_bits=3, initial_layers_count=0,
                         mode=V.MODE_CAPTURE_ONLY)["l0"]
    T = 300
    k = sample_keys(T * hkv, seed=72).reshape(T, hkv, D).bfloat16()
    v = torch.randn(T, hkv, D, generator=torch.Generator().manual_seed(73)).bfloat16()
    impl.do_kv_cache_update(None, k.to(dev), v.to(dev), kv, torch.arange(T, device=dev))
    assert st.store.num_tokens == T - 128 and st.engine.ring.size == 128
    k1 = sample_keys(hkv, seed=74).reshape(1, hkv, D).bfloat16()
    v1 = torch.randn(1, hkv, D, generator=torch.Generator().manual_seed(75)).bfloat16()
    impl.do_kv_cache_update(None, k1.to(dev), v1.to(dev), kv, torch.tensor([T], device=dev))
    assert st.store.num_tokens == T and st.engine.ring.size == 1

    # oracle replay of the same writes
    ref = R.Store(_oracle_codec(st), D, hkv)
    ring = R.Ring(128, hkv, D)
    ref.append_chunk(k[: T - 128], v[: T - 128])
    ring.write(k[T - 128:], v[T - 128:], 128)
    spill = ring.write(k1, v1, 1)
    ref.append_chunk(*spill)
    assert torch.equal(st.store.get_flat_cache().key_q.indices.cpu(), ref.get_flat_cache().key_q.indices)

    V.set_mode(V.MODE_HYBRID)
    q = torch.randn(1, hq, D, generator=torch.Generator().manual_seed(76)).bfloat16()
    out = torch.zeros(2, hq * D, dtype=torch.bfloat16, device=dev)
    m = meta(1, 1, seq_lens=torch.tensor([T + 1], device=dev), block_table=torch.zeros(1, 32, dtype=torch.int32))
    res = impl.forward(None, q.reshape(1, -1).to(dev), k1.to(dev), v1.to(dev), kv, m, output=out)
    assert res is out and impl.calls == ["update", "update"]
    rk, rv = ring.peek()
    want = R.hybrid_attention(q, ref, rk, rv, hq)
    assert_attn_close(out[:1].view(1, hq, D), want, "adapter reference layout")
    assert not out[1:].any()
    # a 3-D query without an output buffer comes back in the query's shape
    res3 = impl.forward(None, q.to(dev), k1.to(dev), v1.to(dev), kv, m)
    assert res3.shape == (1, hq, D)
    assert_attn_close(res3, want, "adapter reference layout, 3-D query")
    s = I.get_stats(runner)["l0"]
    assert s["compressed_tokens"] == T and s["buffered_tokens"] == 1 and s["memory_bytes"] > 0


def test_paged_pools_batch_decode(dev):
    hq, hkv, D, bs, nblk = 32, 8, 128, 16, 64
    impl = FakeFlashImpl(hq, hkv, D)
    kv = torch.zeros(2, nblk, bs, hkv, D, dtype=torch.bfloat16, device=dev)
    runner = make_runner({"l0": impl}, dev, {"l0": kv})
    calib = {"l0": R.fit_sigma_centered(sample_keys(64, seed=81))}
    st = I.install_hooks(runner, calibration_covariances=calib, key_bits=3, initial_layers_count=0,
                         mode=V.MODE_CAPTURE_ONLY, paged=True)["l0"]
    lens = [40, 97, 130, 16]
    B = len(lens)
    g = torch.Generator().manual_seed(82)
    perm = torch.randperm(nblk, generator=g)
    table = torch.zeros(B, 12, dtype=torch.int32)
    o = 0
    for b, L in enumerate(lens):
        n = (L + 2 + bs - 1) // bs                   # room for two decode steps
        table[b, :n] = perm[o:o + n].to(torch.int32)
        o += n
    keys = [sample_keys((L + 2) * hkv, seed=90 + b).reshape(L + 2, hkv, D).bfloat16() for b, L in enumerate(lens)]
    vals = [torch.randn(L + 2, hkv, D, generator=torch.Generator().manual_seed(95 + b)).bfloat16()
            for b, L in enumerate(lens)]

    def slot(b, t):
        return int(table[b, t // bs]) * bs + t % bs

    # one varlen prefill write for all sequences, then a decode write with a padded slot
    pk = torch.cat([keys[b][:L] for b, L in enumerate(lens)])
    pv = torch.cat([vals[b][:L] for b, L in enumerate(lens)])
    ps = torch.tensor([slot(b, t) for b, L in enumerate(lens) for t in range(L)])
    impl.do_kv_cache_update(None, pk.to(dev), pv.to(dev), kv, ps.to(dev))
    dk = torch.cat([keys[b][L:L + 1] for b, L in enumerate(lens)] + [torch.zeros(1, hkv, D, dtype=torch.bfloat16)])
    dv = torch.cat([vals[b][L:L + 1] for b, L in enumerate(lens)] + [torch.zeros(1, hkv, D, dtype=torch.bfloat16)])
    ds = torch.tensor([slot(b, L) for b, L in enumerate(lens)] + [-1])
    impl.do_kv_cache_update(None, dk.to(dev), dv.to(dev), kv, ds.to(dev))
    assert st.paged.tokens_written == sum(lens) + B and st.engine.ring.size == 0

    codec = _oracle_codec(st)

    def check(step):
        n_tok = [L + 1 + step for L in lens]
        q = torch.randn(B, hq, D, generator=torch.Generator().manual_seed(100 + step)).bfloat16()
        out = torch.zeros(B, hq * D, dtype=torch.bfloat16, device=dev)
        m = meta(B, 1, seq_lens=torch.tensor(n_tok, dtype=torch.int32, device=dev),
                 block_table=table.to(dev), max_seq_len=max(n_tok))
        res = impl.forward(None, q.reshape(B, -1).to(dev), None, None, kv, m, output=out)
        assert res is out
        for b in range(B):
            ref = R.Store(codec, D, hkv)
            ref.append_chunk(keys[b][:n_tok[b]], vals[b][:n_tok[b]])
            want = R.hybrid_attention(q[b:b + 1], ref, None, None, hq)
            assert_attn_close(out[b:b + 1].view(1, hq, D), want, f"paged adapter seq {b} step {step}")
            # the pools hold the oracle's codes at the rows of the sequence's slots
            rows = torch.tensor([(int(table[b, t // bs]) * hkv + h) * bs + t % bs
                                 for t in range(n_tok[b]) for h in range(hkv)])
            got = st.paged.pools["k_codes"].cpu()[rows].view(n_tok[b], hkv, -1).transpose(0, 1)
            assert torch.equal(got, ref.get_flat_cache().key_q.indices)

    V.set_mode(V.MODE_HYBRID)
    check(0)
    assert impl.calls == ["update", "update"]        # the layer's own forward never ran
    # after vLLM's cache is freed the pools keep serving
    assert I.free_kv_cache(runner) > 0
    kv_small = runner.compilation_config.static_forward_context["l0"].kv_cache[0]
    nk = torch.cat([keys[b][L + 1:L + 2] for b, L in enumerate(lens)])
    nv = torch.cat([vals[b][L + 1:L + 2] for b, L in enumerate(lens)])
    impl.do_kv_cache_update(None, nk.to(dev), nv.to(dev), kv_small,
                            torch.tensor([slot(b, L + 1) for b, L in enumerate(lens)], device=dev))
    check(1)
    s = I.get_stats(runner)["l0"]
    assert s["compressed_tokens"] == sum(lens) + 2 * B and s["memory_bytes"] == st.paged.memory_bytes()


def test_reference_layout_plan_reuse(dev):
    """Decode steps of the reference layout re-use the layer's plan while the
    history is unchanged (only the ring's fill moves) and rebuild it when a
    spill grows the history; every step equals a one-shot
    compute_hybrid_attention over the same store and ring bit for bit, and
    is written straight into the output buffer."""
    from smaq_amd.score import compute_hybrid_attention
    hq, hkv, D, C = 8, 2, 128, 16
    impl = FakeFlashImpl(hq, hkv, D)
    kv = torch.zeros(2, 32, 16, hkv, D, dtype=torch.bfloat16, device=dev)
    runner = make_runner({"l0": impl}, dev, {"l0": kv})
    calib = {"l0": R.fit_sigma_centered(sample_keys(64, seed=171))}
    st = I.install_hooks(runner, calibration_covariances=calib, key_bits=3, initial_layers_count=0,
                         mode=V.MODE_CAPTURE_ONLY, ring_capacity=C)["l0"]
    T = 200
    k = sample_keys((T + 40) * hkv, seed=172).reshape(T + 40, hkv, D).bfloat16().to(dev)
    v = torch.randn(T + 40, hkv, D, generator=torch.Generator().manual_seed(173)).bfloat16().to(dev)
    impl.do_kv_cache_update(None, k[:T], v[:T], kv, torch.arange(T, device=dev))
    V.set_mode(V.MODE_HYBRID)
    plans, hist = [], []
    for step in range(20):
        t = T + step
        impl.do_kv_cache_update(None, k[t:t + 1], v[t:t + 1], kv, torch.tensor([t], device=dev))
        q = torch.randn(1, hq * D, generator=torch.Generator().manual_seed(180 + step)).bfloat16().to(dev)
        out = torch.zeros(1, hq * D, dtype=torch.bfloat16, device=dev)
        m = meta(1, 1, seq_lens=torch.tensor([t + 1], device=dev), block_table=torch.zeros(1, 32, dtype=torch.int32))
        assert impl.forward(None, q, k[t:t + 1], v[t:t + 1], kv, m, output=out) is out
        rk, rv = st.engine.ring.peek()
        want = compute_hybrid_attention(q.view(1, hq, D), st.store, rk, rv, hq, scale=impl.scale)
        assert torch.equal(out.view(1, hq, D), want), f"step {step}"
        plans.append(st.ref_plan)
        hist.append(st.store.num_tokens)
    # one plan per history length (the ring spills every C tokens)
    for a in range(1, len(plans)):
        assert (plans[a] is plans[a - 1]) == (hist[a] == hist[a - 1]), a
    assert len(set(hist)) >= 2 and len({id(p) for p in plans}) == len(set(hist))
    assert impl.calls.count("forward") == 0


def test_paged_plan_reuse(dev):
    """Paged decode steps re-use one plan per batch shape and length bucket
    (next power of two of the longest sequence): lengths move within the
    bucket without a rebuild, a new bucket builds a second plan, and every
    step matches a plan built for that step's exact lengths."""
    from smaq_amd.batch import PagedQuantizedKV
    hq, hkv, D, bs = 32, 8, 128, 16
    B, nblk = 5, 200
    st_ = I.install_hooks(make_runner({"l0": FakeFlashImpl(hq, hkv, D)}, dev,
                                      {"l0": torch.zeros(2, nblk, bs, hkv, D, dtype=torch.bfloat16, device=dev)}),
                          calibration_covariances={"l0": R.fit_sigma_centered(sample_keys(64, seed=191))},
                          key_bits=3, initial_layers_count=0, mode=V.MODE_HYBRID, paged=True)["l0"]
    pc = st_.paged
    g = torch.Generator().manual_seed(192)
    pc.ensure(nblk, bs, torch.bfloat16, torch.bfloat16, dev)
    slots = torch.randperm(nblk * bs, generator=g)[: 600].to(dev)
    keys = sample_keys(600 * hkv, seed=193).reshape(600, hkv, D).bfloat16().to(dev)
    vals = torch.randn(600, hkv, D, generator=g).bfloat16().to(dev)
    pc.write(keys, vals, slots)
    table = torch.randint(0, nblk, (B, 40), generator=g, dtype=torch.int32).to(dev)
    made = []
    for step, lens in enumerate([[100, 300, 17, 250, 64], [101, 301, 18, 251, 65], [101, 520, 18, 251, 65]]):
        q = torch.randn(B, hq, D, generator=torch.Generator().manual_seed(200 + step)).bfloat16().to(dev)
        sl = torch.tensor(lens, dtype=torch.int32, device=dev)
        out = torch.empty(B, hq, D, dtype=torch.bfloat16, device=dev)
        pc.decode(q, table, sl, max(lens), hq, 1.0 / D ** 0.5, out)
        made.append(len(pc._plans))
        pools = {name: t.view(nblk, hkv, bs, *t.shape[1:]) for name, t in pc.pools.items()}
        fresh = PagedQuantizedKV(st_.store.key_strategy, pools["k_codes"], pools["k_norms"], pools["v_data"],
                                 pools["v_scales"], pools["v_zeros"], table, lens, bs, 2, 32)
        want = fresh.attention(q, scale=1.0 / D ** 0.5)
        assert_attn_close(out, want.cpu(), f"paged plan re-use step {step}")
    assert made == [1, 1, 2]
