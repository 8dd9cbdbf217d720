"""The allocation-free attention entry point (smaq_attn_hybrid_noalloc)
against the workspace entry point (smaq_attn_hybrid), both called through
the C ABI with the same parameters: outputs must be bit-identical (same
kernels).  Calls run back to back with shrinking inputs, so a later call
finds the previous call's partials in the built-in scratch array."""

from __future__ import annotations

import pytest
import torch

import smaq_amd as S
from smaq_amd import _native
from smaq_amd.batch import PagedQuantizedKV, QuantizedKVBatch
from smaq_amd.synthetic import sample_keys as dev_sample_keys
from tests.conftest import sample_keys

pytestmark = pytest.mark.gpu


def _strategy(dev, seed):
    return S.SMAQFullMetricScalarStrategy(128, bits=3, device=dev).fit(sample_keys(64, seed=seed))


def _both(plan, q, dev, what):
    """Run one plan through both entry points; compare bit for bit."""
    plan.load_query(q)
    _native.attn_hybrid(plan.params, dev)
    ref = plan.out.clone()
    plan.out.fill_(float("nan"))
    _native.attn_hybrid_noalloc(plan.params, dev)
    torch.cuda.synchronize(dev)
    assert torch.equal(plan.out, ref), f"{what}: noalloc output differs"
    assert not torch.isnan(ref.float()).any(), f"{what}: NaN output"
    return ref


def test_noalloc_matches_workspace_entry_point(dev):
    g = torch.Generator().manual_seed(190)
    strat = _strategy(dev, 191)
    # 1) c3-shaped uniform batch on the matrix-core decode kernel, several splits
    B, N = 16, 8192
    keys = dev_sample_keys(B * N * 8, seed=192, device=dev, dtype=torch.bfloat16).view(B, N, 8, 128)
    vals = torch.randn(B, N, 8, 128, generator=torch.Generator(device=dev).manual_seed(189), device=dev).bfloat16()
    kvb = QuantizedKVBatch.encode(strat, keys, vals)
    q = torch.randn(B, 1, 32, 128, generator=g).bfloat16().to(dev)
    plan = kvb.plan(q)
    assert _native.attn_workspace_bytes(plan.params) <= _native.NOALLOC_SCRATCH_BYTES
    _both(plan, q, dev, "uniform decode 16 x 8192")
    del keys, vals
    # 2) smaller ragged batch with an exact recent window (longest-first order,
    #    recent partials, combine over history + recent)
    lens = [700, 90, 1500]
    keys = [sample_keys(n * 8, seed=193 + i).view(n, 8, 128).bfloat16().to(dev) for i, n in enumerate(lens)]
    vals = [torch.randn(n, 8, 128, generator=g).bfloat16().to(dev) for n in lens]
    kvr = QuantizedKVBatch.encode(strat, keys, vals)
    q2 = torch.randn(3, 1, 32, 128, generator=g).bfloat16().to(dev)
    rk = torch.randn(3, 16, 8, 128, generator=g).bfloat16().to(dev)
    rv = torch.randn(3, 16, 8, 128, generator=g).bfloat16().to(dev)
    plan2 = kvr.plan(q2, recent_k=rk, recent_v=rv, recent_len=torch.tensor([16, 5, 11], device=dev))
    _both(plan2, q2, dev, "ragged decode + recent window")
    # 3) smaller still: paged history on the generic kernels
    plens = [40, 200]
    nblk = [(n + 15) // 16 for n in plens]
    table = torch.zeros(2, max(nblk), dtype=torch.int32)
    perm = torch.randperm(sum(nblk), generator=g)
    table[0, :nblk[0]] = perm[:nblk[0]].to(torch.int32)
    table[1, :nblk[1]] = perm[nblk[0]:].to(torch.int32)
    pk = PagedQuantizedKV.encode(strat, [sample_keys(n * 8, seed=197 + i).view(n, 8, 128).bfloat16().to(dev)
                                         for i, n in enumerate(plens)],
                                 [torch.randn(n, 8, 128, generator=g).bfloat16().to(dev) for n in plens],
                                 table.to(dev), num_blocks=sum(nblk), block_size=16)
    q3 = torch.randn(2, 1, 32, 128, generator=g).bfloat16().to(dev)
    _both(pk.plan(q3, impl=1), q3, dev, "paged, generic kernels")


def test_noalloc_rejects_oversized_workspace(dev):
    """A shape whose workspace exceeds the built-in scratch is refused before
    any launch, and the workspace entry point still serves it."""
    p = _native.AttnParams()
    p.batch, p.q_len, p.n_q_heads, p.n_kv_heads, p.head_dim = 4096, 1, 32, 8, 128
    p.has_history, p.max_hist_len, p.impl = 1, 1 << 20, 1
    assert _native.attn_workspace_bytes(p) > _native.NOALLOC_SCRATCH_BYTES
    with pytest.raises(ValueError, match="built-in scratch"):
        _native.attn_hybrid_noalloc(p, dev)
