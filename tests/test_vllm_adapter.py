"""Host logic of the vLLM adapter (smaq/integration/vllm.py,
smaq/vllm_attn_backend.py) against fake vLLM objects, on the CPU: hook
installation, mode handling, pass-through paths, statistics and cache freeing.
Nothing here reaches a HIP kernel (no store receives tokens); the serving
paths are covered by tests/test_gpu_vllm_adapter.py."""

from __future__ import annotations

import logging

import pytest
import torch

import smaq_amd.integration as I
import smaq_amd.integration.vllm as V
import smaq_amd.vllm_attn_backend as LB
from tests.vllm_fakes import FakeFlashImpl, FakeFlashImplNoUpdate, FakeMLAImpl, make_runner, meta

CPU = torch.device("cpu")


@pytest.fixture(autouse=True)
def _restore_modes():
    yield
    V.set_mode(V.MODE_CAPTURE_ONLY)
    LB._GLOBAL_MODE = LB.MODE_ACCUMULATE


def _runner(n_layers=2, hq=8, hkv=2, d=64, mla=False, with_cache=True, blocks=4, bs=16):
    impls = {f"model.layers.{i}.self_attn.attn": FakeFlashImpl(hq, hkv, d) for i in range(n_layers)}
    if mla:
        impls["model.layers.mla.attn"] = FakeMLAImpl()
    caches = None
    if with_cache:
        caches = {name: torch.zeros(2, blocks, bs, hkv, d) for name in impls if "mla" not in name}
    return make_runner(impls, CPU, caches), impls


def test_modes_and_validation():
    assert I.get_mode() == V.MODE_CAPTURE_ONLY
    for m in (V.MODE_OFF, V.MODE_HYBRID, V.MODE_FULL_SMAQ, V.MODE_CAPTURE_ONLY):
        I.set_mode(m)
        assert I.get_mode() == m
    with pytest.raises(ValueError):
        I.set_mode("turbo")
    with pytest.raises(ValueError):
        LB.set_mode("hybrid")
    LB.set_mode(LB.MODE_ACTIVE)
    assert LB.get_mode() == LB.MODE_ACTIVE and V.get_mode() == V.MODE_HYBRID
    LB.set_mode(LB.MODE_SHADOW)
    assert V.get_mode() == V.MODE_CAPTURE_ONLY


def test_install_hooks_layer_configs():
    runner, impls = _runner(n_layers=6, mla=True)
    sig = torch.eye(64) * 2.0
    states = I.install_hooks(runner, calibration_covariances={"model.layers.1.self_attn.attn": sig},
                             initial_layers_count=4, mode=V.MODE_OFF)
    names = list(states)
    assert len(states) == 7 and "not_attention" not in states
    # layer order follows the forward context; the first 4 get key_bits + 1
    bits = [states[n].config.key_bits for n in names]
    assert bits == [4, 4, 4, 4, 3, 3, 3]
    st1 = states["model.layers.1.self_attn.attn"]
    assert st1.config.Sigma_q is sig and st1.config.num_query_heads == 8 and st1.config.head_dim == 64
    mla = states["model.layers.mla.attn"]
    assert mla.config.backend_kind == "mla" and not mla.supports_hybrid and mla.config.head_dim == 64
    assert all(states[n].config.layer_idx == i for i, n in enumerate(names))
    assert runner._smaq_layer_states is states and runner._smaq_no_alloc is False
    assert V.get_mode() == V.MODE_OFF
    for name, impl in impls.items():
        assert impl._smaq_layer_state is states[name]
    # explicit initial-layer bits and value group clamp
    runner2, _ = _runner(n_layers=2, d=16)
    st2 = I.install_hooks(runner2, key_bits=2, initial_layers_count=1, initial_layers_key_bits=3,
                          value_group_size=32)
    assert [s.config.key_bits for s in st2.values()] == [3, 2]
    assert all(s.config.value_group_size == 16 for s in st2.values())


def test_query_head_inference():
    impl = FakeFlashImpl(0, 2, 64)
    impl.num_heads = None
    r = make_runner({"a": impl}, CPU, num_heads={"a": 12})
    assert I.install_hooks(r)["a"].config.num_query_heads == 12
    impl2 = FakeFlashImpl(0, 2, 64)
    impl2.num_heads = None
    r2 = make_runner({"b": impl2}, CPU)
    assert I.install_hooks(r2)["b"].config.num_query_heads == 2


def test_passthrough_off_and_capture_only():
    runner, impls = _runner(n_layers=1)
    name = next(iter(impls))
    impl = impls[name]
    states = I.install_hooks(runner, mode=V.MODE_OFF)
    st = states[name]
    kv = runner.compilation_config.static_forward_context[name].kv_cache[0]
    k = torch.randn(5, 2, 64)
    v = torch.randn(5, 2, 64)
    slots = torch.tensor([0, 1, 2, 3, 4])
    impl.do_kv_cache_update(None, k, v, kv, slots)
    assert impl.calls == ["update"] and st.engine.ring.size == 0
    assert torch.equal(kv[0].view(-1, 2, 64)[:5], k)
    # capture-only: the layer still writes, the ring receives the prefill
    I.set_mode(V.MODE_CAPTURE_ONLY)
    impl.do_kv_cache_update(None, k, v, kv, slots)
    assert st.engine.ring.size == 5 and st.store.num_tokens == 0
    impl.do_kv_cache_update(None, k[:1], v[:1], kv, slots[:1])
    assert st.engine.ring.size == 6
    # forward falls through to the layer's own attention in both modes
    q = torch.randn(1, 8 * 64)
    m = meta(1, 1, seq_lens=torch.tensor([5]), block_table=torch.tensor([[0]]))
    out = impl.forward(None, q, k[:1], v[:1], kv, m)
    assert impl.calls[-1] == "forward" and out.shape == (1, 8, 64)
    assert impl.forward(None, q, k, v, kv, None) is q


def test_hybrid_below_min_history_falls_through():
    """Hybrid mode with fewer than 16 compressed tokens serves nothing itself
    (smaq/integration/vllm.py:224-226): the layer's forward runs, and with
    no_alloc a zero result is returned."""
    runner, impls = _runner(n_layers=1)
    name = next(iter(impls))
    impl = impls[name]
    I.install_hooks(runner, mode=V.MODE_HYBRID)
    kv = runner.compilation_config.static_forward_context[name].kv_cache[0]
    q = torch.randn(2, 8, 64)
    m = meta(2, 1, seq_lens=torch.tensor([1, 1]), block_table=torch.tensor([[0], [1]]))
    impl.forward(None, q, q[:, :2], q[:, :2], kv, m)
    assert impl.calls == ["forward"]
    runner2, impls2 = _runner(n_layers=1)
    impl2 = next(iter(impls2.values()))
    I.install_hooks(runner2, mode=V.MODE_HYBRID, no_alloc=True)
    z = impl2.forward(None, q, q[:, :2], q[:, :2], kv, m)
    assert impl2.calls == [] and torch.equal(z, torch.zeros_like(q))
    z2 = impl2.forward(None, q.reshape(2, -1), q[:, :2], q[:, :2], kv, m)
    assert z2.shape == (2, 8 * 64) and not z2.any()


def test_no_alloc_prefill_sdpa():
    """no_alloc prefill: causal SDPA over the step's tokens with GQA by
    repetition, delivered into `output` (smaq/integration/vllm.py:133-218)."""
    runner, impls = _runner(n_layers=1, hq=4, hkv=2, d=32)
    impl = next(iter(impls.values()))
    I.install_hooks(runner, mode=V.MODE_HYBRID, no_alloc=True)
    g = torch.Generator().manual_seed(0)
    T = 7
    q = torch.randn(T, 4, 32, generator=g)
    k = torch.randn(T, 2, 32, generator=g)
    v = torch.randn(T, 2, 32, generator=g)
    out = torch.zeros(T + 2, 4 * 32)
    res = impl.forward(None, q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1), None, meta(T, T), output=out)
    assert res is out and impl.calls == []
    kk, vv = k.repeat_interleave(2, 1), v.repeat_interleave(2, 1)
    s = torch.einsum("thd,shd->hts", q, kk) / 32 ** 0.5
    s = s.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    ref = torch.einsum("hts,shd->thd", s.softmax(-1), vv)
    assert torch.allclose(out[:T].view(T, 4, 32), ref, atol=1e-5)
    assert not out[T:].any()
    res3 = impl.forward(None, q, k, v, None, meta(T, T))
    assert res3.shape == (T, 4, 32) and torch.allclose(res3, ref, atol=1e-5)


def test_forward_capture_without_separate_update():
    impl = FakeFlashImplNoUpdate(8, 2, 64)
    runner = make_runner({"l0": impl}, CPU, {"l0": torch.zeros(2, 4, 16, 2, 64)})
    states = I.install_hooks(runner, mode=V.MODE_CAPTURE_ONLY)
    assert not hasattr(impl, "do_kv_cache_update")
    k = torch.randn(3, 2, 64)
    impl.forward(None, torch.randn(3, 8, 64), k, k, runner.kv_caches[0], meta(3, 3))
    assert states["l0"].engine.ring.size == 3 and impl.calls == ["forward"]
    V.set_mode(V.MODE_OFF)
    impl.forward(None, torch.randn(3, 8, 64), k, k, runner.kv_caches[0], meta(3, 3))
    assert states["l0"].engine.ring.size == 3


def test_mla_passthrough(caplog):
    mla = FakeMLAImpl()
    runner = make_runner({"mla": mla}, CPU)
    I.install_hooks(runner, mode=V.MODE_HYBRID)
    with caplog.at_level(logging.INFO, logger="smaq.integration.vllm"):
        mla.do_kv_cache_update(None, None, None, None, None, None)
        mla.do_kv_cache_update(None, None, None, None, None, None)
    assert mla.calls == ["mla_update", "mla_update"]
    assert sum("MLA update observed" in r.getMessage() for r in caplog.records) == 1
    q = torch.randn(2, 3)
    assert mla.forward_mqa(q, None, None, None) is q and mla.calls[-1] == "mla_forward"


def test_stats_and_free_kv_cache():
    assert I.get_stats(make_runner({}, CPU)) == {}
    assert I.free_kv_cache(make_runner({}, CPU)) == 0
    runner, impls = _runner(n_layers=2, mla=True, blocks=4, bs=16, hkv=2, d=64)
    runner.kv_caches.append(torch.zeros(3))       # a cache the adapter does not own
    states = I.install_hooks(runner, mode=V.MODE_CAPTURE_ONLY)
    name0 = next(iter(impls))
    k = torch.randn(4, 2, 64)
    impls[name0].do_kv_cache_update(None, k, k, runner.compilation_config.static_forward_context[name0].kv_cache[0],
                                    torch.arange(4))
    stats = I.get_stats(runner)
    assert stats[name0] == {"compressed_tokens": 0, "buffered_tokens": 4, "memory_bytes": 0,
                            "supports_hybrid": True}
    assert stats["_totals"] == {"compressed_tokens": 0, "buffered_tokens": 4, "memory_bytes": 0, "layers": 3}
    freed = I.free_kv_cache(runner)
    assert freed == 2 * (2 * 4 * 16 * 2 * 64 * 4)
    ctx = runner.compilation_config.static_forward_context
    for name in impls:
        if "mla" not in name:
            assert ctx[name].kv_cache[0].numel() == 1
    assert [t.numel() for t in runner.kv_caches] == [1, 1, 3]
    assert set(states) == set(I.get_stats(runner)) - {"_totals"}


def test_legacy_install_and_no_alloc_inert(caplog):
    runner, _ = _runner(n_layers=1)
    states = LB.install_smaq_hooks(runner, mode=LB.MODE_ACTIVE, buffer_size=64, no_alloc=True)
    st = next(iter(states.values()))
    assert LB.get_mode() == LB.MODE_ACTIVE and V.get_mode() == V.MODE_HYBRID
    assert st.config.ring_capacity == 64 and st.engine.ring.capacity == 64
    assert runner._smaq_states is states and runner._smaq_no_alloc is True
    runner2, _ = _runner(n_layers=1)
    LB.install_smaq_hooks(runner2, mode="bogus")
    assert V.get_mode() == V.MODE_CAPTURE_ONLY
    with caplog.at_level(logging.WARNING, logger="smaq.attn"):
        assert LB.enable_no_alloc(key_bits=4) is None
    assert LB._SMAQ_NO_ALLOC_CONFIG["key_bits"] == 4
    assert any("inert" in r.getMessage() for r in caplog.records)


def test_paged_layer_geometry_checks():
    runner, impls = _runner(n_layers=1, blocks=4, bs=16, hkv=2, d=64)
    states = I.install_hooks(runner, mode=V.MODE_HYBRID, paged=True)
    st = next(iter(states.values()))
    assert st.paged is not None and st.paged.pools is None and st.config.paged
    with pytest.raises(ValueError):
        V.PagedLayerCache.cache_geometry(torch.zeros(2, 4, 16, 3, 64), 2, 64)
    assert V.PagedLayerCache.cache_geometry(torch.zeros(2, 4, 16, 2, 64), 2, 64) == (4, 16)
    # MLA layers never get pools
    runner2 = make_runner({"mla": FakeMLAImpl()}, CPU)
    assert I.install_hooks(runner2, paged=True)["mla"].paged is None


def test_enable_no_alloc_patches_fake_vllm(monkeypatch):
    """With (fake) vLLM importable: the executor's KV-cache sizing first
    installs active no-alloc hooks on every worker through collective_rpc
    (the call is picklable, carrying the recorded configuration), the runner's
    layout update maps shared-cache layers, and patching happens once."""
    import pickle
    import sys
    import types

    class Executor:
        def __init__(self, workers):
            self.workers, self.rpc_calls = workers, 0

        def collective_rpc(self, fn):
            self.rpc_calls += 1
            fn = pickle.loads(pickle.dumps(fn))      # what a multi-process executor does
            return [fn(w) for w in self.workers]

        def get_kv_cache_specs(self):
            return "specs"

    class GPUModelRunner:
        def _update_hybrid_attention_mamba_layout(self, kv_caches):
            return sorted(kv_caches)

    mods = {"vllm": types.ModuleType("vllm"), "vllm.v1": types.ModuleType("vllm.v1"),
            "vllm.v1.executor": types.ModuleType("vllm.v1.executor"),
            "vllm.v1.executor.abstract": types.ModuleType("vllm.v1.executor.abstract"),
            "vllm.v1.worker": types.ModuleType("vllm.v1.worker"),
            "vllm.v1.worker.gpu_model_runner": types.ModuleType("vllm.v1.worker.gpu_model_runner")}
    mods["vllm.v1.executor.abstract"].Executor = Executor
    mods["vllm.v1.worker.gpu_model_runner"].GPUModelRunner = GPUModelRunner
    for name, mod in mods.items():
        monkeypatch.setitem(sys.modules, name, mod)
    monkeypatch.setattr(LB, "_SMAQ_NO_ALLOC_CONFIG", None)

    runner, _ = _runner(n_layers=2)
    worker = types.SimpleNamespace(model_runner=runner)
    ex = Executor([worker])
    assert ex.get_kv_cache_specs() == "specs" and ex.rpc_calls == 0       # before enable: untouched
    LB.enable_no_alloc(buffer_size=32, key_bits=4)
    LB.enable_no_alloc(buffer_size=32, key_bits=4)                        # idempotent
    assert Executor._smaq_patched and GPUModelRunner._smaq_layout_patch
    assert ex.get_kv_cache_specs() == "specs" and ex.rpc_calls == 1
    states = runner._smaq_states
    assert len(states) == 2 and runner._smaq_no_alloc is True
    st = next(iter(states.values()))
    assert st.engine.ring.capacity == 32 and st.config.key_bits == 4
    assert LB.get_mode() == LB.MODE_ACTIVE and V.get_mode() == V.MODE_HYBRID
    gm = GPUModelRunner()
    gm.shared_kv_cache_layers = {"b": "a", "c": "missing"}
    caches = {"a": 1}
    assert gm._update_hybrid_attention_mamba_layout(caches) == ["a", "b"] and caches["b"] == 1


def test_reference_logger_names():
    """The adapter, the backend installer and the score-kernel seam log
    under the reference's logger names (smaq/integration/vllm.py:25,
    smaq/vllm_attn_backend.py:14, smaq/triton_kernels.py:20), so a
    deployment's logging configuration applies unchanged."""
    import smaq_amd.kernels as K
    import smaq_amd.vllm_attn_backend as B
    assert V.logger.name == "smaq.integration.vllm"
    assert B.logger.name == "smaq.attn"
    assert K.logger.name == "smaq.triton"
