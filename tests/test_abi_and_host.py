"""CPU tests: the C ABI library loads and exports every declared entry point,
status codes map to the reference's exception types, and the host-side
logic (tables, calibration, row addressing, ring buffer, capture routing,
strategy plumbing) matches the oracle.  No kernel is launched."""

from __future__ import annotations

import ctypes
import re
import types
from pathlib import Path

import pytest
import torch

import smaq_amd as S
from smaq_amd import _native
from oracle import smaq_ref as R
from tests.conftest import sample_keys, spectral_sigma

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    text = (ROOT / "include" / "smaq_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(smaq_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    declared = _declared_symbols()
    assert len(declared) >= 12
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/smaq_hip.h but not exported"
    assert set(declared) == set(_native.EXPORTED)
    assert lib.smaq_version() == 100


def test_status_codes_map_to_exceptions():
    lib = _native.lib()
    # null pointers: rejected before any device call
    st = lib.smaq_pack_values(None, 0, 1, 1, 0, 0, 0, 128, 2, 32, None, None, None, None)
    assert st == -1
    assert b"null pointer" in lib.smaq_last_error()
    with pytest.raises(ValueError, match="null pointer"):
        _native._check(st, "smaq_pack_values")
    dummy = ctypes.c_void_p(16)
    st = lib.smaq_pack_values(dummy, 0, 1, 1, 0, 0, 0, 100, 2, 32, dummy, dummy, dummy, None)
    assert st == -1 and b"divisible by group_size" in lib.smaq_last_error()
    st = lib.smaq_encode_blockvq(dummy, 0, 1, 1, 0, 0, 0, 16, 8, 512, dummy, dummy, dummy, None, None)
    assert st == -1 and b"n_centroids" in lib.smaq_last_error()
    st = lib.smaq_encode_scalar(dummy, 0, 1, 1, 0, 0, 0, 512, dummy, None, dummy, 7, 3, dummy, dummy, None, None)
    assert st == -1 and b"head_dim" in lib.smaq_last_error()
    st = lib.smaq_pack_values(dummy, 7, 1, 1, 0, 0, 0, 128, 2, 32, dummy, dummy, dummy, None)
    assert st == -2
    with pytest.raises(RuntimeError):
        _native._check(st, "smaq_pack_values")
    p = _native.AttnParams()
    assert lib.smaq_attn_hybrid(ctypes.byref(p), None) == -1


def test_attn_workspace_size():
    p = _native.AttnParams()
    p.batch, p.q_len, p.n_q_heads, p.n_kv_heads, p.head_dim = 32, 1, 32, 8, 128
    p.has_history, p.max_hist_len = 1, 32768
    n = _native.attn_workspace_bytes(p)
    assert n > 0 and n % 4 == 0


def test_cpu_tensors_fail_loudly():
    qz = S.SMAQQuantizer(128, bits=3, device="cpu")
    with pytest.raises(ValueError, match="HIP kernels"):
        qz.quantize(torch.randn(4, 128))
    with pytest.raises(ValueError, match="HIP kernels"):
        S.quantize_values(torch.randn(4, 128))


@pytest.mark.parametrize("shape,perm", [((5, 8, 128), None), ((64, 8, 128), (1, 0, 2)), ((1, 3, 7, 128), None)])
def test_row_view(shape, perm):
    x = torch.arange(torch.Size(shape).numel(), dtype=torch.float32).reshape(shape)
    if perm:
        x = x.permute(*perm).unsqueeze(0)
    no, ni, so, si = _native.row_view(x)
    flat = x.reshape(-1, x.shape[-1])
    base = x.storage_offset()
    store = x.untyped_storage()
    src = torch.tensor([], dtype=torch.float32).set_(store)
    for r in range(flat.shape[0]):
        o, i = divmod(r, ni)
        assert torch.equal(src[base + o * so + i * si: base + o * so + i * si + x.shape[-1]], flat[r])


def test_codec_tables_match_oracle():
    for bits in (2, 3, 4):
        qz = S.SMAQQuantizer(128, bits=bits, device="cpu")
        c, b, db = R.scalar_tables(bits)
        assert torch.equal(qz.centroids, c) and torch.equal(qz.boundaries, b)
        assert torch.equal(qz.decision_boundaries, db)
        ad = S.RotationAdapter(128, bits=bits, device="cpu")
        c2, b2, db2 = R.midpoint_tables(bits)
        assert torch.equal(ad.centroids, c2) and torch.equal(ad.decision_boundaries, db2)


def test_fit_matches_oracle():
    q = sample_keys(64, seed=3)
    qz = S.SMAQQuantizer(128, bits=4, device="cpu").fit(q)
    E, Ei = R.build_metric(R.fit_sigma_centered(q))
    assert torch.equal(qz.E, E) and torch.equal(qz.E_inv, Ei)
    sigma, _, _ = spectral_sigma(128, 4)
    qz2 = S.SMAQQuantizer(128, Sigma_q=sigma, device="cpu")
    E2, _ = R.build_metric(sigma)
    assert torch.equal(qz2.E, E2)
    sd = qz.state_dict()
    assert set(sd) == {"E", "E_inv", "centroids", "boundaries", "decision_boundaries"}


def test_blockvq_fit_host_matches_oracle():
    keys, queries = sample_keys(1024, seed=5), sample_keys(1024, seed=6)
    vq = S.SMAQBlockVQ(128, block_dim=8, n_centroids=32, device="cpu").fit(keys, queries, kmeans_iters=2)
    Eb, Eib, C, Dc = R.blockvq_fit(keys, queries, block_dim=8, n_centroids=32, iters=2)
    assert torch.equal(vq.E_blocks, Eb) and torch.equal(vq.centroids, C) and torch.equal(vq.decoded_centroids, Dc)
    with pytest.raises(ValueError):
        S.SMAQBlockVQ(100, block_dim=8)


def test_ring_buffer_matches_oracle():
    ring = S.RingBuffer(8, 2, 4, device=torch.device("cpu"), dtype=torch.float32)
    ref = R.Ring(8, 2, 4, dtype=torch.float32)
    g = torch.Generator().manual_seed(0)
    for n in (3, 5, 1, 9, 16, 2, 7):
        x = torch.randn(n, 2, 4, generator=g)
        a, b = ring.write(x, x + 1, n), ref.write(x, x + 1, n)
        assert (a is None) == (b is None)
        if a is not None:
            assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
        pa, pb = ring.peek(), ref.peek()
        assert (pa is None) == (pb is None)
        if pa is not None:
            assert torch.equal(pa[0], pb[0])
    assert ring.total_written == ref.total


@pytest.mark.parametrize("cap", [1, 3, 8])
def test_ring_buffer_spill_arithmetic(cap):
    """Random write sizes (empty, single, several capacities at once, writes
    into a full ring) against the oracle's slot-by-slot restatement; inputs
    in another dtype spill in the ring's dtype, as writing them into the
    slots first would."""
    g = torch.Generator().manual_seed(cap)
    ring = S.RingBuffer(cap, 2, 4, device=torch.device("cpu"), dtype=torch.bfloat16)
    ref = R.Ring(cap, 2, 4, dtype=torch.bfloat16)
    for step in range(60):
        n = int(torch.randint(0, 3 * cap + 2, (1,), generator=g))
        x = torch.randn(max(n, 1), 2, 4, generator=g)           # fp32 input
        a, b = ring.write(x, 2 * x, n), ref.write(x, 2 * x, n)
        assert (a is None) == (b is None), step
        if a is not None:
            assert a[0].dtype == torch.bfloat16
            assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]), step
        pa, pb = ring.peek(), ref.peek()
        assert (pa is None) == (pb is None), step
        if pa is not None:
            assert torch.equal(pa[0], pb[0]) and torch.equal(pa[1], pb[1]), step
    assert ring.total_written == ref.total


class _FakeStore:
    """Records append_chunk calls (the reference tests' SimpleNamespace idiom)."""

    def __init__(self):
        self.num_kv_heads, self.head_dim, self.device = 1, 4, torch.device("cpu")
        self.chunks = []
        self.num_tokens = 0

    def append_chunk(self, k, v):
        self.chunks.append(k.clone())
        self.num_tokens += k.shape[0]

    def reset(self):
        self.chunks.clear()


def test_capture_engine_routing():
    st = _FakeStore()
    eng = S.KVCaptureEngine(st, ring_capacity=4, device=torch.device("cpu"), dtype=torch.float32)
    x = torch.arange(40, dtype=torch.float32).reshape(10, 1, 4)
    eng.ingest_prefill(x, x, 10)                 # 6 compressed, last 4 exact
    assert [c.shape[0] for c in st.chunks] == [6] and eng.total_buffered_tokens == 4
    eng.ingest_decode(x[:1], x[:1], 1)           # ring full -> whole ring flushed
    assert [c.shape[0] for c in st.chunks] == [6, 4] and eng.total_buffered_tokens == 1
    assert torch.equal(st.chunks[1], x[6:10])
    eng.flush()
    assert [c.shape[0] for c in st.chunks] == [6, 4, 1]
    # paged prefill gather [2, blocks, bs, H, D]
    kv = torch.arange(2 * 5 * 2 * 1 * 4, dtype=torch.float32).reshape(2, 5, 2, 1, 4)
    st2 = _FakeStore()
    eng2 = S.KVCaptureEngine(st2, ring_capacity=2, device=torch.device("cpu"), dtype=torch.float32)
    eng2.ingest_prefill_from_paged_cache(kv, 5, torch.tensor([3, 0, 4]), 2)
    want = torch.cat([kv[0, 3], kv[0, 0], kv[0, 4, :1]])
    assert torch.equal(st2.chunks[0], want[:3])
    assert torch.equal(eng2.ring.peek()[0], want[3:])


def test_strategy_plumbing_and_memory_bytes():
    s = S.SMAQFullMetricScalarStrategy(128, bits=3, device="cpu")
    a = S.SMAQQuantized(torch.zeros(1, 2, 5, 64, dtype=torch.uint8), torch.zeros(1, 2, 5), 3)
    b = S.SMAQQuantized(torch.ones(1, 2, 3, 64, dtype=torch.uint8), torch.ones(1, 2, 3), 3)
    cat = s.concat_quantized([s.flatten_quantized(a), s.flatten_quantized(b)])
    assert cat.indices.shape == (2, 8, 64) and cat.norms.shape == (2, 8)
    assert s.select_head(cat, 1).indices.shape == (8, 64)
    assert s.memory_bytes(cat) == 2 * 8 * 64 + 2 * 8 * 2
    assert s.supports_kernel and s.fused_history().kind == "scalar"
    caps = S.ExactShadowStrategy().capabilities
    assert caps.compressed_history_shadow_only and not caps.values_compressed
    vqs = S.SMAQBlockVQStrategy(128, device="cpu")
    q = S.BlockVQQuantized(torch.zeros(2, 7, 16, dtype=torch.uint8), 16, 8)
    assert vqs.memory_bytes(q) == 2 * 7 * 16
    assert vqs.fused_history().kind == "block_vq"


def test_calibration_providers():
    p = S.StaticCalibrationProvider({0: "s0", "layer_1": "s1"})
    assert p.get_sigma_q(0, 64) == "s0" and p.get_sigma_q(1, 64) == "s1" and p.get_sigma_q(2, 64) is None
    assert S.IdentityCalibrationProvider().get_sigma_q(0, 128) is None
    caps = S.CacheCapabilities("diag", "m", "scalar", True, False, True, True, False)
    assert caps.compressed_history and not caps.compressed_history_shadow_only


def test_fake_layer_namespace_idiom():
    """The reference tests' fake-shape idiom still works against the contracts."""
    info = S.LayoutInfo("generic", 128, 128, 128)
    assert not info.unified_kv
    fake = types.SimpleNamespace(shape=(1, 8, 16, 128))
    assert fake.shape[-1] == 128


def test_attn_params_mirror_the_header():
    """The ctypes AttnParams lists the fields of include/smaq_hip.h's
    smaq_attn_params in the same order with the same kinds (int, float,
    long long, pointer), hist_rows last: the struct layout both sides read."""
    import re
    from pathlib import Path
    hdr = (Path(__file__).resolve().parents[1] / "include" / "smaq_hip.h").read_text()
    body = hdr[hdr.index("typedef struct smaq_attn_params {"):hdr.index("} smaq_attn_params;")]
    body = re.sub(r"/\*.*?\*/", "", body.split("{", 1)[1], flags=re.S)
    fields = []
    for decl in body.split(";"):
        decl = " ".join(decl.split())
        if not decl:
            continue
        m = re.match(r"((?:const )?(?:unsigned )?(?:long long|int|float|void|char)\s*\**)\s*(.*)", decl)
        assert m, decl
        base, names = m.group(1), m.group(2)
        for nm in names.split(","):
            nm = nm.strip()
            ptr = "*" in base or nm.startswith("*")
            nm = nm.lstrip("*").strip()
            kind = "ptr" if ptr else ("ll" if "long long" in base else ("float" if "float" in base else "int"))
            fields.append((nm, kind))
    kinds = {ctypes.c_int: "int", ctypes.c_float: "float", ctypes.c_longlong: "ll", ctypes.c_void_p: "ptr"}
    mirror = [(nm, kinds[t]) for nm, t in _native.AttnParams._fields_]
    assert mirror == fields
    assert fields[-1] == ("hist_rows", "ll")
