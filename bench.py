#!/usr/bin/env python
"""SMAQ quantized-KV hot path benchmark on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload all|decode|paged|prefill|encode]

Prints ONE JSON line.  The default (``all``) runs the four BASELINE workloads
back to back on one GPU; the headline fields are config 3, the others are
records under ``extra``:

* c3 (headline) fused quantized-KV decode attention at Llama-3-8B shape --
  batch 32, context 32768, 32 query / 8 KV heads, head_dim 128, 3-bit scalar
  SMAQ keys (calibrated metric), 2-bit values (group 32), bf16 storage and
  queries, one new token per sequence.  One step = one decode-attention pass
  of one layer over the whole batch, cache resident in HBM; ``value`` is
  tokens/s = batch / step time.
* c5 paged decode (256 sequences, 16-token blocks, shuffled block tables).
* c4 hybrid chunked prefill (2048 causal queries over 65408 block-VQ history
  tokens + 128 exact recent tokens, Qwen2-7B heads).
* c2 block-VQ key encode + 2-bit value pack of 4.19M bf16 token-heads.

Every workload: a settle phase (back-to-back steps for ``--settle-ms`` of
wall time: on MI355X the first few ms of a heavy load run inside a
power-management transient during which this kernel first runs fast, then
up to 30% slower, before it settles), then W untimed warm-up steps, then K
timed steps between two HIP events on the launch stream.  ``roofline`` is
the dominant kernel alone: HIP events on its launch stream (torch's current
stream) around K back-to-back launches, against its algorithmic bytes or
flops.  ``cpu_baseline`` times the CPU oracle (the op-for-op torch
restatement of the reference) on a bounded sample on this host.
"""

from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "quantized-KV decode attn tokens/s + achieved HBM GB/s (% peak); encode GB/s"
HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3
F16_PEAK_TFLOPS = 2500.0

# What the decode kernels compute in (storage is bf16): QK as three f16
# products of hi/lo splits (~22-bit scores), PV as two bf16 products of a
# hi/lo split weight against exact 2-bit codes, fp32 softmax and accumulation.
DECODE_DTYPE = "bf16 storage; QK 3x f16 hi/lo MFMA (~22-bit), PV 2x bf16 hi/lo MFMA on exact codes, fp32 accumulate"
PREFILL_DTYPE = ("fp16 storage; QK f16 hi/lo keys x f16 queries (2x f16 MFMA, +1 when a query is not f16-exact), "
                 "PV f16 values x f16 hi/lo weights (2x f16 MFMA; +1 with a value-lo plane on key ranges whose "
                 "f16 value rounding exceeds 1.96e-3), fp32 accumulate")
ENCODE_DTYPE = "bf16 in; fp32-exact distances (f16 hi/lo MFMA + exact recount), u8 indices, 2-bit values"


def _events(n):
    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def cpu_threads() -> int:
    """Threads the CPU baseline uses: the host's cores as this process may use
    them (affinity), capped by OMP_NUM_THREADS when the environment sets it
    (the GPU boxes give one GPU's job a 16-thread share of the host)."""
    n = os.cpu_count() or 1
    try:
        n = min(n, len(os.sched_getaffinity(0)))
    except AttributeError:
        pass
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return n


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_fields() -> dict:
    return {"cores": torch.get_num_threads(), "cpu_model": cpu_model(), "cpu_count": os.cpu_count()}


def settle(step, ms: float) -> dict:
    """Back-to-back steps for `ms` of wall time (synchronising every 16), so
    the timed steps run at the GPU's steady clocks."""
    n = 0
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(16):
            step()
        n += 16
        torch.cuda.synchronize()
    return {"ms": round((time.perf_counter() - t0) * 1e3, 1), "steps": n}


def time_steps(step, args) -> tuple[float, dict]:
    """Settle, W warm-up steps, then the mean time of K steps (ms)."""
    st = settle(step, args.settle_ms) if args.settle_ms > 0 else {"ms": 0.0, "steps": 0}
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start, end = _events(2)
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / args.steps, st


def kernel_ms(launch, steps: int) -> float:
    """Mean duration of `launch` alone: HIP events on the launch stream
    (torch's current stream) around `steps` back-to-back launches."""
    launch()
    a, b = _events(2)
    a.record()
    for _ in range(steps):
        launch()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def _median_time(fn, reps: int = 3) -> float:
    fn()  # warm-up
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return statistics.median(times)


def recorded_traffic(name: str, config: dict):
    """HBM bytes per launch of the dominant kernel, as measured by the
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes recorded in profiles/<name>.md
    (line ``traffic_bytes_per_launch = N``, with the config it was taken on).
    None when no record matches this configuration."""
    path = os.path.join(ROOT, "profiles", name + ".md")
    if not os.path.exists(path):
        return None
    rec = {}
    keys = ("traffic_bytes_per_launch", *config)
    with open(path) as f:
        for line in f:
            m = re.fullmatch(r"\s*(\w+)\s*=\s*(\d+)\s*", line)
            if m and m.group(1) in keys:
                rec[m.group(1)] = int(m.group(2))
    if "traffic_bytes_per_launch" not in rec or any(rec.get(k) != v for k, v in config.items()):
        return None
    return rec["traffic_bytes_per_launch"]


def _record(args, *, value, unit, ms_step, dtype, data, config, roofline, cpu, settle_info, extra=None):
    res = {
        "metric": METRIC,
        "value": value,
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": data,
        "config": config,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "settle": dict(settle_info, why="steps run back to back before the warm-up so that the timed steps "
                                        "see steady GPU clocks (a power-management transient slows the first "
                                        "few ms of a heavy load)"),
    }
    if extra:
        res["extra"] = extra
    return res


# --------------------------------------------------------------- decode ---

def bench_decode(args, dev):
    """c3: fused decode attention at Llama-3-8B shape (headline)."""
    import smaq_amd as S
    from smaq_amd import _native
    from smaq_amd.batch import QuantizedKVBatch
    from smaq_amd.synthetic import sample_keys, sample_values

    B, N, Hq, Hkv, D, bits = args.batch, args.context, 32, 8, 128, 3
    calib = sample_keys(64, seed=3)
    strat = S.SMAQFullMetricScalarStrategy(D, bits=bits, device=dev).fit(calib)
    keys = sample_keys(B * N * Hkv, seed=11, device=dev, dtype=torch.bfloat16).view(B, N, Hkv, D)
    vals = sample_values(B * N * Hkv, seed=12, device=dev, dtype=torch.bfloat16).view(B, N, Hkv, D)
    strat.quantizer.tie_counter = _native.TieCounter(dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    kvb = QuantizedKVBatch.encode(strat, keys, vals, value_bits=2, value_group=32)
    torch.cuda.synchronize()
    encode_s = time.perf_counter() - t0
    ties = strat.quantizer.tie_counter.value()
    q = torch.randn(B, Hq, D, generator=torch.Generator(device=dev).manual_seed(13), device=dev).bfloat16()
    bytes_per_th = kvb.nbytes_per_token_head()
    algo_bytes = B * N * Hkv * bytes_per_th
    plan = kvb.plan(q)
    # timed region: K whole decode steps (query load + rotate, history
    # partials, split combine), no events inside
    ms_step, st = time_steps(lambda: plan.run(q), args)
    plan.load_query(q)
    plan.launch(phases=8)    # the query rotation, once: the timed launches are the decode kernel alone
    kern = kernel_ms(lambda: plan.launch(phases=1), args.steps)
    achieved = algo_bytes / (kern * 1e-3) / 1e9
    cpu = None if args.no_cpu_baseline else cpu_baseline_decode(strat, keys, vals, q, Hq, Hkv, D, bits)
    del keys, vals
    ring = bench_decode_ring(args, kvb, q, Hkv, D, algo_bytes)
    return _record(
        args, value=B / (ms_step * 1e-3), unit="tokens/s", ms_step=ms_step, dtype=DECODE_DTYPE,
        data="synthetic (seeded N(0, U diag(1/i) U^T) keys, N(0,1) values)",
        config={"workload": "c3 fused decode attention, Llama-3-8B shape", "batch": B, "context": N,
                "q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "key_bits": bits, "value_bits": 2,
                "value_group": 32, "storage_dtype": "bf16", "layout": "contiguous FlatCache"},
        roofline={"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                  "frac": achieved / HBM_PEAK_GBS,
                  "traffic": recorded_traffic("decode_mfma_c3", dict(batch=B, context=N)),
                  "kernel": "decode_mfma_kernel", "kernel_ms": kern,
                  "algorithmic_bytes": algo_bytes, "bytes_per_token_head": bytes_per_th},
        cpu=cpu, settle_info=st,
        extra={"encode_cache_s": encode_s, "encode_boundary_ties": ties,
               "hbm_gbs_whole_step": algo_bytes / (ms_step * 1e-3) / 1e9, "c3_ring128": ring})


def bench_decode_ring(args, kvb, q, Hkv, D, hist_bytes, R: int = 128):
    """c3 with the exact recent ring the vLLM adapter always serves beside
    the history (1..128 tokens; here full, 128 bf16 tokens per sequence): the
    history phase writes split partials, the recent phase adds one partial
    per (sequence, KV head), the combine merges them.  Same step definition
    as the headline; phases timed apart on the launch stream."""
    dev = q.device
    B = q.shape[0]
    g = torch.Generator(device=dev).manual_seed(14)
    rk = torch.randn(B, R, Hkv, D, generator=g, device=dev).bfloat16()
    rv = torch.randn(B, R, Hkv, D, generator=g, device=dev).bfloat16()
    plan = kvb.plan(q, recent_k=rk, recent_v=rv)
    ms_step, st = time_steps(lambda: plan.run(q), args)
    plan.load_query(q)
    phase = {name: kernel_ms(lambda m=m: plan.launch(phases=m), args.steps)
             for name, m in (("rotation_ms", 8), ("history_ms", 1), ("recent_ms", 2), ("combine_ms", 4))}
    byts = hist_bytes + B * R * Hkv * D * 2 * 2
    return {"value": B / (ms_step * 1e-3), "unit": "tokens/s", "ms_per_step": ms_step,
            "config": {"workload": "c3 + exact recent ring", "recent_tokens": R, "recent_dtype": "bf16"},
            "hbm_gbs_whole_step": byts / (ms_step * 1e-3) / 1e9, "algorithmic_bytes": byts,
            "phases": phase, "settle": st}


def cpu_baseline_decode(strat, keys, vals, q, Hq, Hkv, D, bits):
    """CPU oracle decoding one sequence of the batch: all KV heads, full
    context.  Encoding is not timed."""
    from oracle import smaq_ref as R
    qz = strat.quantizer
    codec = R.ScalarCodec(D, bits, E=qz.E.cpu(), E_inv=qz.E_inv.cpu())
    st = R.Store(codec, D, Hkv)
    st.append_chunk(keys[0].cpu(), vals[0].cpu())
    st.get_flat_cache()
    qc = q[0:1].cpu()
    t = _median_time(lambda: R.hybrid_attention(qc, st, None, None, Hq))
    return dict({"value": 1.0 / t, "unit": "tokens/s", "kind": "port",
                 "sample": f"1 of {keys.shape[0]} sequences (all {Hkv} KV heads, {keys.shape[1]} tokens), "
                           f"median of 3 after 1 warm-up; {t * 1e3:.1f} ms per sequence-step"}, **_cpu_fields())


# ---------------------------------------------------------------- paged ---

def bench_paged(args, dev):
    """c5: paged decode, 256 sequences with lengths U[1024, 16384] (seeded),
    block size 16, shuffled block tables, Student-t(3) keys with 3-bit scalar
    SMAQ, 2-bit values, 32 query / 8 KV heads, one decode token."""
    import smaq_amd as S
    from smaq_amd import _native
    from smaq_amd.batch import PagedQuantizedKV, _encode_rows
    from smaq_amd.synthetic import paged_lengths_and_table, sample_keys, student_t

    B, Hq, Hkv, D, bs = args.paged_seqs, 32, 8, 128, 16
    lens, table, total = paged_lengths_and_table(B, bs, seed=4)
    strat = S.SMAQFullMetricScalarStrategy(D, bits=3, device=dev).fit(sample_keys(64, seed=3))
    gd = torch.Generator(device=dev).manual_seed(41)
    kp = torch.empty(total, bs, Hkv, D, dtype=torch.bfloat16, device=dev)
    vp = torch.empty_like(kp)
    for i in range(0, total, 8192):
        j = min(total, i + 8192)
        kp[i:j] = student_t((j - i, bs, Hkv, D), gd, dev)
        vp[i:j] = torch.randn((j - i, bs, Hkv, D), generator=gd, device=dev).to(torch.bfloat16)
    strat.quantizer.tie_counter = _native.TieCounter(dev)
    codes, norms, vd, vsc, vz = _encode_rows(strat, kp.permute(0, 2, 1, 3), vp.permute(0, 2, 1, 3), 2, 32)
    del kp, vp
    pk = PagedQuantizedKV(strat, codes, norms, vd, vsc, vz, table.to(dev), lens.tolist(), bs, 2, 32)
    q = torch.randn(B, Hq, D, generator=torch.Generator(device=dev).manual_seed(43), device=dev).bfloat16()
    plan = pk.plan(q)
    token_heads = int(lens.sum()) * Hkv
    algo = token_heads * pk.nbytes_per_token_head()
    ms_step, st = time_steps(lambda: plan.run(q), args)
    plan.run(q)   # rotation and longest-first schedule, once: the timed launches are the decode kernel alone
    kern = kernel_ms(lambda: plan.launch(phases=1 | 16), args.steps)
    achieved = algo / (kern * 1e-3) / 1e9
    cpu = None if args.no_cpu_baseline else cpu_baseline_paged(strat, table, lens, bs, codes, norms, vd, vsc, vz,
                                                                  q, Hq, Hkv, D)
    adapter = bench_paged_adapter(args, strat, codes, norms, vd, vsc, vz, table, lens, total, q, plan, ms_step)
    return _record(
        args, value=B / (ms_step * 1e-3), unit="tokens/s", ms_step=ms_step, dtype=DECODE_DTYPE,
        data="synthetic (Student-t(3) keys, N(0,1) values, seeded lengths and block tables)",
        config={"workload": "c5 paged decode", "seqs": B, "block_size": bs, "q_heads": Hq, "kv_heads": Hkv,
                "head_dim": D, "key_bits": 3, "value_bits": 2, "value_group": 32, "storage_dtype": "bf16",
                "total_tokens": int(lens.sum()), "physical_blocks": total},
        roofline={"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                  "frac": achieved / HBM_PEAK_GBS,
                  "traffic": recorded_traffic("decode_mfma_paged_c5", dict(seqs=B, total_tokens=int(lens.sum()))),
                  "kernel": "decode_mfma_kernel (paged)", "kernel_ms": kern, "algorithmic_bytes": algo,
                  "bytes_per_token_head": pk.nbytes_per_token_head()},
        cpu=cpu, settle_info=st, extra={"encode_boundary_ties": strat.quantizer.tie_counter.value(),
                                         "adapter": adapter})


class _FlashImpl:
    """The attributes of a vLLM flash attention impl that the adapter's hooks
    read (vLLM is not installed); its own forward never runs in hybrid mode."""

    def __init__(self, num_heads, num_kv_heads, head_size):
        self.num_heads, self.num_kv_heads, self.head_size = num_heads, num_kv_heads, head_size
        self.scale = head_size ** -0.5

    def do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping):
        pass

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None, output_scale=None,
                output_block_scale=None):
        raise RuntimeError("the layer's own attention ran: the SMAQ paged decode did not serve the step")


def bench_paged_adapter(args, strat, codes, norms, vd, vsc, vz, table, lens, total, q, plan, ms_plan):
    """c5 through the vLLM adapter: hooks installed (paged, hybrid) on a
    one-layer runner whose layer pools are the workload's encoded pools, and
    each step is the hooked attention forward with vLLM's decode metadata
    (int32 seq_lens and block table, a [B, Hq * D] query, an output buffer):
    the adapter's cached plan, its length and table rebinding and the direct
    write into the output, against plan.run on the same pools."""
    from types import SimpleNamespace
    import smaq_amd.integration.vllm as V
    dev = q.device
    B, Hq, D = q.shape
    Hkv, bs = codes.shape[1], codes.shape[2]
    impl = _FlashImpl(Hq, Hkv, D)
    ctx = {"layer0": SimpleNamespace(impl=impl, num_heads=Hq)}
    runner = SimpleNamespace(compilation_config=SimpleNamespace(static_forward_context=ctx), device=dev,
                             kv_caches=[])
    state = V.install_hooks(runner, key_bits=3, initial_layers_count=0, mode=V.MODE_HYBRID, paged=True)["layer0"]
    state.store.key_strategy = strat
    state.store.quantizer = strat
    pc = state.paged
    pc.pools = {"k_codes": codes.view(-1, codes.shape[-1]), "k_norms": norms.view(-1),
                "v_data": vd.view(-1, vd.shape[-1]), "v_scales": vsc.view(-1, vsc.shape[-1]),
                "v_zeros": vz.view(-1, vz.shape[-1])}
    pc.num_blocks, pc.block_size = total, bs
    meta = SimpleNamespace(num_actual_tokens=B, max_query_len=1, seq_lens=lens.to(dev, torch.int32),
                           block_table=table.to(dev, torch.int32), max_seq_len=int(lens.max()))
    qf = q.reshape(B, Hq * D)
    out = torch.empty(B, Hq * D, dtype=q.dtype, device=dev)

    def step():
        impl.forward(None, qf, None, None, None, meta, output=out)

    ms_step, st = time_steps(step, args)
    want = plan.run(q).reshape(B, Hq * D)
    torch.cuda.synchronize()
    diff = (out.float() - want.float()).abs().max().item()
    return {"value": B / (ms_step * 1e-3), "unit": "tokens/s", "ms_per_step": ms_step,
            "vs_plan_run": ms_plan / ms_step, "max_abs_diff_vs_plan_run": diff,
            "plans_built": len(pc._plans), "settle": st,
            "path": "install_hooks(paged=True) + hooked impl.forward (PagedLayerCache.decode)"}


class _FlatStore:
    """The oracle Store interface (what its hybrid_attention reads) over a
    flat cache taken from the GPU pool, so that a CPU baseline times the
    oracle's attention without re-encoding the history on the host."""

    def __init__(self, flat, codec, head_dim, num_kv_heads, value_group_size=32):
        self.flat, self.codec = flat, codec
        self.head_dim, self.num_kv_heads, self.value_group_size = head_dim, num_kv_heads, value_group_size

    def get_flat_cache(self):
        return self.flat


def cpu_baseline_paged(strat, table, lens, bs, codes, norms, vd, vsc, vz, q, Hq, Hkv, D):
    """CPU oracle decoding the median-length sequence of the paged batch (all
    KV heads), its codes gathered from the GPU pool; scaled to the batch by
    total tokens / sample tokens (decode time is linear in the context)."""
    from oracle import smaq_ref as R
    b = int(torch.argsort(lens)[len(lens) // 2])
    L = int(lens[b])
    nb = (L + bs - 1) // bs
    blocks = table[b, :nb].long().to(codes.device)

    def gather(x):  # pool [blocks, Hkv, bs, ...] -> [Hkv, L, ...] on the host
        y = x[blocks].transpose(0, 1).reshape(Hkv, nb * bs, *x.shape[3:])[:, :L]
        return y.cpu().contiguous()

    qz = strat.quantizer
    codec = R.ScalarCodec(D, 3, E=qz.E.cpu(), E_inv=qz.E_inv.cpu())
    flat = R.FlatCache(R.ScalarQ(gather(codes), gather(norms), 3),
                       R.ValueQ(gather(vd), gather(vsc), gather(vz), 2), L)
    st = _FlatStore(flat, codec, D, Hkv)
    qc = q[b:b + 1].cpu()
    t = _median_time(lambda: R.hybrid_attention(qc, st, None, None, Hq))
    t_batch = t * float(lens.sum()) / L
    return dict({"value": len(lens) / t_batch, "unit": "tokens/s", "kind": "port",
                 "sample": f"sequence {b} ({L} tokens, the median length; all {Hkv} KV heads; codes from the GPU "
                           f"pool), median of 3 after 1 warm-up, {t * 1e3:.1f} ms; scaled to the batch by "
                           f"{int(lens.sum())} / {L} tokens"}, **_cpu_fields())


# -------------------------------------------------------------- prefill ---

def bench_prefill(args, dev):
    """c4: hybrid chunked prefill at Qwen2-7B shape: 28 query / 4 KV heads,
    2048 causal queries over 65408 block-VQ history tokens (block_dim 2, 256
    centroids = 4 bits/dim, 4 outlier channels x20) + 128 fp16 recent tokens,
    2-bit values."""
    import smaq_amd as S
    from smaq_amd.score import plan_hybrid_attention
    from smaq_amd.synthetic import sample_keys, sample_values

    Hq, Hkv, D = 28, 4, 128
    N, R, T = args.prefill_context - 128, 128, args.prefill_queries
    g = torch.Generator().manual_seed(3)
    outl = torch.randperm(D, generator=g)[:4]
    calib_k = sample_keys(4096, seed=31)
    calib_k[:, outl] *= 20
    calib_q = sample_keys(4096, seed=32)
    strat = S.SMAQBlockVQStrategy(D, block_dim=2, n_centroids=256, device=dev)
    strat.quantizer.fit(calib_k, calib_q, kmeans_iters=args.fit_iters)
    keys = sample_keys(N * Hkv, seed=33, device=dev, dtype=torch.float16).view(N, Hkv, D)
    keys[..., outl.to(dev)] *= 20
    vals = sample_values(N * Hkv, seed=34, device=dev, dtype=torch.float16).view(N, Hkv, D)
    st = S.CompressedKVStore(D, Hkv, device=dev, key_strategy=strat)
    st.append_chunk(keys, vals)
    kr = sample_keys(R * Hkv, seed=35, device=dev, dtype=torch.float16).view(R, Hkv, D)
    kr[..., outl.to(dev)] *= 20
    vr = sample_values(R * Hkv, seed=36, device=dev, dtype=torch.float16).view(R, Hkv, D)
    q = sample_keys(T * Hq, seed=37, device=dev, dtype=torch.float16).view(T, Hq, D)
    pos = torch.arange(N + R - T, N + R, device=dev)
    plan = plan_hybrid_attention(q, st, kr, vr, Hq, query_positions=pos)
    q1 = q.unsqueeze(0)
    ms, st_info = time_steps(lambda: plan.run(q1), args)
    # history phase alone (block-VQ keys -> f16 tile images, then the
    # matrix-core kernel), events on its launch stream
    plan.load_query(q1)
    plan.launch(phases=8)
    kern = kernel_ms(lambda: plan.launch(phases=1), args.steps)
    # QK + PV multiply-adds over the causal pairs, 2 flops each
    pairs = sum(min(int(p) + 1, N + R) for p in pos.tolist()) * Hq
    flops = pairs * D * 2 * 2
    hist_pairs = sum(min(int(p) + 1, N) for p in pos.tolist()) * Hq
    hist_flops = hist_pairs * D * 2 * 2
    byts = N * Hkv * (64 + 32 + 8 + 8) + R * Hkv * D * 2 * 2 + T * Hq * D * 2 * 2
    cpu = None if args.no_cpu_baseline else cpu_baseline_prefill(strat, st, kr, vr, q, pos, Hq, Hkv, D)
    achieved = hist_flops / (kern * 1e-3) / 1e12
    return _record(
        args, value=T / (ms * 1e-3), unit="tokens/s", ms_step=ms, dtype=PREFILL_DTYPE,
        data="synthetic (seeded keys with 4 outlier channels x20, N(0,1) values)",
        config={"workload": "c4 hybrid chunked prefill, Qwen2-7B shape", "q_heads": Hq, "kv_heads": Hkv,
                "head_dim": D, "queries": T, "history": N, "recent": R, "key_format": "block-VQ bd=2 nc=256",
                "value_bits": 2, "storage_dtype": "fp16", "causal": True},
        roofline={"bound": "mfma", "achieved": achieved, "peak": F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                  "frac": achieved / F16_PEAK_TFLOPS,
                  "traffic": recorded_traffic("prefill_mfma_c4", dict(history=N, queries=T)),
                  "kernel": "prefill_mfma_kernel (history phase, with decode_hist_planes_kernel)",
                  "kernel_ms": kern, "algorithmic_flops": hist_flops, "step_flops": flops,
                  "step_tflops": flops / (ms * 1e-3) / 1e12, "algorithmic_bytes": byts},
        cpu=cpu, settle_info=st_info)


def cpu_baseline_prefill(strat, st, kr, vr, q, pos, Hq, Hkv, D, n_q: int = 64):
    """CPU oracle for the last n_q query tokens of the chunk (full causal
    context: the block-VQ history from the GPU store plus the exact recent
    window)."""
    from oracle import smaq_ref as R
    qz = strat.quantizer
    codec = R.BlockVQCodec(qz.E_blocks.cpu(), qz.centroids.cpu(), qz.decoded_centroids.cpu())
    gf = st.get_flat_cache()
    flat = R.FlatCache(R.BlockQ(gf.key_q.indices.cpu(), gf.key_q.n_blocks, gf.key_q.block_dim),
                       R.ValueQ(gf.value_q.data.cpu(), gf.value_q.scales.cpu(), gf.value_q.zeros.cpu(),
                                gf.value_q.bits), gf.num_tokens)
    ost = _FlatStore(flat, codec, D, Hkv)
    qs, ps, krc, vrc = q[-n_q:].cpu(), pos[-n_q:].cpu(), kr.cpu(), vr.cpu()
    t = _median_time(lambda: R.hybrid_attention(qs, ost, krc, vrc, Hq, query_positions=ps))
    return dict({"value": n_q / t, "unit": "tokens/s", "kind": "port",
                 "sample": f"the last {n_q} of {q.shape[0]} query tokens over the full context "
                           f"({gf.num_tokens} history + {kr.shape[0]} recent), median of 3 after 1 warm-up, "
                           f"{t * 1e3:.1f} ms"}, **_cpu_fields())


# --------------------------------------------------------------- encode ---

def bench_encode(args, dev):
    """c2: block-VQ key encode + 2-bit value pack of [16 seq x 32768 tok x 8
    heads x 128] bf16 keys and values (4.19M token-heads), cache resident in
    HBM.  One step = encode every key (16 uint8 indices per token-head) and
    pack every value (32 B codes + 4 bf16 scales + 4 bf16 zeros).  The
    codebook is fitted untimed: k-means++ and Lloyd on the device by default
    (``--host-fit`` runs the reference's CPU fit instead, ~50 s)."""
    import smaq_amd as S
    from smaq_amd import _native
    from smaq_amd.kv_cache import quantize_values
    from smaq_amd.synthetic import sample_keys, sample_values

    seqs, toks, H, D = 16, args.encode_tokens, 8, 128
    rows = seqs * toks * H
    strat = S.SMAQBlockVQStrategy(D, block_dim=8, n_centroids=256, device=dev)
    calib_k = sample_keys(args.fit_samples, seed=21)
    calib_q = sample_keys(args.fit_samples, seed=22)
    t_fit = time.perf_counter()
    strat.quantizer.fit(calib_k, calib_q, kmeans_iters=args.fit_iters, on_device=not args.host_fit)
    torch.cuda.synchronize()
    t_fit = time.perf_counter() - t_fit
    keys = sample_keys(rows, seed=23, device=dev, dtype=torch.bfloat16).view(seqs, toks, H, D)
    vals = sample_values(rows, seed=24, device=dev, dtype=torch.bfloat16).view(seqs, toks, H, D)
    strat.quantizer.tie_counter = _native.TieCounter(dev)

    def step():
        strat.quantize(keys)
        quantize_values(vals, bits=2, group_size=32)

    ms_step, st = time_steps(step, args)
    k_ms = kernel_ms(lambda: strat.quantize(keys), args.steps)
    v_ms = kernel_ms(lambda: quantize_values(vals, bits=2, group_size=32), args.steps)
    bytes_per_th = 2 * D * 2 + 16 + 32 + 16      # K + V in; indices, codes, scales/zeros out
    algo = rows * bytes_per_th
    # per token-block: the 8 x 8 metric rotation and the 256-centroid x 8-dim
    # distance contraction, 2 flops per multiply-add
    flops = rows * 16 * (8 * 8 + 256 * 8) * 2
    ties = strat.quantizer.tie_counter.value()
    cpu = None if args.no_cpu_baseline else cpu_baseline_encode(strat, keys, vals)
    del keys, vals
    fit_how = "host (the reference's CPU draw)" if args.host_fit else "device"
    return _record(
        args, value=algo / (ms_step * 1e-3) / 1e9, unit="GB/s", ms_step=ms_step, dtype=ENCODE_DTYPE,
        data="synthetic (seeded N(0, U diag(1/i) U^T) keys, N(0,1) values)",
        config={"workload": "c2 block-VQ key encode + 2-bit value pack", "seqs": seqs, "tokens": toks,
                "kv_heads": H, "head_dim": D, "block_dim": 8, "n_centroids": 256, "storage_dtype": "bf16",
                "codebook_fit": f"k-means++ on {args.fit_samples} samples, {args.fit_iters} Lloyd iterations "
                                f"({fit_how}, {t_fit:.1f} s, untimed)"},
        # the fp32-accurate rotation + distance contraction (algorithmic_flops)
        # against the FP32 matrix peak; the kernel issues the distances as
        # f16 hi/lo products (one 16x16x32 f16 MFMA per 16 centroids x 16
        # tokens), and its limiter is VALU issue for the argmin
        roofline={"bound": "mfma", "kernel": "encode_blockvq_mfma_kernel", "kernel_ms": k_ms,
                  "achieved": flops / (k_ms * 1e-3) / 1e12, "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                  "frac": flops / (k_ms * 1e-3) / 1e12 / FP32_PEAK_TFLOPS,
                  "traffic": recorded_traffic("encode_blockvq_c2", dict(rows=rows)), "pack_values_ms": v_ms,
                  "hbm_gbs": algo / ((k_ms + v_ms) * 1e-3) / 1e9, "algorithmic_bytes": algo,
                  "algorithmic_flops": flops,
                  # 16 blocks x 16 MFMAs (16 x 16 x 32 x 2 flop) per 16 tokens
                  "issued_f16_tflops": rows * 16 * 16 * (16 * 16 * 32 * 2) / 16 / (k_ms * 1e-3) / 1e12,
                  "f16_peak": F16_PEAK_TFLOPS},
        cpu=cpu, settle_info=st, extra={"boundary_ties": ties})


def cpu_baseline_encode(strat, keys, vals, n: int = 2048):
    """CPU oracle encoding n token-heads (block-VQ keys + value pack)."""
    from oracle import smaq_ref as R
    qz = strat.quantizer
    kc = keys.reshape(-1, keys.shape[-1])[:n].cpu()
    vc = vals.reshape(-1, vals.shape[-1])[:n].cpu()
    Eb, C = qz.E_blocks.cpu(), qz.centroids.cpu()
    t = _median_time(lambda: (R.blockvq_encode(kc, Eb, C), R.quantize_values(vc, bits=2, group_size=32)))
    return dict({"value": n * (2 * 256 + 64) / t / 1e9, "unit": "GB/s", "kind": "port",
                 "sample": f"{n} token-heads, median of 3 after 1 warm-up ({t * 1e3:.1f} ms)"}, **_cpu_fields())


# ---------------------------------------------------------- HBM ceiling ---

def copy_ceiling(dev, nbytes: int = 1 << 30, reps: int = 20):
    """The practical HBM ceilings next to the 8 TB/s peak: a plain streaming
    read of nbytes (smaq_probe_read, 16-byte non-temporal loads; the
    read-bound kernels' ceiling) and a device-to-device copy (read + write
    bytes / time; also the counter-calibration kernel), each the mean of
    `reps` back-to-back launches between HIP events on the launch stream."""
    from smaq_amd import _native
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    ms = kernel_ms(lambda: dst.copy_(src), reps)
    rms = kernel_ms(lambda: _native.probe_read(src, sink), reps)
    del src, dst
    return {"copy_bytes": nbytes, "copy_ms": ms, "copy_gbs": 2 * nbytes / (ms * 1e-3) / 1e9,
            "read_ms": rms, "read_gbs": nbytes / (rms * 1e-3) / 1e9, "read_kernel": "smaq_probe_read"}


def _summary(rec: dict) -> dict:
    """A workload's record without the fields the headline line already has."""
    keep = ("value", "unit", "ms_per_step", "dtype", "data", "config", "roofline", "cpu_baseline", "settle", "extra")
    return {k: rec[k] for k in keep if k in rec}


# --------------------------------------------------------------- main ---

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--settle-ms", type=float, default=300.0,
                    help="back-to-back steps before the warm-up (ms of wall time; 0 = none)")
    ap.add_argument("--workload", default="all", choices=["all", "decode", "encode", "paged", "prefill"])
    ap.add_argument("--prefill-context", type=int, default=65536, help="c4 context (history + 128 recent)")
    ap.add_argument("--prefill-queries", type=int, default=2048, help="c4 causal query tokens")
    ap.add_argument("--paged-seqs", type=int, default=256, help="c5 sequences")
    ap.add_argument("--encode-tokens", type=int, default=32768, help="c2 tokens per sequence")
    ap.add_argument("--fit-samples", type=int, default=65536, help="c2 codebook calibration samples")
    ap.add_argument("--fit-iters", type=int, default=20, help="c2/c4 Lloyd iterations")
    ap.add_argument("--host-fit", action="store_true", help="c2: fit the codebook on the host CPU")
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--context", type=int, default=32768)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a 1 GiB device copy (HBM ceiling and counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(the hot path would shard by sequence / KV head, each GPU attending over its own "
              "sequences and heads with no exchange). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    torch.set_num_threads(cpu_threads())
    dev = torch.device("cuda:0")
    if args.copy_probe:
        print(json.dumps(copy_ceiling(dev)), flush=True)
        return
    one = {"decode": bench_decode, "encode": bench_encode, "paged": bench_paged, "prefill": bench_prefill}
    if args.workload != "all":
        print(json.dumps(one[args.workload](args, dev)), flush=True)
        return
    res = bench_decode(args, dev)
    print(f"# c3 decode: {res['value']:.0f} tokens/s, kernel {res['roofline']['kernel_ms'] * 1e3:.1f} us",
          file=sys.stderr, flush=True)
    torch.cuda.empty_cache()
    extra = res.setdefault("extra", {})
    for name, fn in (("c5_paged_decode", bench_paged), ("c4_prefill", bench_prefill), ("c2_encode", bench_encode)):
        rec = fn(args, dev)
        extra[name] = _summary(rec)
        print(f"# {name}: {rec['value']:.4g} {rec['unit']}", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
    extra["hbm_ceiling"] = copy_ceiling(dev)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
