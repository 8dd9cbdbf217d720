#!/usr/bin/env python
"""SMAQ quantized-KV hot path benchmark on one MI355X.

Default workload: fused quantized-KV decode attention at
Llama-3-8B shape -- batch 32, context 32768, 32 query / 8 KV heads, head_dim
128, keys 3-bit scalar SMAQ (calibrated metric), values 2-bit (group 32),
bf16 queries, one new token per sequence.  One step = one decode-attention
pass of one layer over the whole batch, cache resident in HBM.

    python bench.py [--steps K] [--warmup W] [--workload decode|encode|paged]

Prints ONE JSON line.  ``value`` is decode tokens/s (batch / step time);
``roofline`` is the dominant kernel (decode_mfma_kernel, history partials) timed with HIP
events on the launch stream, against its algorithmic bytes (114 B per
token-head); ``cpu_baseline`` times the CPU oracle on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "quantized-KV decode attn tokens/s + achieved HBM GB/s (% peak); encode GB/s"
HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3


def _events(n):
    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def _cores() -> int:
    return torch.get_num_threads()


# --------------------------------------------------------------- decode ---

def bench_decode(args, dev):
    import smaq_amd as S
    from smaq_amd.batch import QuantizedKVBatch
    from smaq_amd.synthetic import sample_keys, sample_values

    B, N, Hq, Hkv, D, bits = args.batch, args.context, 32, 8, 128, 3
    calib = sample_keys(64, seed=3)
    strat = S.SMAQFullMetricScalarStrategy(D, bits=bits, device=dev).fit(calib)
    keys = sample_keys(B * N * Hkv, seed=11, device=dev, dtype=torch.bfloat16).view(B, N, Hkv, D)
    vals = sample_values(B * N * Hkv, seed=12, device=dev, dtype=torch.bfloat16).view(B, N, Hkv, D)
    from smaq_amd import _native
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

    for _ in range(args.warmup):
        plan.run(q)
    torch.cuda.synchronize()
    # timed region: K whole decode steps (query load + rotate, history
    # partials, split combine), no events inside
    start, end = _events(2)
    start.record()
    for _ in range(args.steps):
        plan.run(q)
    end.record()
    torch.cuda.synchronize()
    ms_step = start.elapsed_time(end) / args.steps
    # dominant kernel: HIP events on its launch stream (torch's current
    # stream, which the plan launches on) around the history phase alone
    ea, eb = _events(args.steps), _events(args.steps)
    for i in range(args.steps):
        plan.load_query(q)
        ea[i].record()
        plan.launch(phases=1)
        eb[i].record()
        plan.launch(phases=4)
    torch.cuda.synchronize()
    kern_ms = statistics.mean(a.elapsed_time(b) for a, b in zip(ea, eb))
    achieved = algo_bytes / (kern_ms * 1e-3) / 1e9
    traffic = recorded_traffic("decode_mfma_c3", dict(batch=B, context=N))

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_decode(strat, keys, vals, q, Hq, Hkv, D, bits)
    res = {
        "metric": METRIC,
        "value": B / (ms_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0, U diag(1/i) U^T) keys, N(0,1) values)",
        "config": {"workload": "c3 fused decode attention, Llama-3-8B shape", "batch": B, "context": N,
                   "q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "key_bits": bits, "value_bits": 2,
                   "value_group": 32, "storage_dtype": "bf16", "layout": "contiguous FlatCache"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "kernel": "decode_mfma_kernel", "kernel_ms": kern_ms,
                     "algorithmic_bytes": algo_bytes, "bytes_per_token_head": bytes_per_th},
        "cpu_baseline": cpu,
        "extra": {"encode_cache_s": encode_s, "encode_boundary_ties": ties,
                  "hbm_gbs_whole_step": algo_bytes / (ms_step * 1e-3) / 1e9},
    }
    return res


def cpu_baseline_decode(strat, keys, vals, q, Hq, Hkv, D, bits):
    """CPU oracle (op-for-op torch restatement of the reference) decoding one
    sequence of the batch: all KV heads, full context.  Encoding is not timed."""
    from oracle import smaq_ref as R
    qz = strat.quantizer
    codec = R.ScalarCodec(D, bits, E=qz.E.cpu(), E_inv=qz.E_inv.cpu())
    st = R.Store(codec, D, Hkv)
    st.append_chunk(keys[0].cpu(), vals[0].cpu())
    st.get_flat_cache()
    qc = q[0:1].cpu()
    R.hybrid_attention(qc, st, None, None, Hq)          # warm-up
    times = []
    for _ in range(3):
        t = time.perf_counter()
        R.hybrid_attention(qc, st, None, None, Hq)
        times.append(time.perf_counter() - t)
    t = statistics.median(times)
    return {"value": 1.0 / t, "unit": "tokens/s", "cores": _cores(), "kind": "port",
            "sample": f"1 of {keys.shape[0]} sequences (all {Hkv} KV heads, {keys.shape[1]} tokens), "
                      f"median of 3 after 1 warm-up; {t * 1e3:.1f} ms per sequence-step"}


def recorded_traffic(name: str, config: dict):
    """HBM bytes per launch of the dominant kernel, as measured by the
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes recorded in profiles/<name>.md
    (line ``traffic_bytes_per_launch = N``, with the config it was taken on).
    None when no record matches this configuration."""
    path = os.path.join(ROOT, "profiles", name + ".md")
    if not os.path.exists(path):
        return None
    rec = {}
    with open(path) as f:
        for line in f:
            if "=" in line and line.strip().startswith(("traffic_bytes_per_launch", "batch", "context")):
                k, v = line.split("=", 1)
                rec[k.strip()] = int(v.strip())
    if "traffic_bytes_per_launch" not in rec or any(rec.get(k) != v for k, v in config.items()):
        return None
    return rec["traffic_bytes_per_launch"]


def copy_ceiling(dev, nbytes: int = 1 << 30, reps: int = 10):
    """Device-to-device copy of nbytes: the practical HBM ceiling (read +
    write bytes / time) and the reference kernel for counter calibration."""
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    a, b = _events(2)
    a.record()
    for _ in range(reps):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    # read-only ceiling: a full reduction over the same bytes as fp32
    xf = src.view(torch.float32)
    for _ in range(2):
        xf.sum()
    torch.cuda.synchronize()
    a.record()
    for _ in range(reps):
        xf.sum()
    b.record()
    torch.cuda.synchronize()
    rms = a.elapsed_time(b) / reps
    return {"copy_bytes": nbytes, "copy_ms": ms, "copy_gbs": 2 * nbytes / (ms * 1e-3) / 1e9,
            "read_ms": rms, "read_gbs": nbytes / (rms * 1e-3) / 1e9}


# --------------------------------------------------------------- main ---

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="decode", choices=["decode"])
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--context", type=int, default=32768)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a 1 GiB device copy (HBM ceiling and counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(the hot path shards by sequence/KV head with no exchange; see DESIGN.md). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    if args.copy_probe:
        print(json.dumps(copy_ceiling(dev)), flush=True)
        return
    res = bench_decode(args, dev)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
