"""Benchmark of the OSCAR INT2 KV-cache hot path on one MI355X.

Headline (BASELINE metric): 4-token MTP decode attention over a 24,579-token
INT2 history (Hq=6, Hk=1, D=256, 193 shuffled 128-token pages, FP32
sink/recent window) in microseconds per layer and achieved HBM GB/s, plus the
quantize-write GB/s of a 65,536-token bulk write (random slots, ~1/16
skipped).

A step is one layer's decode attention.  Steps cycle through `--layers`
distinct per-layer caches (64 x ~13 MB, beyond the 256 MB Infinity Cache) so
reads come from HBM.  The launches are captured once in a HIP graph and the
graph is replayed; HIP events on the launch stream bracket exactly `--steps`
layer decodes.  Inputs are resident in HBM before timing starts.

cpu_baseline: the CPU oracle's read path (history dequant + window splice +
causal SDPA, oracle/attention.py) on the same C2 inputs, timed on this host.

Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "MTP decode attn µs/layer + HBM GB/s at 24K INT2 history; quant-write GB/s"
HBM_PEAK_GBPS = 8000.0
C2_HISTORY, C2_QLEN, HQ, HK, D, BS = 24579, 4, 6, 1, 256, 128


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def c2_case(seed=93):
    from tests.scenarios import decode_case

    return decode_case([C2_HISTORY], [C2_QLEN], hq=HQ, hk=HK, bs=BS, seed=seed)


def decode_bytes(case) -> dict:
    """Algorithmic HBM bytes of one C2 layer decode."""
    L = case.layer
    owner = L.arena.owner if L.arena is not None else None
    hist = case.seqs[0] - C2_QLEN
    staged = 0
    if owner is not None:
        pos = list(range(hist))
        pages = case.bt[0][[p // BS for p in pos]].long()
        rows = pages % owner.shape[0]
        staged = int((owner[rows, [p % BS for p in pos]] == pages).sum())
    int2 = (hist - staged) * HK * 136
    window = staged * HK * 2 * D * 4
    owner_tbl = owner.numel() * 8 if owner is not None else 0
    qkv = C2_QLEN * HQ * D * 4 + C2_QLEN * HK * 2 * D * 4
    out = C2_QLEN * HQ * D * 4
    bt = case.bt.numel() * 4
    total = int2 + window + owner_tbl + qkv + out + bt
    return {"total": total, "int2": int2, "window": window, "staged_tokens": staged,
            "int2_160B_variant": (hist - staged) * HK * 160 + window + owner_tbl + qkv + out + bt}


def bench_decode(args, dev):
    import torch

    from oscar_amd.kernels import decode

    case = c2_case()
    L = case.layer
    q, k, v = case.rotated()
    nbytes = decode_bytes(case)
    plans = []
    stage = L.stage()
    for _ in range(args.layers):
        kc, vc = L.k_cache.to(dev), L.v_cache.to(dev)
        st = tuple(t.to(dev) for t in stage)
        plans.append(decode.plan(q.to(dev), k.to(dev), v.to(dev), kc, vc, case.bt.to(dev),
                                 case.qsl, case.seqs, L.scale, st))
    torch.cuda.synchronize()
    # Correctness gate on layer 0 before timing.
    from oracle import attention as oatt

    want = oatt.paged_attention_ref(q, k, v, L.k_cache, L.v_cache, case.bt, case.qsl, case.seqs,
                                    L.scale, stage)
    got = plans[0].launch().cpu()
    err = (got - want).abs().max().item() / want.abs().max().item()
    if not err <= 1e-3:
        raise SystemExit(f"decode parity gate failed: rel err {err:.3e}")

    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for p in plans:
            p.launch()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for p in plans:
            p.launch()
    reps_w = max(1, args.warmup // args.layers)
    reps = max(1, args.steps // args.layers)
    for _ in range(reps_w):
        graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        graph.replay()
    e1.record(stream)
    e1.synchronize()
    steps = reps * args.layers
    ms = e0.elapsed_time(e1)
    us_per_layer = ms * 1000.0 / steps
    gbps = nbytes["total"] / (us_per_layer * 1e-6) / 1e9
    return {"us_per_layer": us_per_layer, "steps": steps, "ms": ms, "gbps": gbps, "bytes": nbytes,
            "parity_rel_err": err, "case": case}


def bench_quant_write(args, dev):
    import torch

    from oscar_amd import synthetic
    from oscar_amd.kernels import _lib, quant

    N = 65536
    pages = N // BS + 32
    sets = 4
    g = torch.Generator().manual_seed(55)
    Rk, Rv = synthetic.rotations(D, seed=56)
    ops = [quant.rotation_operand(R.to(dev)) for R in (Rk, Rv)]
    launches = []
    keep = []
    valid_total = 0
    for s in range(sets):
        k, v = synthetic.kv(N, HK, D, seed=100 + s)
        slots = torch.randperm(pages * BS, generator=g)[:N].to(torch.int64)
        slots[torch.rand(N, generator=g) < 1 / 16] = -1
        valid_total += int((slots >= 0).sum())
        kd, vd, sd = k.to(dev), v.to(dev), slots.to(dev)
        kc = torch.zeros(pages, BS, HK, D, dtype=torch.int8, device=dev)
        vc = torch.zeros_like(kc)
        keep += [kd, vd, sd, kc, vc]
        bs, npages, kst, vst = quant.cache_geometry(kc, vc)
        launches.append((_lib.ptr(kd), _lib.ptr(vd), N, HK, D, HK * D, _lib.ptr(ops[0]), _lib.ptr(ops[1]),
                         _lib.ptr(sd), _lib.ptr(kc), _lib.ptr(vc), bs, npages, *kst, *vst, 245, 235))
    valid = valid_total / sets
    nbytes = N * HK * 2 * D * 2 + valid * HK * 136 + N * 8 + 2 * D * D * 4
    stream = torch.cuda.current_stream(dev)
    h = stream.cuda_stream
    for i in range(8):
        _lib.call("oscar_quant_write", *launches[i % sets], h)
    torch.cuda.synchronize()
    iters = max(8, args.qw_iters)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(iters):
        _lib.call("oscar_quant_write", *launches[i % sets], h)
    e1.record(stream)
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / iters
    return {"us_per_call": us, "gbps": nbytes / (us * 1e-6) / 1e9, "bytes": nbytes, "tokens": N,
            "valid_slots": valid}


def cpu_baseline(case, seconds: float):
    import torch

    from oracle import attention as oatt

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    L = case.layer
    q, k, v = case.rotated()
    stage = L.stage()

    def once():
        oatt.paged_attention_ref(q, k, v, L.k_cache, L.v_cache, case.bt, case.qsl, case.seqs, L.scale, stage)

    once()
    samples = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(samples) < 6:
        t0 = time.perf_counter()
        once()
        samples.append(time.perf_counter() - t0)
    med = statistics.median(samples)
    try:
        model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except Exception:
        model = "unknown"
    return {"value": med * 1e6, "unit": "us/layer", "cores": cores, "kind": "port",
            "sample": f"median of {len(samples)} runs of the oracle C2 read path "
                      f"(dequant 24579-token INT2 history + FP32 window splice + causal SDPA, "
                      f"4 queries x 6 heads); host CPU {model}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=640)
    ap.add_argument("--warmup", type=int, default=128)
    ap.add_argument("--layers", type=int, default=64)
    ap.add_argument("--qw-iters", type=int, default=64)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (one TP rank's share "
              "per GPU, no collectives); run with --gpus 1", file=sys.stderr)
        raise SystemExit(2)
    import torch

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    dev = torch.device("cuda:0")
    log("bench: decode C2")
    dec = bench_decode(args, dev)
    log(f"bench: decode {dec['us_per_layer']:.3f} us/layer; quant-write C5")
    qw = bench_quant_write(args, dev)
    log(f"bench: quant-write {qw['gbps']:.1f} GB/s")
    cpu = None
    if not args.no_cpu_baseline:
        log("bench: cpu baseline")
        cpu = cpu_baseline(dec["case"], args.cpu_seconds)
    line = {
        "metric": METRIC,
        "value": round(dec["us_per_layer"], 4),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": dec["steps"],
        "warmup": max(1, args.warmup // args.layers) * args.layers,
        "ms_per_step": dec["us_per_layer"] / 1000.0,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": "C2: MTP decode, 1 request x 4 query tokens, Hq=6 Hk=1 D=256, 24579-token INT2 "
                        "history in 193 shuffled 128-token pages, FP32 sink=128/recent=256 window "
                        "(staging 8192), clip 0.96/0.92, int8-geometry caches, 64 distinct layers",
            "arith": "INT2 dequant to f16, f16 MFMA with f32 accumulation, f32 online softmax",
            "decode_hbm_gbps": round(dec["gbps"], 1),
            "decode_bytes_per_layer": dec["bytes"]["total"],
            "decode_bytes_per_layer_160B_variant": dec["bytes"]["int2_160B_variant"],
            "staged_tokens": dec["bytes"]["staged_tokens"],
            "decode_parity_rel_err": dec["parity_rel_err"],
            "quant_write": {"workload": "C5 write: 65536 tokens bf16, Hk=1, random slots ~1/16 skipped, "
                                        "rotation on MFMA, clip 0.96/0.92",
                            "us_per_call": round(qw["us_per_call"], 3), "gbps": round(qw["gbps"], 1),
                            "frac_of_hbm_peak": round(qw["gbps"] / HBM_PEAK_GBPS, 4),
                            "bytes_per_call": qw["bytes"]},
        },
        "roofline": {"bound": "hbm", "achieved": round(dec["gbps"], 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(dec["gbps"] / HBM_PEAK_GBPS, 4), "traffic": None},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
