"""Benchmark of the OSCAR INT2 KV-cache hot path on one MI355X.

Headline metric: 4-token MTP decode attention over a 24,579-token
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


class LayerState:
    """One FULL layer's state right before its decode read, written on the GPU
    by the product write path (fused quantize-write + window-write kernels)."""

    def __init__(self, impl, layer, caches, bt, qsl, seqs, q_rot, k_rot, v_rot):
        self.impl, self.layer, self.caches, self.bt = impl, layer, caches, bt
        self.qsl, self.seqs = qsl, seqs
        self.q_rot, self.k_rot, self.v_rot = q_rot, k_rot, v_rot

    def stage(self):
        return self.impl._stage(self.layer)


def make_impl(dev, window=True):
    from oscar_amd.backend import OscarAttentionBackendImpl

    impl = OscarAttentionBackendImpl.__new__(OscarAttentionBackendImpl)
    impl.head_size, impl.num_kv_heads, impl.num_heads = D, HK, HQ
    impl.scale = D ** -0.5
    impl.key_cache = impl.value_cache = None
    import contextlib
    import io

    with contextlib.redirect_stdout(io.StringIO()):
        impl._oscar_setup()
    cfg = impl._oscar
    cfg.k_clip_ratio, cfg.v_clip_ratio = 0.96, 0.92
    cfg.sink_tokens, cfg.recent_tokens, cfg.staging_tokens = 128, 256, 8192
    cfg.window_enabled = window
    return impl


def build_layer(dev, history: list, q_len: int, pool: int, seed: int, window=True) -> LayerState:
    """Prefill-write every request's history, then write the MTP step's tokens."""
    from types import SimpleNamespace as NS

    import torch

    from oscar_amd import synthetic

    impl = make_impl(dev, window)
    Rk, Rv = synthetic.rotations(D, seed)
    layer = NS(layer_name="model.layers.0.self_attn.attn", _oscar_rots=(Rk.to(dev), Rv.to(dev)))
    caches = [torch.zeros(pool, BS, HK, D, dtype=torch.int8, device=dev) for _ in range(2)]
    B = len(history)
    need = [(h + q_len + BS - 1) // BS for h in history]
    perm = synthetic.page_permutation(pool, seed + 1)
    T = max(need)
    bt = torch.zeros(B, T, dtype=torch.int32)
    off = 0
    for i, n in enumerate(need):
        bt[i, :n] = perm[off:off + n]
        off += n

    def write(counts, starts, seqs, kseed):
        n = sum(counts)
        k, v = synthetic.kv(n, HK, D, seed=kseed)
        slots = torch.cat([synthetic.slots_for(bt[i], st, c, BS) for i, (st, c) in enumerate(zip(starts, counts))])
        qsl = [0]
        for c in counts:
            qsl.append(qsl[-1] + c)
        md = NS(num_actual_tokens=n, slot_mapping=slots.to(dev), query_start_loc_cpu=torch.tensor(qsl),
                seq_lens_list=list(seqs), block_tables=bt.to(dev))
        kd, vd = k.to(dev), v.to(dev)
        impl.do_kv_cache_update(layer, kd, vd, caches, md.slot_mapping)
        if window:
            impl._ensure_staging(layer, caches)
            impl._staging_write(layer, kd, vd, md)
        return kd, vd, qsl

    write(history, [0] * B, history, seed + 2)
    seqs = [h + q_len for h in history]
    kd, vd, qsl = write([q_len] * B, history, seqs, seed + 3)
    q = synthetic.queries(q_len * B, HQ, D, seed=seed + 4).to(dev)
    rk, rv = layer._oscar_rots
    torch.cuda.synchronize()
    return LayerState(impl, layer, caches, bt.to(dev), qsl, seqs, q.float() @ rk, kd.float() @ rk,
                      vd.float() @ rv)


def clone_layer(st: LayerState) -> LayerState:
    from types import SimpleNamespace as NS

    layer = NS(**vars(st.layer))
    for name in ("_oscar_stage_k", "_oscar_stage_v", "_oscar_slot_owner", "_oscar_seat_winner",
                 "_oscar_stage_kimg", "_oscar_stage_vimg"):
        if getattr(st.layer, name, None) is not None:
            setattr(layer, name, getattr(st.layer, name).clone())
    return LayerState(st.impl, layer, [c.clone() for c in st.caches], st.bt, st.qsl, st.seqs,
                      st.q_rot, st.k_rot, st.v_rot)


def decode_bytes(st: LayerState) -> dict:
    """Algorithmic HBM bytes of one layer decode: every history token's INT2
    slot bytes (8 meta + 64 K + 64 V codes), the staged fp32 K/V of tokens the
    window owns, the owner table, q / new k / new v / out in fp32 and the
    block-table entries."""
    import torch

    owner = st.stage()[2].cpu() if st.stage() is not None else None
    bt = st.bt.cpu()
    n_q = st.q_rot.shape[0]
    hist_tokens = window = staged = 0
    for i, (a, b) in enumerate(zip(st.qsl, st.qsl[1:])):
        hist = st.seqs[i] - (b - a)
        pos = torch.arange(hist)
        pages = bt[i][pos // BS].long()
        s_i = 0
        if owner is not None:
            s_i = int((owner[pages % owner.shape[0], pos % BS] == pages).sum())
        staged += s_i
        hist_tokens += hist
        window += s_i * HK * 2 * D * 4
    int2 = hist_tokens * HK * 136
    owner_tbl = owner.numel() * 8 if owner is not None else 0
    qkv = n_q * HQ * D * 4 + n_q * HK * 2 * D * 4
    out = n_q * HQ * D * 4
    bt_bytes = sum((s + BS - 1) // BS for s in st.seqs) * 4
    fixed = window + owner_tbl + qkv + out + bt_bytes
    return {"total": int2 + fixed, "int2": int2, "window": window, "staged_tokens": staged,
            "int2_160B_variant": hist_tokens * HK * 160 + fixed}


def decode_only_bytes(st: LayerState) -> dict:
    """Algorithmic HBM bytes of one DecodeOnly read: every history position's
    INT2 slot bytes, the staged fp32 K/V of the positions the windowed read
    takes from the arena (the sink when all of its seats hold it, the staged
    run ending at the last position inside the recent window), the owner
    entries of the sink and tail pages, q and out in fp32, block-table entries."""
    import torch

    stage = st.stage()
    bt = st.bt.cpu()
    cfg = st.impl._oscar
    n_q = st.q_rot.shape[0]
    used = hist_tokens = owner_entries = 0
    for i, seq in enumerate(st.seqs):
        hist_tokens += seq
        if stage is None:
            continue
        owner = stage[2].cpu()
        pos = torch.arange(seq)
        pages = bt[i][pos // BS].long()
        staged = owner[pages % owner.shape[0], pos % BS] == pages
        sink = (cfg.sink_tokens // BS) * BS
        head = sink if 0 < sink < seq and bool(staged[:sink].all()) else 0
        t0 = max(seq - cfg.recent_tokens, head)
        cut = seq
        while cut > t0 and bool(staged[cut - 1]):
            cut -= 1
        used += head + (seq - cut)
        owner_entries += head + (seq - t0)
    int2 = hist_tokens * HK * 136
    fixed = used * HK * 2 * D * 4 + owner_entries * 8 + 2 * n_q * HQ * D * 4 + \
        sum((s + BS - 1) // BS for s in st.seqs) * 4
    return {"total": int2 + fixed, "int2": int2, "window": used * HK * 2 * D * 4, "staged_tokens": used,
            "int2_160B_variant": hist_tokens * HK * 160 + fixed}


def bench_decode(args, dev, history, q_len, pool, layers, seed=93, decode_only=False):
    import torch

    from oscar_amd.kernels import decode

    base = build_layer(dev, history, q_len, pool, seed, window=bool(args.window))
    nbytes = decode_only_bytes(base) if decode_only else decode_bytes(base)
    states = [base] + [clone_layer(base) for _ in range(layers - 1)]
    if decode_only:
        cfg = base.impl._oscar
        plans = [decode.decode_only_plan(st.q_rot, st.caches[0], st.caches[1], st.bt, st.seqs, st.impl.scale,
                                         st.stage(), cfg.sink_tokens, cfg.recent_tokens, tiles_per_split=args.tps)
                 for st in states]
    else:
        plans = [decode.plan(st.q_rot, st.k_rot, st.v_rot, st.caches[0], st.caches[1], st.bt, st.qsl,
                             st.seqs, st.impl.scale, st.stage(), tiles_per_split=args.tps) for st in states]
    torch.cuda.synchronize()
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
    reps_w = max(1, args.warmup // layers)
    reps = max(1, args.steps // layers)
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
    steps = reps * layers
    ms = e0.elapsed_time(e1)
    us = ms * 1000.0 / steps
    out0 = plans[0].launch().clone()
    torch.cuda.synchronize()
    return {"us_per_layer": us, "steps": steps, "ms": ms, "gbps": nbytes["total"] / (us * 1e-6) / 1e9,
            "bytes": nbytes, "state": base, "out0": out0, "warmup": reps_w * layers}


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


def copy_probe(dev, mib: int) -> None:
    """A plain device-to-device copy of known size (reads and writes `mib` MiB
    per launch), the reference point for scaling PMC byte counters."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"bench: copy probe {mib} MiB x 4")


def traffic_from_profile(kernel_src: Path):
    """HBM bytes per decode call from the committed PMC summary, if it was
    measured on the current kernel source (sha256 recorded in the summary)."""
    import hashlib

    prof = ROOT / "profiles" / "decode_c2_traffic.txt"
    if not prof.exists():
        return None
    fields = dict(l.split(":", 1) for l in prof.read_text().splitlines() if ":" in l and not l.startswith(" "))
    digest = hashlib.sha256(kernel_src.read_bytes()).hexdigest()
    if fields.get("source_sha256", "").strip() != digest:
        return None
    try:
        return int(fields["traffic_bytes_per_call"].strip())
    except (KeyError, ValueError):
        return None


def decode_only_cpu_baseline(st, gpu_out, seconds: float):
    """The oracle's DecodeOnly read (INT2 middle + FP32 sink/tail, LSE merge) on
    the same GPU-written state, on this host, and the parity of the timed kernel
    against it (fp32 contract for this read: 2e-3 relative to the output scale)."""
    import torch

    from oracle import attention as oatt

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    q, kc, vc, bt = st.q_rot.cpu(), st.caches[0].cpu(), st.caches[1].cpu(), st.bt.cpu()
    stage = st.stage()
    cfg = st.impl._oscar
    arena = None
    if stage is not None:
        arena = (stage[0].cpu(), stage[1].cpu(), stage[2].cpu(), (cfg.sink_tokens // BS) * BS, cfg.recent_tokens)

    def once():
        return oatt.decode_only_ref(q, kc, vc, bt, st.seqs, st.impl.scale, HK, D, arena)

    want = once()
    rel = (gpu_out.cpu() - want).abs().max().item() / max(want.abs().max().item(), 1e-30)
    samples = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(samples) < 6:
        t0 = time.perf_counter()
        once()
        samples.append(time.perf_counter() - t0)
    return {"value": round(statistics.median(samples) * 1e6, 1), "unit": "us/layer", "cores": cores,
            "kind": "port", "sample": f"median of {len(samples)} runs of the oracle DecodeOnly read on the same "
                                      f"state ({sum(st.seqs)}-token INT2 history, FP32 sink + tail, fp32)"}, rel


def cpu_baseline(st, gpu_out, seconds: float, label: str = "C2"):
    """The oracle's read path on the same (GPU-written) C2 state, on this host.

    Also the parity gate of the measured kernel: its output must match the
    oracle within the fp32 contract (1e-3 relative to the output scale).
    """
    import torch

    from oracle import attention as oatt

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    q, k, v = st.q_rot.cpu(), st.k_rot.cpu(), st.v_rot.cpu()
    kc, vc = st.caches[0].cpu(), st.caches[1].cpu()
    bt = st.bt.cpu()
    stage = tuple(t.cpu() for t in st.stage()[:3]) if st.stage() is not None else None

    def once():
        return oatt.paged_attention_ref(q, k, v, kc, vc, bt, st.qsl, st.seqs, st.impl.scale, stage)

    want = once()
    rel = (gpu_out.cpu() - want).abs().max().item() / max(want.abs().max().item(), 1e-30)
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
    base = {"value": round(med * 1e6, 1), "unit": "us/layer", "cores": cores, "kind": "port",
            "sample": f"median of {len(samples)} runs (~{seconds:.0f} s) of the oracle read path on the {label} "
                      f"layer state (dequant {sum(st.seqs) - q.shape[0]}-token INT2 history + FP32 window splice "
                      f"+ causal SDPA, {q.shape[0]} queries x {q.shape[1]} heads, fp32); host CPU {model}"}
    return base, rel


SUITE = {
    "C3": {"workload": "C3: concurrent MTP decode, 32 requests x 4 query tokens, Hq=6 Hk=1 D=256, histories "
                       "uniform in [2048, 16384] in 128-token pages drawn from a shared 8192-page pool, FP32 "
                       "sink=128/recent=256 window (staging 8192), clip 0.96/0.92, 16 distinct layers",
           "q_len": 4, "pool": 8192, "layers": 16},
    "C5-decode": {"workload": "C5 decode: 8 requests x 1 query token, 32768-token histories, Hq=6 Hk=1 D=256, "
                              "pages scattered over a 2056-page pool (2048 history pages + 8 for the step's "
                              "token), FP32 sink=128/recent=256 window (staging 8192), 16 distinct layers",
                  "q_len": 1, "pool": 2056, "layers": 16},
    "C2-decode-only": {"workload": "C2 DecodeOnly: the read without fresh K/V, 1 request x 1 query token over "
                                   "its whole 24580-token INT2 history in 193 shuffled 128-token pages, Hq=6 "
                                   "Hk=1 D=256, FP32 sink=128/recent=256 window (staging 8192), 64 distinct layers",
                       "q_len": 1, "pool": 193, "layers": 64, "decode_only": True},
    "C4": {"workload": "C4: prefill continuation, 1 request, 15360-token INT2 history + 9256 new tokens "
                       "(causal over history + new), Hq=6 Hk=1 D=256, 128-token pages, FP32 window"},
}
MFMA_BF16_PEAK_TFLOPS = 2500.0


def suite_histories(name: str):
    import torch

    if name == "C3":
        g = torch.Generator().manual_seed(2024)
        return [int(x) for x in torch.randint(2048, 16385, (32,), generator=g)]
    if name == "C2-decode-only":
        return [24579]
    return [32768] * 8


def bench_prefill(args, dev, seed=71):
    """C4: the prefill-continuation kernel on the written 15360 + 9256 state."""
    import torch

    from oscar_amd.kernels import prefill

    hist, new = 15360, 9256
    st = build_layer(dev, [hist], new, pool=(hist + new + BS - 1) // BS, seed=seed)
    stage = st.stage()
    stage3 = None if stage is None else stage[:3]

    def run():
        return prefill.prefill_continuation(st.q_rot, st.k_rot, st.v_rot, st.caches[0], st.caches[1],
                                            st.bt[0], hist, st.impl.scale, stage3)

    for _ in range(2):
        out = run()
    torch.cuda.synchronize()
    reps = 10
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        run()
    e1.record(stream)
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / reps
    visible = new * (hist + 1) + new * (new - 1) // 2
    flops = 4 * D * HQ * visible
    return {"us": us, "flops": flops, "tflops": flops / (us * 1e-6) / 1e12, "state": st, "out0": out}


def prefill_cpu_baseline(st, gpu_out, hist: int, seconds: float):
    """The oracle's dense read path for C4 (dequant + splice + chunked causal SDPA), and the parity
    of the timed kernel against it (bf16 contract: 2e-2 + 2^-8 |oracle| elementwise)."""
    import torch

    from oracle import attention as oatt

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    q, k, v = st.q_rot.cpu(), st.k_rot.cpu(), st.v_rot.cpu()
    kc, vc, bt = st.caches[0].cpu(), st.caches[1].cpu(), st.bt.cpu()
    stage = tuple(t.cpu() for t in st.stage()[:3]) if st.stage() is not None else None
    samples, want = [], None
    t_end = time.perf_counter() + seconds
    while not samples or (time.perf_counter() < t_end and len(samples) < 6):
        t0 = time.perf_counter()
        want = oatt.paged_attention_ref(q, k, v, kc, vc, bt, st.qsl, st.seqs, st.impl.scale, stage)
        samples.append(time.perf_counter() - t0)
    got = gpu_out.cpu()
    ok = bool(((got - want).abs() <= 2e-2 + 2.0 ** -8 * want.abs()).all())
    err = (got - want).abs().max().item()
    return {"value": round(statistics.median(samples) * 1e3, 1), "unit": "ms/layer", "cores": cores,
            "kind": "port", "sample": f"median of {len(samples)} runs of the oracle dense read path on the "
                                      f"C4 state (dequant + window splice + chunked causal SDPA, fp32)"}, ok, err


def suite(args, dev):
    """One JSON line per extra workload: C3 and C5 decode (HBM roofline), C4 prefill (MFMA roofline)."""
    for name in args.suite.split(","):
        cfg = SUITE[name]
        if name == "C4":
            r = bench_prefill(args, dev)
            cpu, ok, err = prefill_cpu_baseline(r["state"], r["out0"], 15360, args.cpu_seconds)
            if not ok:
                raise SystemExit(f"C4 parity gate failed: max abs err {err:.3e}")
            line = {"config": name, "workload": cfg["workload"], "value": round(r["us"], 2),
                    "unit": "us/layer", "arith": "bf16-contract: INT2 dequant to f16, f16 MFMA, f32 softmax",
                    "roofline": {"bound": "mfma", "achieved": round(r["tflops"], 1),
                                 "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                 "frac": round(r["tflops"] / MFMA_BF16_PEAK_TFLOPS, 4), "flops": r["flops"]},
                    "parity_max_abs_err": err, "cpu_baseline": cpu}
        else:
            hist = suite_histories(name)
            only = cfg.get("decode_only", False)
            dec = bench_decode(args, dev, hist, cfg["q_len"], pool=cfg["pool"], layers=cfg["layers"],
                               decode_only=only)
            if only:
                cpu, rel = decode_only_cpu_baseline(dec["state"], dec["out0"], args.cpu_seconds)
            else:
                cpu, rel = cpu_baseline(dec["state"], dec["out0"], args.cpu_seconds, name)
            if not rel <= (2e-3 if only else 1e-3):
                raise SystemExit(f"{name} parity gate failed: rel err {rel:.3e}")
            line = {"config": name, "workload": cfg["workload"], "value": round(dec["us_per_layer"], 3),
                    "unit": "us/layer", "steps": dec["steps"],
                    "roofline": {"bound": "hbm", "achieved": round(dec["gbps"], 1), "peak": HBM_PEAK_GBPS,
                                 "unit": "GB/s", "frac": round(dec["gbps"] / HBM_PEAK_GBPS, 4),
                                 "bytes_per_layer": dec["bytes"]["total"]},
                    "history_tokens": sum(dec["state"].seqs) if only else sum(hist),
                    "staged_tokens": dec["bytes"]["staged_tokens"],
                    "parity_rel_err": rel, "cpu_baseline": cpu}
        print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=640)
    ap.add_argument("--warmup", type=int, default=128)
    ap.add_argument("--layers", type=int, default=64)
    ap.add_argument("--qw-iters", type=int, default=64)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--tps", type=int, default=0, help="decode tiles per split (0: automatic)")
    ap.add_argument("--skip-quant-write", action="store_true")
    ap.add_argument("--window", type=int, default=1, help="diagnostic: 0 disables the FP32 window")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="run a plain device copy of this many MiB first (PMC byte-counter calibration)")
    ap.add_argument("--suite", default="",
                    help="comma list of extra workloads (C3, C5-decode, C2-decode-only, C4): one JSON "
                         "line each instead of the headline line")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (one TP rank's share "
              "per GPU, no collectives); run with --gpus 1", file=sys.stderr)
        raise SystemExit(2)
    import torch

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    dev = torch.device("cuda:0")
    if args.suite:
        suite(args, dev)
        return
    if args.copy_probe_mib > 0:
        copy_probe(dev, args.copy_probe_mib)
    log("bench: decode C2")
    dec = bench_decode(args, dev, [C2_HISTORY], C2_QLEN, pool=193, layers=args.layers)
    log(f"bench: decode {dec['us_per_layer']:.3f} us/layer ({dec['gbps']:.1f} GB/s)")
    qw = None
    if not args.skip_quant_write:
        qw = bench_quant_write(args, dev)
        log(f"bench: quant-write {qw['gbps']:.1f} GB/s")
    cpu, rel = None, None
    if not args.no_cpu_baseline:
        log("bench: cpu baseline + parity gate")
        cpu, rel = cpu_baseline(dec["state"], dec["out0"], args.cpu_seconds)
        if not rel <= 1e-3:
            raise SystemExit(f"decode parity gate failed: rel err {rel:.3e}")
    line = {
        "metric": METRIC,
        "value": round(dec["us_per_layer"], 4),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": dec["steps"],
        "warmup": dec["warmup"],
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
            "decode_parity_rel_err_vs_oracle": rel,
            "quant_write": None if qw is None else {"workload": "C5 write: 65536 tokens bf16, Hk=1, random slots ~1/16 skipped, "
                                        "rotation on MFMA, clip 0.96/0.92",
                            "us_per_call": round(qw["us_per_call"], 3), "gbps": round(qw["gbps"], 1),
                            "frac_of_hbm_peak": round(qw["gbps"] / HBM_PEAK_GBPS, 4),
                            "bytes_per_call": qw["bytes"]},
        },
        "roofline": {"bound": "hbm", "achieved": round(dec["gbps"], 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(dec["gbps"] / HBM_PEAK_GBPS, 4),
                     "traffic": traffic_from_profile(ROOT / "oscar_amd" / "csrc" / "paged_decode.hip")},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
