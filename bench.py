"""Benchmark of the OSCAR INT2 KV-cache hot path on one MI355X.

Headline metric: 4-token MTP decode attention over a 24,579-token INT2
history (Hq=6, Hk=1, D=256, 193 shuffled 128-token pages, FP32 sink/recent
window) in microseconds per layer and achieved HBM GB/s, plus the
quantize-write GB/s of a 65,536-token bulk write (random slots, ~1/16
skipped).

A step is one pass of the decode attention (`oscar_paged_decode`: split +
merge kernels) over all `--layers` distinct per-layer states (64 x ~13 MB,
beyond the 256 MB Infinity Cache), one call per layer, so every timed step
reads every layer's history from HBM whatever `--steps` is.  Exactly
`--warmup` steps are replayed from one HIP graph, then exactly `--steps`
steps from another, bracketed by device synchronisations and HIP events on
the replay stream; `value` is µs per layer (a step's time / layers) and
`ms_per_step` the time of one pass.  Inputs are resident in HBM before
timing starts.

Also in the line (config):
* forward: the whole impl forward of the same MTP step per layer (fused step
  write, decode, merge with R_v^T and the bf16 cast), timed the same way;
* quant_write: the 65,536-token bulk write;
* suite: the other workloads, each with its roofline, parity gate against
  the oracle and the oracle's CPU time: 32 x 4 concurrent MTP decode, 8 x 1
  long-context decode through the MTP and DecodeOnly entries, and the
  15360 + 9256 prefill continuation.

roofline.traffic (HBM bytes per call) and mfma_util come from the committed
rocprofv3 summaries profiles/hbm_traffic.txt and profiles/mfma_counters.txt,
and only while every source file they were measured on is unchanged (each
summary records their sha256); otherwise they are null.

cpu_baseline: the CPU oracle's forward of the same step (rotate + clip +
INT2 write + window write of the 4 new tokens, then history dequant + window
splice + causal SDPA + output rotation, fp32) on this host's cores, and at 2
threads as the reference's own harness runs.

Prints one JSON line.
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import os
import statistics
import sys
import time
from pathlib import Path
from types import SimpleNamespace as NS

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "MTP decode attn µs/layer + HBM GB/s at 24K INT2 history; quant-write GB/s"
HBM_PEAK_GBPS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
C2_HISTORY, C2_QLEN, HQ, HK, D, BS = 24579, 4, 6, 1, 256, 128
BF16_ABS, BF16_REL = 2e-2, 2.0 ** -8


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class LayerState:
    """One FULL layer's state right before its decode read, written on the GPU
    by the product write path, plus the step's own inputs."""

    def __init__(self, impl, layer, caches, bt, qsl, seqs, step):
        self.impl, self.layer, self.caches, self.bt = impl, layer, caches, bt
        self.qsl, self.seqs = qsl, seqs
        self.step = step            # q, k, v (bf16), q_rot, k_rot, v_rot (fp32), md

    def stage(self):
        return self.impl._stage(self.layer)


def make_impl(window=True):
    import contextlib
    import io

    from oscar_amd.backend import OscarAttentionBackendImpl

    impl = OscarAttentionBackendImpl.__new__(OscarAttentionBackendImpl)
    impl.head_size, impl.num_kv_heads, impl.num_heads = D, HK, HQ
    impl.scale = D ** -0.5
    impl.key_cache = impl.value_cache = None
    with contextlib.redirect_stdout(io.StringIO()):
        impl._oscar_setup()
    impl._oscar_cfg = dataclasses.replace(impl._oscar, k_clip_ratio=0.96, v_clip_ratio=0.92, sink_tokens=128,
                                          recent_tokens=256, staging_tokens=8192 if window else 0)
    return impl


def build_layer(dev, history: list, q_len: int, pool: int, seed: int, window=True) -> LayerState:
    """Prefill-write every request's history, then write the step's tokens (bulk write path)."""
    import torch

    from oscar_amd import synthetic

    impl = make_impl(window)
    Rk, Rv = synthetic.rotations(D, seed)
    layer = NS(layer_name="model.layers.0.self_attn.attn", _oscar_rots=(Rk.to(dev), Rv.to(dev)))
    caches = [torch.zeros(pool, BS, HK, D, dtype=torch.int8, device=dev) for _ in range(2)]
    B = len(history)
    need = [(h + q_len + BS - 1) // BS for h in history]
    perm = synthetic.page_permutation(pool, seed + 1)
    bt = torch.zeros(B, max(need), dtype=torch.int32)
    off = 0
    for i, n in enumerate(need):
        bt[i, :n] = perm[off:off + n]
        off += n
    btd = bt.to(dev)

    def write(counts, starts, seqs, kseed):
        n = sum(counts)
        k, v = synthetic.kv(n, HK, D, seed=kseed)
        slots = torch.cat([synthetic.slots_for(bt[i], st, c, BS) for i, (st, c) in enumerate(zip(starts, counts))])
        qsl = [0]
        for c in counts:
            qsl.append(qsl[-1] + c)
        md = NS(num_actual_tokens=n, slot_mapping=slots.to(dev), query_start_loc_cpu=torch.tensor(qsl),
                seq_lens_list=list(seqs), block_tables=btd)
        kd, vd = k.to(dev), v.to(dev)
        impl.do_kv_cache_update(layer, kd, vd, caches, md.slot_mapping)
        if window:
            impl._ensure_staging(layer, caches)
            impl._staging_write(layer, kd, vd, md)
        return kd, vd, md

    write(history, [0] * B, history, seed + 2)
    seqs = [h + q_len for h in history]
    kd, vd, md = write([q_len] * B, history, seqs, seed + 3)
    q = synthetic.queries(q_len * B, HQ, D, seed=seed + 4).to(dev)
    rk, rv = layer._oscar_rots
    torch.cuda.synchronize()
    step = NS(q=q, k=kd, v=vd, q_rot=q.float() @ rk, k_rot=kd.float() @ rk, v_rot=vd.float() @ rv, md=md)
    return LayerState(impl, layer, caches, btd, [int(x) for x in md.query_start_loc_cpu], seqs, step)


def clone_layer(st: LayerState) -> LayerState:
    layer = NS(**vars(st.layer))
    for name in ("_oscar_stage_k", "_oscar_stage_v", "_oscar_slot_owner", "_oscar_seat_winner",
                 "_oscar_stage_kimg", "_oscar_stage_vimg"):
        if getattr(st.layer, name, None) is not None:
            setattr(layer, name, getattr(st.layer, name).clone())
    return LayerState(st.impl, layer, [c.clone() for c in st.caches], st.bt, st.qsl, st.seqs, st.step)


def decode_bytes(st: LayerState) -> dict:
    """Algorithmic HBM bytes of one layer decode: every history token's INT2
    slot bytes (8 meta + 64 K + 64 V codes), the staged fp32 K/V of tokens the
    window owns, the owner table, q / new k / new v / out in fp32 and the
    block-table entries."""
    import torch

    owner = st.stage()[2].cpu() if st.stage() is not None else None
    bt = st.bt.cpu()
    n_q = st.step.q_rot.shape[0]
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
    n_q = len(st.seqs)
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


def graph_us(calls: list, steps: int, warmup: int) -> float:
    """Mean µs per call over exactly `steps` passes through all of `calls`
    (one call each, in order), replayed from one HIP graph after `warmup`
    passes replayed from another."""
    import torch

    for c in calls:          # first-call setup (operands, arenas) stays out of the graphs
        c()
    torch.cuda.synchronize()

    def capture(passes):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(passes):
                for c in calls:
                    c()
        return g

    warm = capture(warmup) if warmup > 0 else None
    timed = capture(steps)
    if warm is not None:
        warm.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    timed.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1000.0 / (steps * len(calls))


def layer_states(dev, history, q_len, pool, layers, seed=93, window=True):
    base = build_layer(dev, history, q_len, pool, seed, window=window)
    return [base] + [clone_layer(base) for _ in range(layers - 1)]


def last_queries(st: LayerState):
    """One rotated query per request: each request's last step token."""
    return st.step.q_rot[[b - 1 for b in st.qsl[1:]]].contiguous()


def bench_decode(dev, states, steps, warmup, tps=0, decode_only=False):
    from oscar_amd.kernels import decode

    base = states[0]
    nbytes = decode_only_bytes(base) if decode_only else decode_bytes(base)
    if decode_only:
        cfg = base.impl._oscar
        q1 = last_queries(base)
        plans = [decode.decode_only_plan(q1, st.caches[0], st.caches[1], st.bt, st.seqs, st.impl.scale,
                                         st.stage(), cfg.sink_tokens, cfg.recent_tokens, tiles_per_split=tps)
                 for st in states]
    else:
        s = base.step
        plans = [decode.plan(s.q_rot, s.k_rot, s.v_rot, st.caches[0], st.caches[1], st.bt, st.qsl, st.seqs,
                             st.impl.scale, st.stage(), tiles_per_split=tps) for st in states]
    us = graph_us([p.launch for p in plans], steps, warmup)
    out0 = plans[0].launch().clone()
    return {"us": us, "gbps": nbytes["total"] / (us * 1e-6) / 1e9, "bytes": nbytes, "out0": out0}


def bench_forward(dev, states, steps, warmup):
    """The impl forward of the MTP step on every layer state (fused step write,
    decode, merge with R_v^T and the bf16 cast)."""
    import torch

    outs = [torch.empty(st.step.q.shape[0], HQ * D, dtype=torch.bfloat16, device=dev) for st in states]
    for st in states:
        st.impl.allow_fixed_step_capture()      # every replay repeats this one step

    def call(st, out):
        s = st.step
        return lambda: st.impl.forward(st.layer, s.q, s.k, s.v, st.caches, s.md, output=out)

    calls = [call(st, o) for st, o in zip(states, outs)]
    us = graph_us(calls, steps, warmup)
    out0 = outs[0].clone()
    # The same forwards launched from Python one after another (no graph):
    # the per-layer wall time an eager engine sees, host work included.
    import time

    for c in calls:
        c()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        for c in calls:
            c()
    torch.cuda.synchronize()
    eager = (time.perf_counter() - t0) * 1e6 / (steps * len(calls))
    return {"us": us, "eager_us": eager, "out0": out0}


def bench_quant_write(dev, steps=16):
    import torch

    from oscar_amd import synthetic
    from oscar_amd.kernels import quant

    N = 65536
    pages = N // BS + 32
    g = torch.Generator().manual_seed(55)
    Rk, Rv = synthetic.rotations(D, seed=56)
    ops = [quant.rotation_operand(R.to(dev)) for R in (Rk, Rv)]
    calls, keep = [], []
    valid_total = 0
    for s in range(4):
        k, v = synthetic.kv(N, HK, D, seed=100 + s)
        slots = torch.randperm(pages * BS, generator=g)[:N].to(torch.int64)
        slots[torch.rand(N, generator=g) < 1 / 16] = -1
        valid_total += int((slots >= 0).sum())
        kd, vd, sd = k.to(dev), v.to(dev), slots.to(dev)
        kc = torch.zeros(pages, BS, HK, D, dtype=torch.int8, device=dev)
        vc = torch.zeros_like(kc)
        keep += [kd, vd, sd, kc, vc]
        calls.append(lambda kd=kd, vd=vd, sd=sd, kc=kc, vc=vc: quant.quant_write(
            kd, vd, ops[0], ops[1], kc, vc, sd, 245, 235, HK, D))
    valid = valid_total / 4
    nbytes = N * HK * 2 * D * 2 + valid * HK * 136 + N * 8 + 2 * D * D * 4
    us = graph_us(calls, steps, 8)
    # Short writes (the fp32 path of at most 2048 key + value vectors), as a
    # do_kv_cache_update of a few decode tokens issues them.
    short = {}
    for n in (4, 64):
        sc = []
        for s in range(4):
            k, v = synthetic.kv(n, HK, D, seed=200 + s)
            slots = torch.randperm(pages * BS, generator=g)[:n].to(torch.int64)
            kd, vd, sd = k.to(dev), v.to(dev), slots.to(dev)
            kc = torch.zeros(pages, BS, HK, D, dtype=torch.int8, device=dev)
            vc = torch.zeros_like(kc)
            keep += [kd, vd, sd, kc, vc]
            sc.append(lambda kd=kd, vd=vd, sd=sd, kc=kc, vc=vc: quant.quant_write(
                kd, vd, ops[0], ops[1], kc, vc, sd, 245, 235, HK, D))
        short[str(n)] = round(graph_us(sc, steps, 8), 3)
    return {"us": us, "gbps": nbytes / (us * 1e-6) / 1e9, "bytes": nbytes, "steps": steps, "short_us": short}


def bench_prefill(dev, reps=10, seed=71):
    """The prefill-continuation kernel on the written 15360 + 9256 state."""
    from oscar_amd.kernels import prefill

    hist, new = 15360, 9256
    st = build_layer(dev, [hist], new, pool=(hist + new + BS - 1) // BS, seed=seed)
    stage = st.stage()
    stage3 = None if stage is None else stage[:3]
    s = st.step
    res = {}

    def run():
        res["out"] = prefill.prefill_continuation(s.q_rot, s.k_rot, s.v_rot, st.caches[0], st.caches[1],
                                                  st.bt[0], hist, st.impl.scale, stage3)

    us = graph_us([run], reps, 2)
    run()
    visible = new * (hist + 1) + new * (new - 1) // 2
    flops = 4 * D * HQ * visible
    return {"us": us, "flops": flops, "tflops": flops / (us * 1e-6) / 1e12, "state": st, "out0": res["out"],
            "steps": reps}


def bench_prefill_forward(st: LayerState, reps=5):
    """The impl forward of the 15360 + 9256 continuation step on the written
    state: the INT2 write of the 9256 new tokens (rotation on MFMA, clip,
    quantize, slot write), the window write, the fp32 q/k/v rotations, the
    prefill kernel, the output rotation and the bf16 cast.  The step's tokens
    are rewritten with the same values on every call, so the state does not
    change.  Eager calls (the forward refuses graph capture of a step this
    size), timed with HIP events on the launch stream."""
    import torch

    s = st.step
    out = torch.empty(s.q.shape[0], HQ * D, dtype=torch.bfloat16, device=s.q.device)

    def call():
        st.impl.forward(st.layer, s.q, s.k, s.v, st.caches, s.md, output=out)

    call()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        call()
    e1.record(stream)
    torch.cuda.synchronize()
    return {"us": e0.elapsed_time(e1) * 1000.0 / reps, "steps": reps, "out0": out.clone()}


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


def profile_figures(name: str) -> dict:
    """The figures of a committed rocprofv3 summary (profiles/<name>, lines
    'figure <key>: <value>'), if every source it was measured on (lines
    'source_sha256 <file under oscar_amd/csrc>: <hex>') is unchanged; else {}
    (the bench then reports those figures as null)."""
    import hashlib

    prof = ROOT / "profiles" / name
    if not prof.exists():
        return {}
    figs, sources = {}, 0
    for line in prof.read_text().splitlines():
        if ":" not in line or line.startswith(" "):
            continue
        key, val = (x.strip() for x in line.split(":", 1))
        if key.startswith("source_sha256 "):
            src = ROOT / "oscar_amd" / "csrc" / key.split(" ", 1)[1]
            if not src.exists() or hashlib.sha256(src.read_bytes()).hexdigest() != val:
                return {}
            sources += 1
        elif key.startswith("figure "):
            try:
                figs[key.split(" ", 1)[1]] = float(val)
            except ValueError:
                pass
    return figs if sources else {}


def _traffic(key: str):
    v = profile_figures("hbm_traffic.txt").get(f"traffic {key}")
    return None if v is None else int(v)


def _mfma(key: str):
    return profile_figures("mfma_counters.txt").get(f"mfma_util {key}")


# ---------------------------------------------------------------- CPU oracle
def cpu_model() -> str:
    try:
        return next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except Exception:
        return "unknown"


def timed_median(fn, seconds: float, min_runs: int = 6):
    """One warm-up, then the median of at least min_runs runs or `seconds`."""
    fn()
    samples = []
    t_end = time.perf_counter() + seconds
    while len(samples) < min_runs or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        samples.append(time.perf_counter() - t0)
    return statistics.median(samples), len(samples)


def oracle_layer(st: LayerState):
    """The oracle's layer over CPU copies of a GPU-written state."""
    from oracle.forward import OracleLayer
    from oracle.staging import Arena

    cfg = st.impl._oscar
    rk, rv = (r.cpu() for r in st.layer._oscar_rots)
    L = OracleLayer(st.caches[0].cpu(), st.caches[1].cpu(), rk, rv, HQ, HK, D, st.impl.scale, cfg.k_clip_ratio,
                    cfg.v_clip_ratio, cfg.sink_tokens, cfg.recent_tokens, cfg.staging_tokens)
    stage = st.stage()
    if stage is not None:
        L.arena = Arena(stage[0].cpu(), stage[1].cpu(), stage[2].cpu(), BS, (cfg.sink_tokens // BS) * BS,
                        cfg.recent_tokens)
    return L


def cpu_forward_baseline(st: LayerState, gpu_read, gpu_forward, seconds: float):
    """The oracle's forward of the step (write of the new tokens + read + output
    rotation) on this host, at all cores and at 2 threads, and the parity of the
    GPU decode (fp32, 1e-3 of the output scale) and forward (bf16 contract)."""
    import torch

    from oracle import attention as oatt

    L = oracle_layer(st)
    s = st.step
    md = NS(num_actual_tokens=s.md.num_actual_tokens, slot_mapping=s.md.slot_mapping.cpu(),
            query_start_loc_cpu=s.md.query_start_loc_cpu, seq_lens_list=s.md.seq_lens_list,
            block_tables=st.bt.cpu())
    q, k, v = s.q.cpu(), s.k.cpu(), s.v.cpu()
    # parity on the GPU-written state (the forward rewrote the step's tokens the same way)
    want_read = oatt.paged_attention_ref(s.q_rot.cpu(), s.k_rot.cpu(), s.v_rot.cpu(), L.k_cache, L.v_cache,
                                         md.block_tables, st.qsl, st.seqs, L.scale, L.stage())
    read_rel = (gpu_read.cpu() - want_read).abs().max().item() / max(want_read.abs().max().item(), 1e-30)
    fwd_ok, fwd_err = None, None
    if gpu_forward is not None:
        want_fwd = (want_read @ L.R_v.t()).reshape(gpu_forward.shape)
        got = gpu_forward.cpu().float()
        fwd_ok = bool(((got - want_fwd).abs() <= BF16_ABS + BF16_REL * want_fwd.abs()).all())
        fwd_err = (got - want_fwd).abs().max().item()

    def once():
        L.forward(q.float(), k.float(), v.float(), md)

    cores = len(os.sched_getaffinity(0))
    res = {}
    for threads in (cores, 2):
        torch.set_num_threads(threads)
        res[threads] = timed_median(once, seconds)
    torch.set_num_threads(cores)
    med, n = res[cores]
    base = {"value": round(med * 1e6, 1), "unit": "us/layer", "cores": cores, "kind": "port",
            "value_2_threads": round(res[2][0] * 1e6, 1),
            "sample": f"median of {n} runs (~{seconds:.0f} s) of the oracle forward of the C2 MTP step on the "
                      f"GPU-written layer state: rotate + clip + INT2 write + window write of the 4 new tokens, "
                      f"then dequant of the {sum(st.seqs) - q.shape[0]}-token INT2 history + window splice + "
                      f"causal SDPA (4 queries x 6 heads) + output rotation, fp32; the same at 2 threads "
                      f"({res[2][1]} runs) in value_2_threads; host CPU {cpu_model()}"}
    return base, read_rel, fwd_ok, fwd_err


def cpu_read_baseline(st: LayerState, gpu_out, seconds: float, decode_only=False):
    """The oracle's read on the same state (the paged MTP read, or the
    DecodeOnly windowed read) and the parity of the GPU output against it."""
    import torch

    from oracle import attention as oatt

    L = oracle_layer(st)
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    bt = st.bt.cpu()
    if decode_only:
        q = last_queries(st).cpu()
        A = L.arena
        arena = None if A is None else (A.stage_k, A.stage_v, A.owner, A.sink_eff, L.recent)

        def once():
            return oatt.decode_only_ref(q, L.k_cache, L.v_cache, bt, st.seqs, L.scale, HK, D, arena)
    else:
        s = st.step
        q, k, v = s.q_rot.cpu(), s.k_rot.cpu(), s.v_rot.cpu()

        def once():
            return oatt.paged_attention_ref(q, k, v, L.k_cache, L.v_cache, bt, st.qsl, st.seqs, L.scale, L.stage())

    want = once()
    rel = (gpu_out.cpu() - want).abs().max().item() / max(want.abs().max().item(), 1e-30)
    med, n = timed_median(once, seconds, min_runs=3)
    torch.set_num_threads(2)
    med2, n2 = timed_median(once, seconds, min_runs=3)
    torch.set_num_threads(cores)
    return {"value": round(med * 1e6, 1), "unit": "us/layer", "cores": cores, "kind": "port",
            "value_2_threads": round(med2 * 1e6, 1),
            "sample": f"median of {n} runs of the oracle {'DecodeOnly' if decode_only else 'paged MTP'} read "
                      f"on the same GPU-written state, fp32; the same at 2 threads ({n2} runs) in "
                      f"value_2_threads"}, rel


def cpu_prefill_baseline(st: LayerState, gpu_out, seconds: float):
    """The oracle's dense read for the continuation (dequant + splice + chunked
    causal SDPA, fp32) and the parity of the kernel (bf16 contract)."""
    import torch

    from oracle import attention as oatt

    L = oracle_layer(st)
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    s = st.step
    q, k, v = s.q_rot.cpu(), s.k_rot.cpu(), s.v_rot.cpu()
    bt = st.bt.cpu()
    res = {}

    def once():
        res["want"] = oatt.paged_attention_ref(q, k, v, L.k_cache, L.v_cache, bt, st.qsl, st.seqs, L.scale,
                                               L.stage())

    med, n = timed_median(once, seconds, min_runs=2)
    torch.set_num_threads(2)
    med2, n2 = timed_median(once, seconds, min_runs=2)
    torch.set_num_threads(cores)
    got, want = gpu_out.cpu(), res["want"]
    ok = bool(((got - want).abs() <= BF16_ABS + BF16_REL * want.abs()).all())
    return {"value": round(med * 1e3, 1), "unit": "ms/layer", "cores": cores, "kind": "port",
            "value_2_threads": round(med2 * 1e3, 1),
            "sample": f"median of {n} runs of the oracle dense read of the 15360 + 9256 state, fp32; the same "
                      f"at 2 threads ({n2} runs) in value_2_threads"}, ok, (got - want).abs().max().item(), want


# ---------------------------------------------------------------- suite
def suite_histories(name: str):
    import torch

    if name == "C3":
        g = torch.Generator().manual_seed(2024)
        return [int(x) for x in torch.randint(2048, 16385, (32,), generator=g)]
    return [32768] * 8


SUITE = {
    "C3": {"workload": "32 requests x 4 MTP query tokens, Hq=6 Hk=1 D=256, histories uniform in [2048, 16384] "
                       "in 128-token pages drawn from a shared 8192-page pool, FP32 sink=128/recent=256 window "
                       "(staging 8192), clip 0.96/0.92, 16 distinct layers",
           "q_len": 4, "pool": 8192, "layers": 16},
    "C5_decode": {"workload": "8 requests x 1 query token, 32768-token histories, Hq=6 Hk=1 D=256, pages "
                              "scattered over a 2056-page pool (2048 history pages + 8 for the step's token), "
                              "FP32 sink=128/recent=256 window (staging 8192), 16 distinct layers",
                  "q_len": 1, "pool": 2056, "layers": 16},
    "C5_decode_only": {"workload": "the same 8 x 32768 state read through the DecodeOnly entry (no fresh K/V, "
                                   "one query per request over its whole 32769-token history)",
                       "q_len": 1, "pool": 2056, "layers": 16, "decode_only": True},
    "C4": {"workload": "prefill continuation, 1 request, 15360-token INT2 history + 9256 new tokens (causal "
                       "over history + new), Hq=6 Hk=1 D=256, 128-token pages, FP32 window"},
}


def suite(dev, names, cpu_seconds, steps=8):
    out = {}
    long_states = None
    for name in names:
        cfg = SUITE[name]
        log(f"bench: suite {name}")
        if name == "C4":
            r = bench_prefill(dev)
            cpu, ok, err, want = cpu_prefill_baseline(r["state"], r["out0"], cpu_seconds)
            if not ok:
                raise SystemExit(f"C4 parity gate failed: max abs err {err:.3e}")
            fw = bench_prefill_forward(r["state"])
            want_fwd = (want @ r["state"].layer._oscar_rots[1].cpu().t()).reshape(fw["out0"].shape)
            got_fwd = fw["out0"].cpu().float()
            fwd_err = (got_fwd - want_fwd).abs().max().item()
            if not bool(((got_fwd - want_fwd).abs() <= BF16_ABS + BF16_REL * want_fwd.abs()).all()):
                raise SystemExit(f"C4 forward parity gate failed: max abs err {fwd_err:.3e}")
            out[name] = {"workload": cfg["workload"], "value": round(r["us"], 2), "unit": "us/layer",
                         "steps": r["steps"],
                         "forward_us": round(fw["us"], 1), "forward_steps": fw["steps"],
                         "forward": "the impl forward of the step (INT2 write of the 9256 new tokens with the "
                                    "MFMA rotation and clip, window write, fp32 q/k/v rotations, the prefill "
                                    "kernel, output rotation and bf16 cast), eager, HIP events",
                         "forward_parity_max_abs_err": fwd_err,
                         "arith": "bf16 contract: INT2 codes as exact f16 operands, f16 MFMA, f32 softmax",
                         "roofline": {"bound": "mfma", "achieved": round(r["tflops"], 1),
                                      "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                      "frac": round(r["tflops"] / MFMA_F16_PEAK_TFLOPS, 4), "flops": r["flops"],
                                      "traffic": _traffic("C4")},
                         "mfma_util": _mfma("C4"),
                         "parity_max_abs_err": err, "cpu_baseline": cpu}
            continue
        only = cfg.get("decode_only", False)
        if name.startswith("C5") and long_states is not None:
            states = long_states
        else:
            states = layer_states(dev, suite_histories(name), cfg["q_len"], cfg["pool"], cfg["layers"])
            if name.startswith("C5"):
                long_states = states
        dec = bench_decode(dev, states, steps, 2, decode_only=only)
        cpu, rel = cpu_read_baseline(states[0], dec["out0"], cpu_seconds, decode_only=only)
        if not rel <= 1e-3:
            raise SystemExit(f"{name} parity gate failed: rel err {rel:.3e}")
        out[name] = {"workload": cfg["workload"], "value": round(dec["us"], 3), "unit": "us/layer",
                     "steps": steps, "layers_per_step": len(states), "calls_timed": steps * len(states),
                     "roofline": {"bound": "hbm", "achieved": round(dec["gbps"], 1), "peak": HBM_PEAK_GBPS,
                                  "unit": "GB/s", "frac": round(dec["gbps"] / HBM_PEAK_GBPS, 4),
                                  "bytes_per_layer": dec["bytes"]["total"], "traffic": _traffic(name)},
                     "staged_tokens": dec["bytes"]["staged_tokens"], "parity_rel_err": rel, "cpu_baseline": cpu}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10, help="timed passes over all layer states")
    ap.add_argument("--warmup", type=int, default=2, help="untimed passes before them")
    ap.add_argument("--layers", type=int, default=64)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--suite-cpu-seconds", type=float, default=4.0)
    ap.add_argument("--tps", type=int, default=0, help="decode tiles per split (0: automatic)")
    ap.add_argument("--window", type=int, default=1, help="diagnostic: 0 disables the FP32 window")
    ap.add_argument("--parts", default="forward,quant_write,suite,cpu",
                    help="comma list of what runs besides the headline decode "
                         "(forward, quant_write, suite, cpu; empty: the decode only)")
    ap.add_argument("--suite", default="C3,C5_decode,C5_decode_only,C4", help="suite workloads")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="run a plain device copy of this many MiB first (PMC byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (one TP rank's share per GPU, no "
              "collectives); run with --gpus 1", file=sys.stderr)
        raise SystemExit(2)
    if args.steps <= 0 or args.warmup < 0:
        raise SystemExit("--steps must be positive and --warmup non-negative")
    import torch

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    dev = torch.device("cuda:0")
    parts = set(p for p in args.parts.split(",") if p)
    if args.copy_probe_mib > 0:
        copy_probe(dev, args.copy_probe_mib)
    log("bench: decode C2")
    states = layer_states(dev, [C2_HISTORY], C2_QLEN, 193, args.layers, window=bool(args.window))
    dec = bench_decode(dev, states, args.steps, args.warmup, tps=args.tps)
    log(f"bench: decode {dec['us']:.3f} us/layer ({dec['gbps']:.1f} GB/s)")
    fwd = None
    if "forward" in parts:
        fwd = bench_forward(dev, states, args.steps, args.warmup)
        log(f"bench: forward {fwd['us']:.3f} us/layer (eager {fwd['eager_us']:.1f})")
    qw = None
    if "quant_write" in parts:
        qw = bench_quant_write(dev)
        log(f"bench: quant-write {qw['us']:.2f} us, {qw['gbps']:.1f} GB/s")
    cpu = read_rel = fwd_err = None
    if "cpu" in parts:
        log("bench: cpu baseline + parity gates")
        cpu, read_rel, fwd_ok, fwd_err = cpu_forward_baseline(states[0], dec["out0"],
                                                               None if fwd is None else fwd["out0"],
                                                               args.cpu_seconds)
        if not read_rel <= 1e-3:
            raise SystemExit(f"decode parity gate failed: rel err {read_rel:.3e}")
        if fwd_ok is False:
            raise SystemExit(f"forward parity gate failed: max abs err {fwd_err:.3e}")
    suite_res = suite(dev, args.suite.split(","), args.suite_cpu_seconds) if "suite" in parts else None
    line = {
        "metric": METRIC,
        "value": round(dec["us"], 4),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": dec["us"] * args.layers / 1000.0,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": "C2: MTP decode, 1 request x 4 query tokens, Hq=6 Hk=1 D=256, 24579-token INT2 history in "
                        "193 shuffled 128-token pages, FP32 sink=128/recent=256 window (staging 8192), clip "
                        f"0.96/0.92, int8-geometry caches, {args.layers} distinct layers",
            "step": f"one decode call on each of the {args.layers} distinct layer states; value = a step's "
                    f"time / {args.layers}",
            "layers_per_step": args.layers,
            "calls_timed": args.steps * args.layers,
            "arith": "INT2 codes as exact f16 operands, f16 MFMA with f32 accumulation, f32 online softmax",
            "decode_hbm_gbps": round(dec["gbps"], 1),
            "decode_bytes_per_layer": dec["bytes"]["total"],
            "decode_bytes_per_layer_160B_variant": dec["bytes"]["int2_160B_variant"],
            "staged_tokens": dec["bytes"]["staged_tokens"],
            "decode_parity_rel_err_vs_oracle": read_rel,
            "forward": None if fwd is None else {
                "workload": "the impl forward of the same step per layer: fused step write (q/k/v fp32 rotation, "
                            "INT2 write and window write of the 4 new tokens), decode, merge with R_v^T and the "
                            "bf16 cast; bf16 in and out",
                "us_per_layer": round(fwd["us"], 3), "steps": args.steps, "warmup": args.warmup,
                "calls_timed": args.steps * args.layers,
                "eager_us_per_layer": round(fwd["eager_us"], 3),
                "eager": "the same forwards launched one by one from Python without a graph, wall clock "
                         "over the steps (host work included)",
                "parity_max_abs_err_vs_oracle": fwd_err},
            "quant_write": None if qw is None else {
                "workload": "C5 write: 65536 tokens bf16, Hk=1, random slots ~1/16 skipped, rotation on MFMA, "
                            "clip 0.96/0.92", "steps": qw["steps"], "calls_timed": qw["steps"] * 4,
                "states": "4 distinct inputs and caches (4 x ~55 MB), one call each per step",
                "us_per_call": round(qw["us"], 3), "gbps": round(qw["gbps"], 1),
                "frac_of_hbm_peak": round(qw["gbps"] / HBM_PEAK_GBPS, 4), "bytes_per_call": qw["bytes"],
                "traffic": _traffic("quant_write"), "mfma_util": _mfma("quant_write"),
                "short_write_us": qw["short_us"],
                "short_write": "us per call of 4- and 64-token writes (same caches and clip), the fp32 "
                               "short path"},
            "suite": suite_res,
        },
        "roofline": {"bound": "hbm", "achieved": round(dec["gbps"], 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(dec["gbps"] / HBM_PEAK_GBPS, 4),
                     "traffic": _traffic("C2")},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
