"""Write golden vectors for the two oracle functions nothing else pins.

Run in the build container only (the reference tree is not on the GPU box):

    python tests/golden/make_golden.py

It imports the reference plugin from /root/reference and records, on small
seeded inputs (D = 32 so each fixture stays under 100 KB):

* staging_*.npz — the FP32 window arena state (owner tags, staged K/V) after
  each step of multi-request writes with hash collisions, padding requests,
  skipped slots and recycled pages (AscendOscarAttentionBackendImpl
  ._ensure_staging / _staging_write, oscar_ascend/backend.py:418-481);
* decode_only_*.npz — the windowed DecodeOnly read
  (_decode_attention_windowed, oscar_ascend/backend.py:500-586): INT2 middle,
  FP32 sink when fully staged, the staged run ending at the last position,
  merged by log-sum-exp, on arenas with planted gaps (an unstaged sink seat,
  unstaged positions inside the recent window, a request no longer than the
  sink, seat collisions);
* forward_*.npz — the impl-level forward (rotate + clip + INT2 store +
  staging + read, backend.py:150-415) for a prefill step followed by MTP
  steps, through the default dense route and through the paged route (its
  Triton kernel replaced by the reference's own torch oracle, as the
  reference test does: tests/test_backend.py:320-367), with the INT2 cache
  bytes after the last step.

Only inputs and outputs are saved (numpy, no pickles); the generator is this
file.  tests/test_oracle_golden.py replays the inputs through oracle/ and
compares.
"""
from __future__ import annotations

import sys
from pathlib import Path
from types import SimpleNamespace as NS

import numpy as np
import torch

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent


def ref_modules():
    sys.path.insert(0, str(REF))
    import oscar_ascend.backend as backend
    import oscar_ascend.kernels.paged_attention as paged

    return backend, paged


def make_impl(backend, d, hk, hq, sink, recent, staging, clip=(0.0, 0.0)):
    Impl = backend.AscendOscarAttentionBackendImpl
    impl = Impl.__new__(Impl)
    impl.head_size, impl.num_kv_heads, impl.num_heads = d, hk, hq
    impl.scale = d ** -0.5
    impl.key_cache = impl.value_cache = None
    impl._oscar_setup()
    impl._oscar.sink_tokens, impl._oscar.recent_tokens, impl._oscar.staging_tokens = sink, recent, staging
    impl._oscar.window_enabled = staging > 0 and (sink > 0 or recent > 0)
    impl._oscar.k_clip_ratio, impl._oscar.v_clip_ratio = clip
    return impl


def meta(slots, qsl, seqs, bt):
    return NS(num_actual_tokens=len(slots), slot_mapping=torch.tensor(slots, dtype=torch.int64),
              query_start_loc=torch.tensor(qsl), actual_seq_lengths_q=list(qsl[1:]),
              seq_lens=torch.tensor(seqs), seq_lens_cpu=torch.tensor(seqs), seq_lens_list=list(seqs),
              block_tables=bt)


def staging_case(backend, name, bs, sink, recent, staging, steps, seed, d=32, hk=1):
    g = torch.Generator().manual_seed(seed)
    impl = make_impl(backend, d, hk, 2 * hk, sink, recent, staging)
    rk = torch.linalg.qr(torch.randn(d, d, generator=g)).Q
    rv = torch.linalg.qr(torch.randn(d, d, generator=g)).Q
    layer = NS(layer_name="model.layers.0.self_attn.attn", _oscar_rots=(rk, rv))
    cache = [torch.zeros(64, bs, hk, d, dtype=torch.bfloat16) for _ in range(2)]
    impl._set_caches(cache)
    impl._ensure_staging(layer, cache)
    rec = {"bs": bs, "sink": sink, "recent": recent, "staging": staging, "rk": rk.numpy(), "rv": rv.numpy(),
           "steps": len(steps)}
    for i, (slots, qsl, seqs) in enumerate(steps):
        n = len(slots)
        k = torch.randn(n, hk, d, generator=g)
        v = torch.randn(n, hk, d, generator=g)
        impl._staging_write(layer, k, v, meta(slots, qsl, seqs, torch.zeros(1, 1, dtype=torch.int32)))
        rec[f"s{i}_slots"] = np.asarray(slots, dtype=np.int64)
        rec[f"s{i}_qsl"] = np.asarray(qsl, dtype=np.int64)
        rec[f"s{i}_seqs"] = np.asarray(seqs, dtype=np.int64)
        rec[f"s{i}_k"] = k.numpy()
        rec[f"s{i}_v"] = v.numpy()
        rec[f"s{i}_owner"] = layer._oscar_slot_owner.numpy().copy()
        rec[f"s{i}_stage_k"] = layer._oscar_stage_k.numpy().copy()
        rec[f"s{i}_stage_v"] = layer._oscar_stage_v.numpy().copy()
    np.savez_compressed(OUT / f"staging_{name}.npz", **rec)


def forward_case(backend, paged, name, route, window, clip, seed, d=32, hk=1, hq=6, bs=16, pool=24):
    g = torch.Generator().manual_seed(seed)
    impl = make_impl(backend, d, hk, hq, 16 if window else 0, 16 if window else 0, 64 if window else 0, clip)
    if route == "paged":
        impl._oscar.use_paged = True
        impl._oscar_use_triton = True
        paged.oscar_paged_attention_triton = lambda *a, **kw: paged.oscar_paged_attention_ref(*a)
        import oscar_ascend.kernels.store_kernel as store

        store.oscar_store_triton = store.oscar_store_ref
    else:
        impl._oscar.use_paged = False
        impl._oscar_use_triton = False
    rk = torch.linalg.qr(torch.randn(d, d, generator=g)).Q
    rv = torch.linalg.qr(torch.randn(d, d, generator=g)).Q
    layer = NS(layer_name="model.layers.0.self_attn.attn", _oscar_rots=(rk, rv))
    cache = [torch.zeros(pool, bs, hk, d, dtype=torch.bfloat16) for _ in range(2)]
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    bt = torch.stack([perm[:12], perm[12:24]])
    # (q_lens, seq_lens) per step for two requests: prefill, then MTP steps.
    steps = [([24, 20], [24, 20]), ([4, 3], [28, 23]), ([4, 1], [32, 24]), ([2, 4], [34, 28])]
    rec = {"bs": bs, "pool": pool, "d": d, "hk": hk, "hq": hq, "window": int(window), "clip": np.asarray(clip),
           "route": route, "rk": rk.numpy(), "rv": rv.numpy(), "bt": bt.numpy(), "steps": len(steps)}
    for i, (qlens, seqs) in enumerate(steps):
        n = sum(qlens)
        q = torch.randn(n, hq, d, generator=g)
        k = torch.randn(n, hk, d, generator=g) * torch.linspace(0.5, 3.0, d)
        v = torch.randn(n, hk, d, generator=g)
        qsl, slots = [0], []
        for r, (ql, s) in enumerate(zip(qlens, seqs)):
            qsl.append(qsl[-1] + ql)
            pos = torch.arange(s - ql, s)
            slots += (bt[r][pos // bs].long() * bs + pos % bs).tolist()
        md = meta(slots, qsl, seqs, bt)
        md.attn_state = backend.AscendAttentionState.SpecDecoding
        out = impl.forward(layer, q, k, v, cache, md, output=torch.empty(n, hq, d))
        rec[f"s{i}_q"], rec[f"s{i}_k"], rec[f"s{i}_v"] = q.numpy(), k.numpy(), v.numpy()
        rec[f"s{i}_slots"] = np.asarray(slots, dtype=np.int64)
        rec[f"s{i}_qsl"] = np.asarray(qsl, dtype=np.int64)
        rec[f"s{i}_seqs"] = np.asarray(seqs, dtype=np.int64)
        rec[f"s{i}_out"] = out.numpy().copy()
    rec["kcache"] = cache[0].view(torch.uint8).numpy().copy()
    rec["vcache"] = cache[1].view(torch.uint8).numpy().copy()
    np.savez_compressed(OUT / f"forward_{name}.npz", **rec)


def decode_only_case(backend, name, seed, d=32, hk=1, hq=4, bs=16, pool=40, sink=16, recent=32, staging=64):
    """History written by the reference's own store + window write, gaps planted in
    the owner tags, then the windowed DecodeOnly read."""
    g = torch.Generator().manual_seed(seed)
    impl = make_impl(backend, d, hk, hq, sink, recent, staging)
    impl._oscar_use_triton = False
    import oscar_ascend.kernels.store_kernel as store

    store.oscar_store_triton = store.oscar_store_ref
    rk = torch.linalg.qr(torch.randn(d, d, generator=g)).Q
    rv = torch.linalg.qr(torch.randn(d, d, generator=g)).Q
    layer = NS(layer_name="model.layers.0.self_attn.attn", _oscar_rots=(rk, rv))
    cache = [torch.zeros(pool, bs, hk, d, dtype=torch.bfloat16) for _ in range(2)]
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    seqs = [70, 9, 45, 100]
    per = pool // len(seqs)
    bt = torch.stack([perm[i * per:(i + 1) * per] for i in range(len(seqs))])
    qsl, slots = [0], []
    for r, s in enumerate(seqs):
        qsl.append(qsl[-1] + s)
        pos = torch.arange(s)
        slots += (bt[r][pos // bs].long() * bs + pos % bs).tolist()
    n = sum(seqs)
    k = torch.randn(n, hk, d, generator=g) * torch.linspace(0.5, 3.0, d)
    v = torch.randn(n, hk, d, generator=g)
    md = meta(slots, qsl, seqs, bt)
    impl._set_caches(cache)
    impl._ensure_staging(layer, cache)
    impl.do_kv_cache_update(layer, k, v, cache, md.slot_mapping)
    impl._staging_write(layer, k, v, md)
    owner = layer._oscar_slot_owner
    R = layer._oscar_stage_rows

    def unstage(r, pos):
        page = int(bt[r][pos // bs])
        owner[page % R, pos % bs] = -1

    unstage(0, 3)                     # request 0: a sink seat lost -> no sink segment
    unstage(2, seqs[2] - 4)           # request 2: the staged tail run starts after this gap
    unstage(3, seqs[3] - 1)           # request 3: last position unstaged -> no tail segment
    q = torch.randn(len(seqs), hq, d, generator=g)
    dmd = NS(seq_lens=torch.tensor(seqs), block_tables=bt)
    out = impl._decode_attention(q, cache, dmd, layer)
    rec = {"d": d, "hk": hk, "hq": hq, "bs": bs, "sink": sink, "recent": recent, "staging": staging,
           "rk": rk.numpy(), "rv": rv.numpy(), "bt": bt.numpy(), "seqs": np.asarray(seqs, dtype=np.int64),
           "q": q.numpy(), "out": out.numpy().copy(), "kcache": cache[0].view(torch.uint8).numpy().copy(),
           "vcache": cache[1].view(torch.uint8).numpy().copy(), "owner": owner.numpy().copy(),
           "stage_k": layer._oscar_stage_k.numpy().copy(), "stage_v": layer._oscar_stage_v.numpy().copy(),
           "sink_eff": impl.sink_eff}
    np.savez_compressed(OUT / f"decode_only_{name}.npz", **rec)


def main():
    backend, paged = ref_modules()
    torch.set_num_threads(4)
    # bs=4, 8 rows: two long requests collide in the arena, then an MTP step
    # with a padding request and a skipped slot, then recycled pages.
    steps_small = [
        ([0, 1, 2, 3, 4, 5, 6, 7, 8, 32, 33, 34, 35, 36], [0, 9, 14], [9, 5]),
        ([9, 10, 11, 37, -1, 39], [0, 3, 6, 6], [12, 8, 1]),
        ([40, 41, 42, 43, 44, 45, 46, 47, 0, 1, 2, 3], [0, 12], [40]),
        ([4, 5, 6, 7], [0, 4], [44]),
    ]
    staging_case(backend, "bs4", 4, 4, 4, 8, steps_small, seed=11)
    # bs=16 with a 64-token arena: hashes of pages p and p + rows collide.
    steps_mid = [
        (list(range(0, 50)) + list(range(16 * 5, 16 * 5 + 30)), [0, 50, 80], [50, 30]),
        ([50, 51, 52, 16 * 5 + 30, 16 * 5 + 31], [0, 3, 5], [53, 32]),
        (list(range(16 * 9, 16 * 9 + 20)), [0, 20], [300]),
    ]
    staging_case(backend, "bs16", 16, 16, 20, 64, steps_mid, seed=12)
    for route in ("dense", "paged"):
        for window in (False, True):
            for clip in ((0.0, 0.0), (0.96, 0.92)):
                tag = f"{route}_w{int(window)}_c{int(clip[0] > 0)}"
                forward_case(backend, paged, tag, route, window, clip, seed=21)
    decode_only_case(backend, "gaps", seed=31)
    decode_only_case(backend, "bs8", seed=32, bs=8, pool=64, sink=8, recent=24, staging=32)
    print("golden fixtures written to", OUT)


if __name__ == "__main__":
    main()
