"""Seeded random shapes through every GPU entry point against the oracle.

Each case draws page size, kv heads / group, request count, history and
query lengths (page edges included), window geometry, and cache dtype.  It
runs the MTP decode (1e-3 of the output scale), the DecodeOnly read over
the same caches (1e-3; half that over a 1000-case sweep and on the
window-heavy cases), the pre-rotated quantize-write (bit-exact, random
caches, skipped and out-of-range slots, clip ratios), and the prefill
continuation (bf16 contract 2e-2 + 2^-8 |oracle|).  The seeds are fixed, so
the cases are the same on every run."""
import random

import pytest
import torch

from oracle import attention as oatt
from oracle import rotate as orot
from oracle import store as ostore
from oscar_amd import synthetic
from oscar_amd.kernels import decode, prefill, quant
from tests.scenarios import decode_case

pytestmark = pytest.mark.gpu
D = 256


def decode_cases(seed, n):
    rng = random.Random(seed)
    for _ in range(n):
        bs = rng.choice([32, 64, 128])
        hk, hq = rng.choice([(1, 6), (2, 12), (4, 8), (1, 1), (2, 4)])
        B = rng.randint(1, 6)
        hist = [rng.choice([0, 1, 5, 31, 32, 33, 127, 128, 129, rng.randint(0, 3000)]) for _ in range(B)]
        qlens = [rng.randint(1, 16) if rng.random() < 0.7 else 1 for _ in range(B)]
        window = rng.random() < 0.8
        sink = rng.choice([0, bs, 2 * bs, bs // 2])
        recent = rng.choice([0, 16, bs, 3 * bs, 200])
        staging = rng.choice([bs * 2, 512, 8192])
        cd = rng.choice([torch.int8, torch.bfloat16])
        yield dict(history=hist, q_lens=qlens, bs=bs, hk=hk, hq=hq, seed=rng.randint(0, 10 ** 6), sink=sink,
                   recent=recent, staging=staging, window=window, cache_dtype=cd)


def route_errors(device, params):
    """max |gpu - oracle| / max |oracle| of the MTP read and of the DecodeOnly
    read of one random case (outputs checked finite)."""
    params = dict(params)
    hist, qlens = params.pop("history"), params.pop("q_lens")
    case = decode_case(hist, qlens, **params)
    L = case.layer
    q, k, v = case.rotated()
    stage = L.stage() if L.window_enabled else None
    want = oatt.paged_attention_ref(q, k, v, L.k_cache, L.v_cache, case.bt, case.qsl, case.seqs, L.scale, stage)
    dstage = None if stage is None else tuple(t.to(device) for t in stage)
    kc, vc, bt = L.k_cache.to(device), L.v_cache.to(device), case.bt.to(device)
    got = decode.paged_attention(q.to(device), k.to(device), v.to(device), kc, vc, bt, case.qsl, case.seqs,
                                 L.scale, dstage).cpu()
    assert torch.isfinite(got).all()
    em = ((got - want).abs().max() / max(want.abs().max().item(), 1e-6)).item()
    last = q[[case.qsl[i + 1] - 1 for i in range(len(hist))]]
    arena = None if stage is None else (L.arena.stage_k, L.arena.stage_v, L.arena.owner, L.arena.sink_eff, L.recent)
    want = oatt.decode_only_ref(last, L.k_cache, L.v_cache, case.bt, case.seqs, L.scale, L.num_kv_heads, D, arena)
    got = decode.decode_only(last.to(device), kc, vc, bt, case.seqs, L.scale, dstage, L.sink, L.recent).cpu()
    assert torch.isfinite(got).all()
    ed = ((got - want).abs().max() / max(want.abs().max().item(), 1e-6)).item()
    return em, ed


def check_both_routes(device, params, bar):
    em, ed = route_errors(device, params)
    assert em <= bar and ed <= bar, (em, ed)


@pytest.mark.parametrize("params", list(decode_cases(7, 40)), ids=lambda p: f"seed{p['seed']}")
def test_decode_routes_random_shapes(device, params):
    check_both_routes(device, params, 1e-3)


# Short requests the FP32 window holds almost entirely, where the staged
# values dominate the output: the cases of the seeded sweeps above whose
# error is largest when a staged V value enters the PV pass as a single fp16
# part (5.0e-4 to 5.4e-4 of the output scale from that rounding alone, on the
# oracle).  With the V image's high and low parts they keep half the bar.
WINDOW_HEAVY = [(1234, 217), (7, 225), (7, 231), (7, 241)]


@pytest.mark.parametrize("seed,index", WINDOW_HEAVY, ids=lambda x: str(x))
def test_window_heavy_reads_keep_half_the_bar(device, seed, index):
    params = list(decode_cases(seed, index + 1))[index]
    assert params["window"]
    check_both_routes(device, params, 5e-4)


def test_decode_routes_sweep_1000(device):
    """1000 seeded random cases through both read routes: the worst error of
    each route stays within half the bar (measured worst: 3.6e-4 MTP, 2.6e-4
    DecodeOnly)."""
    worst_m = worst_d = 0.0
    for params in decode_cases(1234, 1000):
        em, ed = route_errors(device, params)
        worst_m, worst_d = max(worst_m, em), max(worst_d, ed)
    print(f"sweep worst: MTP {worst_m:.3e} DecodeOnly {worst_d:.3e}")
    assert worst_m <= 5e-4 and worst_d <= 5e-4, (worst_m, worst_d)


def write_prefill_cases(seed, n):
    rng = random.Random(seed)
    for _ in range(n):
        yield dict(bs=rng.choice([16, 32, 64, 128]), hk=rng.choice([1, 2, 4]), pages=rng.randint(1, 12),
                   frac=rng.random(), cd=rng.choice([torch.int8, torch.bfloat16]),
                   ratios=(rng.choice([0.0, 0.5, 0.92, 0.96, 1.0, 0.004]), rng.choice([0.0, 0.75, 0.92, 0.96])),
                   seed=rng.randint(0, 10 ** 6),
                   hist=rng.choice([0, 1, 31, 128, 500, rng.randint(0, 4000)]),
                   new=rng.choice([17, 33, 100, rng.randint(17, 900)]), pbs=rng.choice([32, 64, 128]),
                   window=rng.random() < 0.7, heads=rng.choice([(1, 6), (2, 12), (1, 2)]),
                   sink_pages=rng.choice([0, 1, 2]), recent=rng.choice([16, 128, 256]),
                   staging=rng.choice([512, 8192]), pseed=rng.randint(0, 10 ** 6))


@pytest.mark.parametrize("c", list(write_prefill_cases(3, 30)), ids=lambda c: f"seed{c['seed']}")
def test_write_and_prefill_random_shapes(device, c):
    bs, hk, pages, cd = c["bs"], c["hk"], c["pages"], c["cd"]
    N = max(1, int(c["frac"] * pages * bs))
    g = torch.Generator().manual_seed(c["seed"])
    k, v = synthetic.kv(N, hk, D, seed=c["seed"])
    Rk, Rv = synthetic.rotations(D, seed=c["seed"] + 1)
    kr, vr = k.float() @ Rk, v.float() @ Rv
    slots = torch.randperm(pages * bs, generator=g)[:N].to(torch.int64)
    slots[torch.rand(N, generator=g) < 0.1] = -1
    if N > 2:
        slots[1] = pages * bs + 5                     # past the cache: skipped
    raw = torch.randint(0, 256, (2, pages, bs, hk, D * (1 if cd == torch.int8 else 2)), generator=g,
                        dtype=torch.uint8)
    caches = [raw[i].view(cd).clone() for i in range(2)]
    want = [x.clone() for x in caches]
    kept = slots.clone()
    kept[kept >= pages * bs] = -1
    ostore.store_ref(orot.clip(kr, c["ratios"][0]), orot.clip(vr, c["ratios"][1]), want[0], want[1], kept)
    dc = [x.to(device) for x in caches]
    quant.quant_write_prerotated(kr.to(device), vr.to(device), dc[0], dc[1], slots.to(device),
                                 quant.clip_index(c["ratios"][0], D), quant.clip_index(c["ratios"][1], D))
    for a, b in zip(dc, want):
        assert torch.equal(a.cpu().view(torch.uint8), b.view(torch.uint8))

    hist, new, pbs = c["hist"], c["new"], c["pbs"]
    phk, phq = c["heads"]
    case = decode_case([hist], [new], bs=pbs, hk=phk, hq=phq, seed=c["pseed"], window=c["window"],
                       sink=c["sink_pages"] * pbs, recent=c["recent"], staging=c["staging"])
    L = case.layer
    q, k2, v2 = case.rotated()
    stage = L.stage() if L.window_enabled else None
    if hist > 0:
        kc, vc = ostore.full_dequant_ref(L.k_cache, L.v_cache, case.bt[0], hist, phk, D)
        if stage is not None:
            kc, vc = L.arena.splice(case.bt[0], hist, kc, vc)
    else:
        kc = vc = torch.zeros(0, phk, D)
    want = oatt.prefill_ref(q, k2, v2, kc, vc, L.scale, phk, D)
    dstage = None if stage is None else tuple(t.to(device) for t in stage)
    got = prefill.prefill_continuation(q.to(device), k2.to(device), v2.to(device), L.k_cache.to(device),
                                       L.v_cache.to(device), case.bt[0].to(device), hist, L.scale, dstage).cpu()
    assert torch.isfinite(got).all()
    assert ((got - want).abs() <= 2e-2 + 2.0 ** -8 * want.abs()).all()
