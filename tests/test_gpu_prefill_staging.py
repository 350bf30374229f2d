"""GPU parity of the window write kernel and kernel 3 (prefill continuation).

* Window write: owner tags bit-exact with the oracle arena
  (restating oscar_ascend/backend.py:439-481); staged fp32 values within
  1e-5 relative of the oracle's fp32 CPU rotation (summation order differs).
* The bulk step write with the window fused in (seat-winner pass + the
  quantize-write kernel's window epilogue): owner tags bit-exact, operand
  images bit-exact with the staged values, INT2 caches bit-identical to the
  window-less write; staged values are the MFMA rotation with R split into
  bf16 high + low parts (R carried to 2^-18 of each entry), within 1e-4 of
  the values' scale of the oracle's fp32 rotation.
* Prefill continuation: against the oracle dense path (history dequant +
  window splice + causal SDPA, restating backend.py:361-415 and
  kernels/decode_kernel.py:70-117) evaluated in fp32, as the reference's own
  gate does (delivery/probe_prefill.py:266-281).  The kernel rounds its MFMA
  operands to bf16; stated tolerance: the bf16 contract's max-abs 2e-2 plus
  half a bf16 ulp of the oracle value, |gpu - oracle| <= 2e-2 + 2^-8 |oracle|.
"""
from types import SimpleNamespace as NS

import pytest
import torch

from oracle import attention as oatt
from oracle import store as ostore
from oracle.staging import Arena
from oscar_amd import synthetic
from oscar_amd.kernels import prefill, quant, staging
from tests.scenarios import decode_case, metadata

pytestmark = pytest.mark.gpu
D = 256


def _gpu_arena(arena, device):
    sk = torch.zeros_like(arena.stage_k, device=device)
    sv = torch.zeros_like(sk)
    owner = torch.full(arena.owner.shape, -1, dtype=torch.int64, device=device)
    winner = staging.winner_buffer(arena.rows, arena.bs, device)
    kimg = vimg = None
    if arena.bs % 32 == 0:
        geom = (arena.rows, arena.bs, arena.stage_k.shape[2])
        kimg = torch.zeros(staging.k_image_shape(*geom), dtype=torch.float16, device=device)
        vimg = torch.zeros(staging.image_shape(*geom), dtype=torch.float16, device=device)
    return sk, sv, owner, winner, kimg, vimg


def _write_both(arena, gpu, key, value, md, Rk, Rv, device):
    arena.write(key, value, md, Rk, Rv)
    qsl, seqs = md.query_start_loc.tolist(), md.seq_lens.tolist()
    B = len(seqs)
    meta = torch.tensor(qsl + seqs, dtype=torch.int32, device=device)
    sk, sv, owner, winner, kimg, vimg = gpu
    staging.staging_write(key.to(device), value.to(device), md.slot_mapping.to(device), meta[:B + 1],
                          meta[B + 1:], B, key.shape[1], D, arena.bs, arena.sink_eff, arena.recent,
                          Rk.to(device), Rv.to(device), sk, sv, owner, winner, kimg, vimg)


@pytest.mark.parametrize("bs,sink,recent,staging_tokens", [(4, 4, 4, 8), (16, 16, 32, 64), (128, 128, 256, 8192)])
def test_window_write_matches_oracle_over_steps(device, bs, sink, recent, staging_tokens):
    hk = 1
    Rk, Rv = synthetic.rotations(D, seed=31)
    arena = Arena.create(bs, hk, D, sink, recent, staging_tokens)
    gpu = _gpu_arena(arena, device)
    g = torch.Generator().manual_seed(7)
    # Step 1: two requests prefill (hash collisions between pages), step 2: MTP
    # writes with a padding request and a skipped slot, step 3: recycled pages.
    pages = max(arena.rows * 3, 16)
    steps = []
    h0, h1 = 5 * bs + 3, 2 * bs + 1
    perm = torch.randperm(pages, generator=g).to(torch.int32)
    bt = torch.stack([perm[:8], perm[8:16]])
    s0 = synthetic.slots_for(bt[0], 0, h0, bs)
    s1 = synthetic.slots_for(bt[1], 0, h1, bs)
    steps.append((torch.cat([s0, s1]), [0, h0, h0 + h1], [h0, h1]))
    s2 = torch.cat([synthetic.slots_for(bt[0], h0, 4, bs), synthetic.slots_for(bt[1], h1, 4, bs)])
    s2[5] = -1
    steps.append((s2, [0, 4, 8, 8], [h0 + 4, h1 + 4, 1]))
    s3 = synthetic.slots_for(bt[0].flip(0), 0, 3 * bs, bs)
    steps.append((s3, [0, 3 * bs], [10 * bs]))
    for i, (slots, qsl, seqs) in enumerate(steps):
        k, v = synthetic.kv(slots.numel(), hk, D, seed=40 + i)
        md = metadata(slots, qsl, seqs, bt)
        _write_both(arena, gpu, k, v, md, Rk, Rv, device)
        torch.cuda.synchronize()
        sk, sv, owner, winner = (t.cpu() for t in gpu[:4])
        assert torch.equal(owner, arena.owner), f"owner tags differ at step {i}"
        if gpu[4] is not None:
            # The fp16 operand images track the fp32 arena exactly (same RNE cast).
            kref, vref = staging.stage_images(gpu[0], gpu[1])
            assert torch.equal(gpu[4], kref) and torch.equal(gpu[5], vref), f"operand images differ at step {i}"
        assert winner[-2].item() == i + 1 and winner[-1].item() == 0     # one epoch per call, counter cleared
        live = arena.owner >= 0
        for got, want in ((sk, arena.stage_k), (sv, arena.stage_v)):
            err = (got[live] - want[live]).abs().max().item() if live.any() else 0.0
            assert err <= 1e-5 * max(1.0, want[live].abs().max().item()), err


@pytest.mark.parametrize("bs,sink,recent,staging_tokens,hk", [(16, 16, 32, 64, 1), (128, 128, 256, 2048, 2)])
def test_fused_bulk_window_write_matches_oracle(device, bs, sink, recent, staging_tokens, hk):
    Rk, Rv = synthetic.rotations(D, seed=33)
    op_k, op_v = quant.rotation_operand(Rk.to(device)), quant.rotation_operand(Rv.to(device))
    clip_k, clip_v = quant.clip_index(0.96, D), quant.clip_index(0.92, D)
    arena = Arena.create(bs, hk, D, sink, recent, staging_tokens)
    gpu = _gpu_arena(arena, device)
    g = torch.Generator().manual_seed(11)
    pages = 4 * (2400 // bs + 2)
    caches_w = [torch.zeros(pages, bs, hk, D, dtype=torch.int8, device=device) for _ in range(2)]
    caches_p = [torch.zeros_like(c) for c in caches_w]
    perm = torch.randperm(pages, generator=g).to(torch.int32)
    T = pages // 4
    bt = torch.stack([perm[:T], perm[T:2 * T]])
    # Step 1: two prefills of 1500 + 700 tokens (fused path; pages collide in
    # the arena's few rows), step 2: a 4 + 4-token step (short path), step 3:
    # a 1200-token prefill over the first request's pages in reverse order.
    h0, h1 = 1500, 700
    steps = [(torch.cat([synthetic.slots_for(bt[0], 0, h0, bs), synthetic.slots_for(bt[1], 0, h1, bs)]),
              [0, h0, h0 + h1], [h0, h1]),
             (torch.cat([synthetic.slots_for(bt[0], h0, 4, bs), synthetic.slots_for(bt[1], h1, 4, bs)]),
              [0, 4, 8], [h0 + 4, h1 + 4]),
             (synthetic.slots_for(bt[0].flip(0), 0, 1200, bs), [0, 1200], [1200])]
    steps[0][0][17] = -1                       # a skipped slot inside the fused step
    for i, (slots, qsl, seqs) in enumerate(steps):
        k, v = synthetic.kv(slots.numel(), hk, D, seed=50 + i)
        md = metadata(slots, qsl, seqs, bt)
        arena.write(k, v, md, Rk, Rv)
        B = len(seqs)
        meta = torch.tensor(qsl + seqs, dtype=torch.int32, device=device)
        kd, vd, sd = k.to(device), v.to(device), slots.to(device)
        window = (meta[:B + 1], meta[B + 1:], B, arena.sink_eff, arena.recent, *gpu)
        quant.quant_write(kd, vd, op_k, op_v, caches_w[0], caches_w[1], sd, clip_k, clip_v, hk, D, window=window)
        quant.quant_write(kd, vd, op_k, op_v, caches_p[0], caches_p[1], sd, clip_k, clip_v, hk, D)
        torch.cuda.synchronize()
        sk, sv, owner = (t.cpu() for t in gpu[:3])
        assert torch.equal(owner, arena.owner), f"owner tags differ at step {i}"
        if gpu[4] is not None:                 # images exist for block sizes that are multiples of 32
            kref, vref = staging.stage_images(gpu[0], gpu[1])
            assert torch.equal(gpu[4], kref) and torch.equal(gpu[5], vref), f"operand images differ at step {i}"
        assert torch.equal(caches_w[0], caches_p[0]) and torch.equal(caches_w[1], caches_p[1])
        live = arena.owner >= 0
        assert live.any()
        for got, want in ((sk, arena.stage_k), (sv, arena.stage_v)):
            err = (got[live] - want[live]).abs().max().item()
            assert err <= 1e-4 * max(1.0, want[live].abs().max().item()), (i, err)


@pytest.mark.parametrize("window", [False, True])
@pytest.mark.parametrize("hist,new", [(0, 40), (1500, 300), (3000, 700)])
def test_prefill_continuation_matches_dense_oracle(device, window, hist, new):
    case = decode_case([hist], [new], seed=hist + new, window=window, sink=128, recent=256)
    L = case.layer
    q, k, v = case.rotated()
    stage = L.stage()
    if hist > 0:
        kc, vc = ostore.full_dequant_ref(L.k_cache, L.v_cache, case.bt[0], hist, 1, D)
        if stage is not None:
            kc, vc = L.arena.splice(case.bt[0], hist, kc, vc)
    else:
        kc = vc = torch.zeros(0, 1, D)
    want = oatt.prefill_ref(q, k, v, kc, vc, L.scale, 1, D)
    dstage = None if stage is None else tuple(t.to(device) for t in stage)
    got = prefill.prefill_continuation(q.to(device), k.to(device), v.to(device), L.k_cache.to(device),
                                       L.v_cache.to(device), case.bt[0].to(device), hist, L.scale, dstage)
    torch.cuda.synchronize()
    got = got.cpu()
    err = (got - want).abs().max().item()
    assert torch.isfinite(got).all()
    assert ((got - want).abs() <= 2e-2 + 2.0 ** -8 * want.abs()).all(), f"max abs err {err:.3e}"
