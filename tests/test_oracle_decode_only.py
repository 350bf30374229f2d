"""Pins for the DecodeOnly oracle (oracle/attention.py: window_bounds,
decode_only_ref), restating backend.py:321-358, 500-586.

The oracle attends two segments and merges them by log-sum-exp; the checks
use other formulations:
  * window_bounds known answers on a hand-built arena (active sink, a gap in
    the tail, an unstaged last position, an unstaged sink seat, a request no
    longer than the sink, recent = 0);
  * decode_only_ref equals one softmax over the whole history in which each
    position takes its staged value exactly where a vectorised bounds rule
    (computed here with tensor ops, not the oracle's scan) says so;
  * with staged values equal to the INT2 values the windowed and plain reads
    agree (any error in the merge weights shows);
  * without an arena it is decode_ref over [0, seq).
"""
import pytest
import torch

from oracle import attention as att
from oracle import store
from tests.scenarios import decode_case


def tiny_arena():
    bs, rows = 4, 8
    bt = torch.tensor([5, 2, 7, 1], dtype=torch.int32)
    owner = torch.full((rows, bs), -1, dtype=torch.int64)
    for p in range(16):
        page = int(bt[p // bs])
        owner[page % rows, p % bs] = page
    return bt, owner, bs


def test_window_bounds_known_answers():
    bt, owner, bs = tiny_arena()
    assert att.window_bounds(owner, bt, 14, bs, 4, 6) == (True, 8)
    o = owner.clone()
    o[7 % 8, 10 % 4] = -1                                     # position 10 (page 7) unstaged
    assert att.window_bounds(o, bt, 14, bs, 4, 6) == (True, 11)
    o = owner.clone()
    o[1 % 8, 13 % 4] = -1                                     # the last position unstaged
    assert att.window_bounds(o, bt, 14, bs, 4, 6) == (True, 14)
    o = owner.clone()
    o[5, 2] = -1                                              # a sink seat unstaged: no sink
    assert att.window_bounds(o, bt, 14, bs, 4, 6) == (False, 8)
    assert att.window_bounds(o, bt, 14, bs, 4, 12) == (False, 3)
    assert att.window_bounds(owner, bt, 4, bs, 4, 6) == (False, 0)     # not longer than the sink
    assert att.window_bounds(owner, bt, 14, bs, 4, 0) == (True, 14)    # recent = 0: no tail
    assert att.window_bounds(owner, bt, 14, bs, 0, 6) == (False, 8)    # no sink pages


def brute_decode_only(q, kc, vc, bt, seqs, scale, hk, D, arena):
    sk, sv, owner, sink_eff, recent = arena
    bs, rows = kc.shape[1], owner.shape[0]
    g = q.shape[1] // hk
    out = torch.zeros(q.shape, dtype=torch.float64)
    for b, seq in enumerate(seqs):
        pos = torch.arange(seq)
        pages = bt[b][pos // bs].long()
        k, v = store.dequant_split_ref(kc.view(torch.uint8), vc.view(torch.uint8), pages, pos % bs, hk, D)
        seat_r, seat_c = pages % rows, pos % bs
        staged = owner[seat_r, seat_c] == pages
        head = sink_eff if sink_eff > 0 and seq > sink_eff and bool(staged[:sink_eff].all()) else 0
        t0 = max(seq - recent, head)
        bad = torch.nonzero(~staged[t0:seq]).flatten()
        cut = t0 + int(bad.max()) + 1 if bad.numel() else t0
        use = (staged & ((pos < head) | (pos >= cut))).view(-1, 1, 1)
        k = torch.where(use, sk[seat_r, seat_c], k).double().repeat_interleave(g, 1)
        v = torch.where(use, sv[seat_r, seat_c], v).double().repeat_interleave(g, 1)
        s = torch.einsum("hd,lhd->hl", q[b].double(), k) * scale
        out[b] = torch.einsum("hl,lhd->hd", torch.softmax(s, -1), v)
    return out


def layer_arena(case):
    L = case.layer
    return (L.arena.stage_k, L.arena.stage_v, L.arena.owner, L.arena.sink_eff, L.recent)


@pytest.mark.parametrize("bs,sink,recent,staging", [(32, 64, 64, 256), (16, 32, 40, 64), (64, 64, 100, 128)])
def test_decode_only_oracle_matches_one_softmax(bs, sink, recent, staging):
    hist = [300, 5, 1000, 129, 63]
    case = decode_case(hist, [1] * len(hist), bs=bs, seed=31, sink=sink, recent=recent, staging=staging,
                       pool_pages=sum((h + bs) // bs for h in hist) + 7, hk=2, hq=6)
    L = case.layer
    q, _, _ = case.rotated()
    arena = layer_arena(case)
    # plant an unstaged sink seat in request 0 and a gap in request 2's tail
    for b, pos in ((0, 1), (2, case.seqs[2] - 5)):
        page = int(case.bt[b][pos // bs])
        L.arena.owner[page % L.arena.rows, pos % bs] = -1
    got = att.decode_only_ref(q, L.k_cache, L.v_cache, case.bt, case.seqs, L.scale, 2, 256, arena)
    want = brute_decode_only(q, L.k_cache, L.v_cache, case.bt, case.seqs, L.scale, 2, 256, arena)
    assert (got.double() - want).abs().max() <= 1e-5 * want.abs().max()
    assert not att.window_bounds(L.arena.owner, case.bt[0].long(), case.seqs[0], bs, L.arena.sink_eff, recent)[0]
    # the planted gap bounds the staged tail (seat collisions may shorten it further)
    assert att.window_bounds(L.arena.owner, case.bt[2].long(), case.seqs[2], bs, L.arena.sink_eff,
                             recent)[1] >= case.seqs[2] - 4


def test_staged_int2_values_make_the_window_invisible():
    bs = 32
    case = decode_case([700, 90], [1, 1], bs=bs, seed=32, sink=64, recent=96, staging=512)
    L = case.layer
    q, _, _ = case.rotated()
    A = L.arena
    k8, v8 = L.k_cache.view(torch.uint8), L.v_cache.view(torch.uint8)
    seated = torch.nonzero(A.owner >= 0)
    for r, c in seated.tolist():
        page = int(A.owner[r, c])
        k, v = store.dequant_split_ref(k8, v8, torch.tensor([page]), torch.tensor([c]), 1, 256)
        A.stage_k[r, c], A.stage_v[r, c] = k[0], v[0]
    plain = att.decode_only_ref(q, L.k_cache, L.v_cache, case.bt, case.seqs, L.scale, 1, 256)
    windowed = att.decode_only_ref(q, L.k_cache, L.v_cache, case.bt, case.seqs, L.scale, 1, 256, layer_arena(case))
    assert (plain - windowed).abs().max() <= 1e-5 * plain.abs().max()


def test_without_arena_it_is_decode_ref():
    case = decode_case([257, 31], [1, 1], bs=32, seed=33, window=False)
    L = case.layer
    q, _, _ = case.rotated()
    got = att.decode_only_ref(q, L.k_cache, L.v_cache, case.bt, case.seqs, L.scale, 1, 256)
    no_stage = (torch.zeros(1, 32, 1, 256), torch.zeros(1, 32, 1, 256), torch.full((1, 32), -1), 0, 0)
    want = brute_decode_only(q, L.k_cache, L.v_cache, case.bt, case.seqs, L.scale, 1, 256, no_stage)
    assert (got.double() - want).abs().max() <= 1e-5 * want.abs().max()
