"""Pins for the attention and window oracles (oracle/attention.py,
oracle/staging.py, oracle/forward.py).

Independent checks, each able to catch a dropped term, shifted causal
boundary, transposed rotation or wrong seat hash:
  * prefill_ref vs a per-query softmax loop over its own visible prefix
    (restating tests/test_prefill.py:15-74's independent reference);
  * paged_attention_ref over a fully staged history equals plain attention on
    the original fp32 K/V (tests/test_backend.py:186-216);
  * query_layout known answer (tests/test_backend.py:215-216);
  * decode_ref vs an explicit softmax over the same INT2 data
    (tests/test_numeric.py:106-130, tolerance 1e-4);
  * split-merge closed form: merging per-chunk (out, lse) reproduces the
    single softmax;
  * window arena: persistence, recycled-page invalidation, collision winner,
    padding requests, and the stable seat sort at the fp32 boundary
    (tests/test_backend.py:76-105, 450-466);
  * the composed layer forward in the rotated domain equals original-domain
    attention over the de-rotated history (tests/test_backend.py:162-183).
"""
import math
from types import SimpleNamespace as NS

import pytest
import torch

from oracle import attention as att
from oracle import store
from oracle.forward import OracleLayer
from oracle.staging import Arena, arena_geometry, staging_order


def meta(slots, ends, seqs, bt=None):
    return NS(num_actual_tokens=len(slots), slot_mapping=torch.tensor(slots),
              query_start_loc=torch.tensor([0] + ends), actual_seq_lengths_q=ends,
              seq_lens=torch.tensor(seqs), seq_lens_cpu=torch.tensor(seqs), seq_lens_list=seqs,
              block_tables=torch.tensor(bt or [[0, 1, 2, 3]], dtype=torch.int32))


def brute_attention(q, k, v, prefix, scale):
    """Query i sees keys 0 .. prefix + i; GQA by head // group.  fp32 loops."""
    n, hq, d = q.shape
    g = hq // k.shape[1]
    out = torch.empty(n, hq, d)
    for i in range(n):
        for h in range(hq):
            kk = k[:prefix + i + 1, h // g].float()
            vv = v[:prefix + i + 1, h // g].float()
            p = torch.softmax((kk @ q[i, h].float()) * scale, 0)
            out[i, h] = p @ vv
    return out


@pytest.mark.parametrize("prefix,n", [(0, 17), (65, 1), (600, 33), (0, 600)])
def test_prefill_right_aligned_causality(prefix, n):
    g = torch.Generator().manual_seed(prefix + n)
    q = torch.randn(n, 4, 64, generator=g)
    k, v = torch.randn(prefix + n, 1, 64, generator=g), torch.randn(prefix + n, 1, 64, generator=g)
    got = att.prefill_ref(q, k[prefix:], v[prefix:], k[:prefix], v[:prefix], 0.125, 1, 64)
    torch.testing.assert_close(got, brute_attention(q, k, v, prefix, 0.125), atol=1e-5, rtol=1e-4)
    # query blocking (512 rows) must not change the result
    small = att.prefill_ref(q, k[prefix:], v[prefix:], k[:prefix], v[:prefix], 0.125, 1, 64, qblock=7)
    torch.testing.assert_close(small, got, atol=1e-6, rtol=1e-5)


def test_query_layout_known_answer():
    req, prefix, starts, ends = att.query_layout([0, 2, 5], [7, 7])
    assert req.tolist() == [0, 0, 1, 1, 1]
    assert prefix.tolist() == [5, 4] and starts.tolist() == [0, 2] and ends.tolist() == [6, 7, 5, 6, 7]
    with pytest.raises(ValueError):
        att.query_layout([0, 3], [2])


def make_cache(pages=8, bs=4, hk=1, d=64):
    return [torch.zeros(pages, bs, hk, d, dtype=torch.bfloat16) for _ in range(2)]


def test_paged_oracle_over_staged_history_equals_fp32_attention():
    g = torch.Generator().manual_seed(8)
    kc, vc = make_cache()
    oldk, oldv = torch.randn(9, 1, 64, generator=g), torch.randn(9, 1, 64, generator=g)
    slots = torch.tensor([12, 13, 14, 15, 4, 16, 17, 18, 19])     # req0: pages 3,1; req1: page 4
    store.store_ref(oldk, oldv, kc, vc, slots)
    arena = Arena.create(4, 1, 64, 4, 4, 8)
    eye = torch.eye(64)
    arena.write(oldk, oldv, meta(slots.tolist(), [5, 9], [5, 4]), eye, eye)
    q, k, v = (torch.randn(5, 2, 64, generator=g), torch.randn(5, 1, 64, generator=g),
               torch.randn(5, 1, 64, generator=g))
    bt = torch.tensor([[3, 1, 2], [4, 7, 0]])
    out = att.paged_attention_ref(q, k, v, kc, vc, bt, [0, 2, 5], [7, 7], 0.125, arena.triple())
    want = torch.cat([att.prefill_ref(q[:2], k[:2], v[:2], oldk[:5], oldv[:5], 0.125, 1, 64),
                      att.prefill_ref(q[2:], k[2:], v[2:], oldk[5:], oldv[5:], 0.125, 1, 64)])
    torch.testing.assert_close(out, want)
    # without the window the INT2 history is visibly different
    plain = att.paged_attention_ref(q, k, v, kc, vc, bt, [0, 2, 5], [7, 7], 0.125, None)
    assert (plain - want).abs().max() > 1e-3


def test_paged_oracle_matches_brute_force_on_int2_history():
    g = torch.Generator().manual_seed(9)
    kc, vc = make_cache(pages=6, bs=4, hk=2, d=32)
    hist_k, hist_v = torch.randn(11, 2, 32, generator=g), torch.randn(11, 2, 32, generator=g)
    bt = torch.tensor([[5, 0, 3]])
    pos = torch.arange(11)
    store.store_ref(hist_k, hist_v, kc, vc, bt[0][pos // 4].long() * 4 + pos % 4)
    kd, vd = store.full_dequant_ref(kc, vc, bt[0], 11, 2, 32)
    q, k, v = (torch.randn(3, 6, 32, generator=g), torch.randn(3, 2, 32, generator=g),
               torch.randn(3, 2, 32, generator=g))
    got = att.paged_attention_ref(q, k, v, kc, vc, bt, [0, 3], [14], 0.2)
    want = brute_attention(q, torch.cat([kd, k]), torch.cat([vd, v]), 11, 0.2)
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-4)


def test_decode_ref_matches_explicit_softmax():
    g = torch.Generator().manual_seed(10)
    kc, vc = make_cache(pages=3, bs=4, hk=2, d=32)
    k, v = torch.randn(7, 2, 32, generator=g) * 1.5, torch.randn(7, 2, 32, generator=g) * 1.5
    store.store_ref(k, v, kc, vc, torch.arange(7))
    q = torch.randn(1, 4, 32, generator=g)
    out, lse = att.decode_ref(q, kc, vc, torch.zeros(1, 3, dtype=torch.int32), torch.tensor([7]), 0.125, 2, 32)
    kd, vd = store.full_dequant_ref(kc, vc, torch.zeros(3, dtype=torch.int32), 7, 2, 32)
    for h in range(4):
        s = (kd[:, h // 2] @ q[0, h]) * 0.125
        torch.testing.assert_close(out[0, h], torch.softmax(s, 0) @ vd[:, h // 2], atol=1e-4, rtol=0)
        assert abs(lse[0, h].item() - torch.logsumexp(s, 0).item()) <= 1e-4


def test_merge_splits_closed_form():
    g = torch.Generator().manual_seed(11)
    s = torch.randn(300, generator=g) * 4
    v = torch.randn(300, 16, generator=g)
    bounds = [0, 1, 50, 50, 173, 300]            # includes an empty split
    outs, lses = [], []
    for a, b in zip(bounds, bounds[1:]):
        if a == b:
            outs.append(torch.zeros(16))
            lses.append(-math.inf)
            continue
        outs.append(torch.softmax(s[a:b], 0) @ v[a:b])
        lses.append(torch.logsumexp(s[a:b], 0).item())
    out, lse = att.merge_splits(torch.stack(outs), torch.tensor(lses))
    torch.testing.assert_close(out, torch.softmax(s, 0) @ v, atol=1e-5, rtol=1e-5)
    assert abs(lse - torch.logsumexp(s, 0).item()) < 1e-4
    zero, none = att.merge_splits(torch.zeros(2, 16), torch.tensor([-math.inf, -math.inf]))
    assert none == -math.inf and torch.count_nonzero(zero) == 0


# ---------------------------------------------------------------- window arena
def test_arena_geometry_known_answers():
    assert arena_geometry(4, 4, 4, 8) == (4, 1, 2, 5)
    assert arena_geometry(128, 64, 256, 8192) == (0, 0, 3, 64)
    assert arena_geometry(16, 40, 20, 0) == (32, 2, 3, 7)


def test_arena_persists_and_invalidates_recycled_pages():
    g = torch.Generator().manual_seed(12)
    arena = Arena.create(4, 1, 64, 4, 4, 8)
    eye = torch.eye(64)
    k, v = torch.randn(4, 1, 64, generator=g), torch.randn(4, 1, 64, generator=g)
    arena.write(k, v, meta([0, 1, 2, 3], [4], [4]), eye, eye)
    arena.write(k[:1] + 5, v[:1], meta([4], [1], [5]), eye, eye)
    torch.testing.assert_close(arena.stage_k[0], k)
    assert arena.owner[0].tolist() == [0, 0, 0, 0] and arena.owner[1, 0].item() == 1
    # pages 0..2 reused by middle tokens of a long request: outside both windows
    arena.write(torch.randn(12, 1, 64, generator=g), torch.randn(12, 1, 64, generator=g),
                meta(list(range(12)), [12], [100]), eye, eye)
    assert (arena.owner[0] == -1).all()


def test_arena_collision_last_writer_wins_and_padding_ignored():
    arena = Arena.create(4, 1, 64, 4, 4, 8)
    eye = torch.eye(64)
    slot = arena.rows * 4                     # same seat as slot 0
    k = torch.stack([torch.ones(1, 64), torch.full((1, 64), 7.0)])
    arena.write(k, k, meta([0, slot], [1, 2, 4], [1, 1, 1]), eye, eye)
    assert arena.owner[0, 0].item() == slot // 4
    torch.testing.assert_close(arena.stage_k[0, 0], k[1])


def test_arena_stages_rotated_unclipped_values():
    g = torch.Generator().manual_seed(13)
    R = torch.linalg.qr(torch.randn(64, 64, generator=g)).Q
    arena = Arena.create(4, 1, 64, 4, 4, 8)
    k = torch.randn(3, 1, 64, generator=g) * 10
    arena.write(k, -k, meta([5, 6, -1], [3], [3]), R, R.t())
    torch.testing.assert_close(arena.stage_k[1, 1:3], k[:2] @ R)
    torch.testing.assert_close(arena.stage_v[1, 1:3], -k[:2] @ R.t())
    assert arena.owner[1].tolist() == [-1, 1, 1, -1]


@pytest.mark.parametrize("capacity", [8192, 2 ** 24, 2 ** 24 + 2])
def test_staging_sort_exact_and_stable_at_float32_boundary(capacity):
    seats = torch.tensor([capacity - 1, 0, capacity - 2, capacity - 1, 0])
    want = torch.argsort(seats, stable=True)
    assert torch.equal(staging_order(seats, capacity), want)
    if capacity > 2 ** 24:
        # fp32 keys would merge capacity-1 and capacity-2 here
        assert not torch.equal(torch.argsort(seats.float(), stable=True), want)


# ---------------------------------------------------------------- composed layer
@pytest.mark.parametrize("window", [False, True])
def test_rotated_forward_matches_original_domain(window):
    g = torch.Generator().manual_seed(7)
    kc, vc = make_cache()
    rk = torch.linalg.qr(torch.randn(64, 64, generator=g)).Q
    rv = torch.linalg.qr(torch.randn(64, 64, generator=g)).Q
    layer = OracleLayer(kc, vc, rk, rv, 2, 1, 64, 0.125, sink=4, recent=4, staging=8 if window else 0,
                        paged_max_qlen=0)
    oldk, oldv = torch.randn(6, 1, 64, generator=g), torch.randn(6, 1, 64, generator=g)
    layer.write(oldk, oldv, meta(list(range(6)), [6], [6]))
    q, k, v = (torch.randn(3, 2, 64, generator=g), torch.randn(3, 1, 64, generator=g),
               torch.randn(3, 1, 64, generator=g))
    md = meta([6, 7, 8], [3], [9])
    kr, vr = store.full_dequant_ref(kc, vc, md.block_tables[0], 6, 1, 64)
    if window:
        kr, vr = layer.arena.splice(md.block_tables[0], 6, kr, vr)
    want = att.prefill_ref(q, k, v, kr @ rk.t(), vr @ rv.t(), 0.125, 1, 64)
    got = layer.forward(q, k, v, md)
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-4)
    # a transposed rotation on the output side is caught
    bad = att.prefill_ref(q @ rk, k @ rk, v @ rv, kr, vr, 0.125, 1, 64) @ rv
    assert (bad - got).abs().max() > 1e-2


def test_short_requests_take_paged_semantics_and_padding_stays_zero():
    g = torch.Generator().manual_seed(14)
    kc, vc = make_cache()
    rk = torch.linalg.qr(torch.randn(64, 64, generator=g)).Q
    rv = torch.linalg.qr(torch.randn(64, 64, generator=g)).Q
    layer = OracleLayer(kc, vc, rk, rv, 6, 1, 64, 0.125, sink=4, recent=4, staging=8)
    oldk, oldv = torch.randn(9, 1, 64, generator=g), torch.randn(9, 1, 64, generator=g)
    oldslots = [16, 17, 18, 19, 4, 5, 0, 1, 2]
    layer.write(oldk, oldv, meta(oldslots, [6, 9], [6, 3]))
    q, k, v = (torch.randn(6, 6, 64, generator=g), torch.randn(6, 1, 64, generator=g),
               torch.randn(6, 1, 64, generator=g))
    md = meta([6, 7, 24, 25, 3], [4, 5, 6], [10, 4, 0], bt=[[4, 1, 6], [0, 0, 0], [0, 0, 0]])
    got = layer.forward(q, k, v, md)
    want = att.paged_attention_ref(q[:5] @ rk, k[:5] @ rk, v[:5] @ rv, kc, vc, md.block_tables[:2],
                                   [0, 4, 5], [10, 4], 0.125, layer.stage()) @ rv.t()
    torch.testing.assert_close(got[:5], want, atol=1e-5, rtol=1e-4)
    assert torch.count_nonzero(got[5:]) == 0
