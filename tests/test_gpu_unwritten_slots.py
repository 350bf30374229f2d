"""Slots nothing wrote may hold any bytes (an engine does not clear its
caches): the decode and the prefill continuation read whole pages and must
keep such slots out of the result.  The caches start as random bytes with
fp16 inf / NaN patterns in the meta; every request's last page is only
partly written.  Same oracles and tolerances as the parity tests:
decode 1e-3 of the output scale; prefill 2e-2 + 2^-8 |want| (bf16 contract).
"""
import pytest
import torch

from oracle import attention as oatt
from oracle import store as ostore
from oscar_amd.kernels import decode, prefill
from tests.scenarios import decode_case

pytestmark = pytest.mark.gpu

D = 256


@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("window", [False, True])
def test_decode_ignores_unwritten_slots(device, bs, window):
    case = decode_case([1500, 333], [2, 4], bs=bs, seed=5, window=window, sink=2 * bs, recent=2 * bs,
                       fill_bytes=True)
    L = case.layer
    q, k, v = case.rotated()
    stage = L.stage()
    want = oatt.paged_attention_ref(q, k, v, L.k_cache, L.v_cache, case.bt, case.qsl, case.seqs, L.scale, stage)
    dstage = None if stage is None else tuple(t.to(device) for t in stage)
    got = decode.paged_attention(q.to(device), k.to(device), v.to(device), L.k_cache.to(device),
                                 L.v_cache.to(device), case.bt.to(device), case.qsl, case.seqs, L.scale, dstage)
    torch.cuda.synchronize()
    got = got.cpu()
    assert torch.isfinite(got).all()
    err = (got - want).abs().max().item()
    assert err <= 1e-3 * want.abs().max().item(), err


@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("window", [False, True])
def test_prefill_ignores_unwritten_slots(device, bs, window):
    hist, new = 1500, 2
    case = decode_case([hist], [new], bs=bs, seed=6, window=window, sink=2 * bs, recent=2 * bs, fill_bytes=True)
    L = case.layer
    q, k, v = case.rotated()
    stage = L.stage()
    kc, vc = ostore.full_dequant_ref(L.k_cache, L.v_cache, case.bt[0], hist, 1, D)
    if stage is not None:
        kc, vc = L.arena.splice(case.bt[0], hist, kc, vc)
    want = oatt.prefill_ref(q, k, v, kc, vc, L.scale, 1, D)
    dstage = None if stage is None else tuple(t.to(device) for t in stage)
    got = prefill.prefill_continuation(q.to(device), k.to(device), v.to(device), L.k_cache.to(device),
                                       L.v_cache.to(device), case.bt[0].to(device), hist, L.scale, dstage)
    torch.cuda.synchronize()
    got = got.cpu()
    assert torch.isfinite(got).all()
    assert ((got - want).abs() <= 2e-2 + 2.0 ** -8 * want.abs()).all(), (got - want).abs().max().item()
