"""Decode and prefill continuation with more than one kv head (grouped
query attention with group 6 and 4): every (request, kv head) item must read
its own head's slot bytes and window rows and write its own heads' outputs.
Oracles and tolerances as in the parity tests: decode 1e-3 of the output
scale (fp32), prefill 2e-2 + 2^-8 |want| (bf16 contract).
"""
import pytest
import torch

from oracle import attention as oatt
from oracle import store as ostore
from oscar_amd.kernels import decode, prefill
from tests.scenarios import decode_case

pytestmark = pytest.mark.gpu

D = 256


@pytest.mark.parametrize("hq,hk", [(12, 2), (8, 2), (8, 4)])
@pytest.mark.parametrize("window", [False, True])
def test_decode_multi_kv_heads(device, hq, hk, window):
    case = decode_case([700, 1300, 129], [4, 1, 9], hq=hq, hk=hk, seed=hq * 10 + hk, window=window)
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


@pytest.mark.parametrize("hq,hk", [(12, 2), (8, 4)])
@pytest.mark.parametrize("window", [False, True])
def test_prefill_multi_kv_heads(device, hq, hk, window):
    hist, new = 1500, 300
    case = decode_case([hist], [new], hq=hq, hk=hk, seed=hq + hk, window=window)
    L = case.layer
    q, k, v = case.rotated()
    stage = L.stage()
    kc, vc = ostore.full_dequant_ref(L.k_cache, L.v_cache, case.bt[0], hist, hk, D)
    if stage is not None:
        kc, vc = L.arena.splice(case.bt[0], hist, kc, vc)
    want = oatt.prefill_ref(q, k, v, kc, vc, L.scale, hk, D)
    dstage = None if stage is None else tuple(t.to(device) for t in stage)
    got = prefill.prefill_continuation(q.to(device), k.to(device), v.to(device), L.k_cache.to(device),
                                       L.v_cache.to(device), case.bt[0].to(device), hist, L.scale, dstage)
    torch.cuda.synchronize()
    got = got.cpu()
    assert torch.isfinite(got).all()
    assert ((got - want).abs() <= 2e-2 + 2.0 ** -8 * want.abs()).all(), (got - want).abs().max().item()
