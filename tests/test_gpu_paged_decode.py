"""GPU parity of kernel 2 (paged MTP decode) against the CPU oracle.

Oracle: oracle.attention.paged_attention_ref (restating
oscar_ascend/kernels/paged_attention.py:41-64) on the same INT2 caches,
staging arena and rotated q/k/v.  Tolerance (fp32 output, stated):
max |gpu - oracle| <= 1e-3 * max |oracle|  (relative to the output scale).
"""
import pytest
import torch

from oracle import attention as oatt
from oscar_amd.kernels import decode
from tests.scenarios import decode_case

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3


def run_case(case, device, with_stage=True):
    L = case.layer
    q, k, v = case.rotated()
    stage = L.stage() if with_stage else None
    want = oatt.paged_attention_ref(q, k, v, L.k_cache, L.v_cache, case.bt, case.qsl, case.seqs,
                                    L.scale, stage)
    dstage = None if stage is None else tuple(t.to(device) for t in stage)
    got = decode.paged_attention(q.to(device), k.to(device), v.to(device), L.k_cache.to(device),
                                 L.v_cache.to(device), case.bt.to(device), case.qsl, case.seqs,
                                 L.scale, dstage)
    torch.cuda.synchronize()
    got = got.cpu()
    err = (got - want).abs().max().item()
    scale = want.abs().max().item()
    assert torch.isfinite(got).all()
    assert err <= REL_TOL * max(scale, 1e-6), f"max err {err:.3e} vs output scale {scale:.3e}"
    return got, want


def test_c1_single_query_identity_pages(device):
    case = decode_case([1024], [1], identity_pages=True, seed=1)
    run_case(case, device)
    run_case(case, device, with_stage=False)


def test_mixed_requests_small_pages_and_window(device):
    case = decode_case([5, 4, 0, 300, 129], [2, 3, 1, 4, 16], bs=32, seed=2, sink=32, recent=32,
                       staging=64)
    run_case(case, device)


def test_empty_request_and_long_mtp(device):
    # A request with no query tokens (qsl repeats) must be skipped.
    case = decode_case([700, 40], [16, 4], seed=3)
    L = case.layer
    q, k, v = case.rotated()
    qsl = [0, 0] + [x for x in case.qsl[1:]]
    seqs = [7] + case.seqs
    bt = torch.cat([case.bt[:1], case.bt])
    want = oatt.paged_attention_ref(q, k, v, L.k_cache, L.v_cache, bt, qsl, seqs, L.scale, L.stage())
    got = decode.paged_attention(q.to(device), k.to(device), v.to(device), L.k_cache.to(device),
                                 L.v_cache.to(device), bt.to(device), qsl, seqs, L.scale,
                                 tuple(t.to(device) for t in L.stage()))
    torch.cuda.synchronize()
    assert (got.cpu() - want).abs().max().item() <= REL_TOL * want.abs().max().item()


@pytest.mark.parametrize("cache_dtype", [torch.int8, torch.bfloat16])
def test_c2_mtp_24k_shuffled_pages(device, cache_dtype):
    case = decode_case([24579], [4], seed=93, cache_dtype=cache_dtype)
    run_case(case, device)


def test_concurrent_requests_shared_pool(device):
    g = torch.Generator().manual_seed(5)
    hist = torch.randint(2048, 6000, (8,), generator=g).tolist()
    case = decode_case(hist, [4] * 8, seed=6, pool_pages=512)
    run_case(case, device)


def test_more_requests_than_one_launch_carries(device):
    # 150 requests: the library launches them in two chunks that share one workspace.
    g = torch.Generator().manual_seed(11)
    hist = torch.randint(0, 400, (150,), generator=g).tolist()
    qlens = torch.randint(1, 5, (150,), generator=g).tolist()
    case = decode_case(hist, qlens, bs=32, seed=12, pool_pages=2400, sink=32, recent=32, staging=64)
    run_case(case, device)


def test_request_without_history_among_many_splits(device):
    """127 requests of 4 steps, a split each (635 partial slots, more than one
    round of resident workgroups), and one request whose only keys are its own
    new tokens: it has no history split to carry its fresh partial, so the
    launch gives every fresh partial a workgroup of its own."""
    hist = [512] * 64 + [0] + [512] * 63
    case = decode_case(hist, [4] * 64 + [2] + [4] * 63, bs=128, seed=14, pool_pages=700, sink=128, recent=128,
                       staging=256)
    run_case(case, device)


def test_window_disabled_matches_pure_int2(device):
    case = decode_case([3000], [4], seed=8, window=False)
    run_case(case, device, with_stage=False)


def test_invalid_layout_rejected(device):
    case = decode_case([10], [2], seed=9)
    q, k, v = case.rotated()
    with pytest.raises(ValueError):
        decode.paged_attention(q.to(device), k.to(device), v.to(device), case.layer.k_cache.to(device),
                               case.layer.v_cache.to(device), case.bt.to(device), [0, 2], [1], 0.0625)


@pytest.mark.parametrize("bs", [32, 128])
@pytest.mark.parametrize("tiles_per_split", [8, 32, 256])
def test_multi_step_splits_with_window(device, bs, tiles_per_split):
    """Workgroups that walk several 128-token steps (prefetched loads, double-buffered
    step buffers, window steps in the middle of a workgroup's range), with pages of
    32 or 128 tokens (a step spans four pages or one)."""
    g = torch.Generator().manual_seed(21 + bs)
    hist = [5000, 333, 4097] + torch.randint(200, 3000, (3,), generator=g).tolist()
    case = decode_case(hist, [4, 1, 3, 2, 4, 1], bs=bs, seed=22, sink=2 * bs, recent=256, staging=8192)
    L = case.layer
    q, k, v = case.rotated()
    stage = L.stage()
    want = oatt.paged_attention_ref(q, k, v, L.k_cache, L.v_cache, case.bt, case.qsl, case.seqs, L.scale, stage)
    dstage = tuple(t.to(device) for t in stage)
    p = decode.plan(q.to(device), k.to(device), v.to(device), L.k_cache.to(device), L.v_cache.to(device),
                    case.bt.to(device), case.qsl, case.seqs, L.scale, dstage, tiles_per_split=tiles_per_split)
    got = p.launch()
    torch.cuda.synchronize()
    got = got.cpu()
    err = (got - want).abs().max().item()
    assert torch.isfinite(got).all()
    assert err <= REL_TOL * want.abs().max().item(), f"max err {err:.3e}"


@pytest.mark.parametrize("q_len,hk,hq", [(1, 1, 6), (2, 1, 4), (1, 2, 16), (1, 1, 1)])
@pytest.mark.parametrize("window", [True, False])
def test_multi_step_small_row_items(device, q_len, hk, hq, window):
    """Launches whose items have at most 8 rows (q_len x group) and more
    128-token steps than splits (48 requests over 1500..4200-token histories)
    run the small-row score tile: parity with the oracle, window on and off."""
    g = torch.Generator().manual_seed(100 * q_len + 10 * hk + hq)
    hist = torch.randint(1500, 4200, (48,), generator=g).tolist()
    case = decode_case(hist, [q_len] * 48, seed=5 + hq, hk=hk, hq=hq, window=window, pool_pages=48 * 34 + 64,
                       bs=128)
    L = case.layer
    q, k, v = case.rotated()
    stage = L.stage() if L.window_enabled else None
    want = oatt.paged_attention_ref(q, k, v, L.k_cache, L.v_cache, case.bt, case.qsl, case.seqs, L.scale, stage)
    dstage = None if stage is None else tuple(t.to(device) for t in stage)
    got = decode.paged_attention(q.to(device), k.to(device), v.to(device), L.k_cache.to(device),
                                 L.v_cache.to(device), case.bt.to(device), case.qsl, case.seqs, L.scale,
                                 dstage).cpu()
    assert torch.isfinite(got).all()
    assert (got - want).abs().max() <= 1e-3 * max(want.abs().max().item(), 1e-6)
