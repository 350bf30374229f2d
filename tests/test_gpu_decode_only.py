"""GPU parity of the DecodeOnly read (oscar_decode_only) against the oracle
(oracle.attention.decode_only_ref, restating oscar_ascend/backend.py:321-358,
500-586): INT2 middle, FP32 sink when fully staged and the staged run ending at
the last position, merged by log-sum-exp.  The library instead runs one pass
in which a staged value replaces the INT2 one only inside those segments.
Tolerance (fp32 output, stated): max |gpu - oracle| <= 1e-3 * max |oracle|;
impl-level (bf16 output): |gpu - oracle| <= 2e-2 + 2^-8 |oracle| elementwise.
The kernel takes q and staged keys as fp16 high + low operand pairs (both to
about 2^-22); staged values and the probabilities are single fp16 operands,
with the row sums taken over the same rounded weights.  What remains is the
fp16 rounding of a staged value (at most 2^-11 of it), largest when one staged
token dominates a short request: the worst of a 150-case random sweep of MTP
and DecodeOnly reads is 0.56e-3 of the output maximum, on such requests.
"""
from types import SimpleNamespace as NS

import pytest
import torch

from oracle import attention as oatt
from oscar_amd.backend import OscarAttentionState
from oscar_amd.kernels import decode
from tests.scenarios import decode_case
from tests.test_gpu_backend import run_steps, within_bf16

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3
D = 256


def run_case(case, device, window=True, plant=()):
    L = case.layer
    bs = L.k_cache.shape[1]
    if plant:
        for b, pos in plant:
            page = int(case.bt[b][pos // bs])
            L.arena.owner[page % L.arena.rows, pos % bs] = -1
    q, _, _ = case.rotated()
    hk = L.num_kv_heads
    arena = (L.arena.stage_k, L.arena.stage_v, L.arena.owner, L.arena.sink_eff, L.recent) if window else None
    want = oatt.decode_only_ref(q, L.k_cache, L.v_cache, case.bt, case.seqs, L.scale, hk, D, arena)
    stage = tuple(t.to(device) for t in L.stage()) if window else None
    got = decode.decode_only(q.to(device), L.k_cache.to(device), L.v_cache.to(device), case.bt.to(device),
                             case.seqs, L.scale, stage, L.sink, L.recent)
    torch.cuda.synchronize()
    got = got.cpu()
    assert torch.isfinite(got).all()
    err = (got - want).abs().max().item()
    assert err <= REL_TOL * want.abs().max().item(), f"max err {err:.3e}"


@pytest.mark.parametrize("hk,hq", [(1, 6), (2, 12)])
def test_mixed_requests_planted_gaps(device, hk, hq):
    hist = [300, 5, 1000, 129, 63, 2047]
    case = decode_case(hist, [1] * len(hist), bs=32, seed=41, sink=64, recent=64, staging=256, hk=hk, hq=hq,
                       pool_pages=sum((h + 32) // 32 for h in hist) + 5)
    run_case(case, device, plant=[(0, 1), (2, case.seqs[2] - 5), (5, case.seqs[5] - 1)])


@pytest.mark.parametrize("hq,sink,recent", [(6, 256, 256), (16, 64, 64), (6, 64, 320), (6, 288, 64)])
def test_planted_gaps_on_both_bounds_paths(device, hq, sink, recent):
    """The small-row split kernel finds the window bounds itself when the
    group has at most 8 heads and the sink and recent spans are at most 256
    positions (the first case, at that limit); more heads per group (the
    cooperative kernel) or a longer span keep the separate bounds kernel."""
    hist = [300, 5, 1000, 129, 63, 2047]
    case = decode_case(hist, [1] * len(hist), bs=32, seed=48, sink=sink, recent=recent, staging=4096, hk=1, hq=hq,
                       pool_pages=sum((h + 32) // 32 for h in hist) + 5)
    run_case(case, device, plant=[(0, 1), (2, case.seqs[2] - 5), (5, case.seqs[5] - 1), (5, case.seqs[5] - 200)])


@pytest.mark.parametrize("bs", [64, 128])
def test_default_window_long_histories(device, bs):
    hist = [5000, 333, 4097, 24, 128]
    case = decode_case(hist, [1] * len(hist), bs=bs, seed=42, sink=128, recent=256, staging=8192)
    run_case(case, device)


def test_window_disabled_is_pure_int2(device):
    case = decode_case([3000, 17], [1, 1], bs=128, seed=43, window=False)
    run_case(case, device, window=False)


def test_unwritten_slots_hold_random_bytes(device):
    case = decode_case([900, 77], [1, 1], bs=64, seed=44, sink=64, recent=128, staging=1024, fill_bytes=True)
    run_case(case, device)


def test_more_requests_than_one_launch_carries(device):
    g = torch.Generator().manual_seed(45)
    hist = torch.randint(0, 300, (150,), generator=g).tolist()
    case = decode_case(hist, [1] * 150, bs=32, seed=46, pool_pages=1700, sink=32, recent=32, staging=64)
    run_case(case, device)


def test_c2_shape_history(device):
    case = decode_case([24579], [1], bs=128, seed=93)
    run_case(case, device)


def test_impl_forward_without_fresh_kv(device):
    """forward(key=None, value=None) in the DecodeOnly state reads through the
    caches and the arena the earlier steps wrote (backend.py:304-307)."""
    steps = [([600, 40], [600, 40]), ([1, 1], [601, 41])]
    impl, layer, caches, olayer, outs = run_steps(device, steps, pool=24, bs=64, seed=7, sink=64, recent=128,
                                                  staging=512)
    for got, want in outs:
        assert within_bf16(got, want)
    q = torch.randn(2, 6, D, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    seqs = [601, 41]
    md = NS(num_actual_tokens=2, query_start_loc=torch.tensor([0, 1, 2]), actual_seq_lengths_q=[1, 2],
            seq_lens=torch.tensor(seqs), seq_lens_cpu=torch.tensor(seqs), seq_lens_list=seqs,
            attn_state=OscarAttentionState.DecodeOnly)
    bt = impl_block_table(olayer, pool=24, seed=7)
    md.block_tables = bt.to(device)
    out = impl.forward(layer, q.to(device), None, None, caches, md,
                       output=torch.empty(2, 6 * D, dtype=torch.bfloat16, device=device))
    torch.cuda.synchronize()
    A = olayer.arena
    want = oatt.decode_only_ref(q.float() @ olayer.R_k, olayer.k_cache, olayer.v_cache, bt, seqs, olayer.scale, 1,
                                D, (A.stage_k, A.stage_v, A.owner, A.sink_eff, olayer.recent)) @ olayer.R_v.t()
    assert within_bf16(out.cpu().float().view(2, 6, D), want)
    md.attn_state = OscarAttentionState.ChunkedPrefill
    with pytest.raises(NotImplementedError):
        impl.forward(layer, q.to(device), None, None, caches, md,
                     output=torch.empty(2, 6 * D, dtype=torch.bfloat16, device=device))


def impl_block_table(olayer, pool, seed):
    from oscar_amd import synthetic

    perm = synthetic.page_permutation(pool, seed + 2)
    per = pool // 2
    return torch.stack([perm[i * per:(i + 1) * per] for i in range(2)])


@pytest.mark.parametrize("cache_dtype", [torch.int8, torch.bfloat16])
def test_four_kv_heads_and_both_cache_geometries(device, cache_dtype):
    hist = [1500, 70, 640]
    case = decode_case(hist, [1] * len(hist), bs=64, seed=47, hk=4, hq=8, sink=64, recent=128, staging=1024,
                       cache_dtype=cache_dtype)
    run_case(case, device, plant=[(2, case.seqs[2] - 3)])
