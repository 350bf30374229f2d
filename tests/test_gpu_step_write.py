"""GPU parity of the fused short-step write (oscar_step_write) and of the
decode with the output rotation in its merge (oscar_paged_decode_rotated).

Oracle: the impl-level write of oracle/forward.py on the same inputs (rotate +
sort-clip + INT2 store, restating oscar_ascend/backend.py:129-189; window
write, backend.py:439-481), rotations in fp32 on the CPU.  Tolerances,
stated:
* rotated q / k / v: |gpu - oracle| <= 1e-5 * max |oracle| per vector (fp32,
  summation order differs);
* cache bytes: the kernel rotates in fp32 like the oracle, so a code can only
  differ where a rotated value sits within fp32 rounding of a bin or clip
  edge: >= 99.99 % of code bytes identical, meta within 1 fp16 ulp, and every
  byte outside the written slots' code and meta bytes untouched;
* window: owner tags bit-exact; staged values within 1e-5 * max |oracle|; the
  fp16 operand images equal the RNE fp16 of the kernel's own staged values;
* decode with R_v^T applied: fp32 output within 1e-3 * max |oracle|, bf16
  output within 2e-2 + 2^-8 |oracle| (the bf16 contract plus half an ulp).
"""
import pytest
import torch

from oracle import attention as oatt
from oracle import format as ofmt
from oracle import store as ostore
from oscar_amd.kernels import decode, quant, staging, step
from tests.scenarios import decode_case, step_case

pytestmark = pytest.mark.gpu
D = 256


def _gpu_stage(arena, device):
    kimg, vimg = staging.stage_images(arena.stage_k, arena.stage_v)
    return (arena.stage_k.to(device), arena.stage_v.to(device), arena.owner.to(device), kimg.to(device),
            vimg.to(device))


def _run(case, device):
    """The step through the oracle (CPU) and through oscar_step_write (GPU)."""
    L = case.layer
    dev_caches = [L.k_cache.to(device), L.v_cache.to(device)]
    stage = _gpu_stage(L.arena, device) if L.arena is not None else None
    sink_eff = L.arena.sink_eff if L.arena is not None else 0
    rows = step.step_write(case.q.to(device), case.k.to(device), case.v.to(device), L.R_k.to(device),
                           L.R_v.to(device), case.md.slot_mapping.to(device), case.qsl, case.seqs, dev_caches[0],
                           dev_caches[1], quant.clip_index(L.clip_k, D), quant.clip_index(L.clip_v, D),
                           L.num_heads, L.num_kv_heads, stage, sink_eff, L.recent)
    torch.cuda.synchronize()
    L.write(case.k, case.v, case.md)          # the oracle's write of the same step
    return [r.cpu() for r in rows], [c.cpu() for c in dev_caches], stage


def _check_rotations(case, rows):
    L = case.layer
    want = (case.q.float() @ L.R_k, case.k.float() @ L.R_k, case.v.float() @ L.R_v)
    for got, w in zip(rows, want):
        scale = w.abs().amax(-1, keepdim=True)
        assert ((got - w).abs() <= 1e-5 * scale).all()


def _check_caches(case, caches):
    L = case.layer
    hk = L.num_kv_heads
    for got, want in zip(caches, (L.k_cache, L.v_cache)):
        assert got.shape == want.shape
    slots = case.md.slot_mapping
    valid = slots[slots >= 0]
    g = ostore.logical_slots(caches[0], caches[1], valid, hk, D)
    w = ostore.logical_slots(L.k_cache, L.v_cache, valid, hk, D)
    codes = torch.cat([g[..., 32:96], g[..., 96:160]], -1)
    codes_w = torch.cat([w[..., 32:96], w[..., 96:160]], -1)
    same = (codes == codes_w).float().mean().item() if codes.numel() else 1.0
    assert same >= 0.9999, f"only {same:.6f} of code bytes match"
    for j in range(4):
        mg = ofmt.f16_from_le(g[..., 2 * j:2 * j + 1], g[..., 2 * j + 1:2 * j + 2])
        mw = ofmt.f16_from_le(w[..., 2 * j:2 * j + 1], w[..., 2 * j + 1:2 * j + 2])
        assert ((mg - mw).abs() <= 2.0 ** -10 * mw.abs() + 1e-12).all(), f"meta {j}"
    # Every byte outside the written slots' code and meta ranges is untouched.
    for got, want in zip(caches, (L.k_cache, L.v_cache)):
        gb, wb = got.view(torch.uint8).clone(), want.view(torch.uint8).clone()
        gb8 = gb.reshape(-1, gb.shape[2], gb.shape[3])
        wb8 = wb.reshape(-1, wb.shape[2], wb.shape[3])
        gb8[valid] = 0
        wb8[valid] = 0
        assert torch.equal(gb, wb)


def _check_window(case, stage):
    L = case.layer
    A = L.arena
    owner = stage[2].cpu()
    assert torch.equal(owner, A.owner)
    live = A.owner >= 0
    for got, want in ((stage[0].cpu(), A.stage_k), (stage[1].cpu(), A.stage_v)):
        if live.any():
            scale = want[live].abs().max().item()
            assert (got[live] - want[live]).abs().max().item() <= 1e-5 * scale
    kref, vref = staging.stage_images(stage[0], stage[1])
    assert torch.equal(stage[3], kref) and torch.equal(stage[4], vref)


@pytest.mark.parametrize("hk,hq", [(1, 6), (2, 8)])
def test_mtp_step_with_seat_collisions(device, hk, hq):
    # Histories equal modulo the page size put every request's new tokens on
    # the same page offsets; with a 5-row arena, pages collide on seats, and
    # the later request's token must win.  One slot is skipped (-1).
    hist = [37 + 64 * i for i in range(9)]
    case = step_case(hist, [3, 1, 4, 2, 1, 4, 3, 2, 1], bs=32, seed=3, hq=hq, hk=hk, sink=32, recent=32,
                     staging=64)
    case.md.slot_mapping[4] = -1
    rows, caches, stage = _run(case, device)
    _check_rotations(case, rows)
    _check_caches(case, caches)
    _check_window(case, stage)


@pytest.mark.parametrize("cache_dtype", [torch.int8, torch.bfloat16])
def test_c2_step_and_unclipped(device, cache_dtype):
    case = step_case([24579], [4], seed=93, cache_dtype=cache_dtype)
    rows, caches, stage = _run(case, device)
    _check_rotations(case, rows)
    _check_caches(case, caches)
    _check_window(case, stage)
    case = step_case([700, 3], [16, 2], bs=64, seed=5, clip=(0.0, 0.0), sink=64, recent=128, staging=512)
    rows, caches, stage = _run(case, device)
    _check_caches(case, caches)
    _check_window(case, stage)


def test_large_step_four_vectors_per_workgroup(device):
    # 32 requests x 16 tokens: 512 tokens, the kernel groups four vectors per workgroup.
    g = torch.Generator().manual_seed(8)
    hist = torch.randint(100, 1500, (32,), generator=g).tolist()
    case = step_case(hist, [16] * 32, bs=64, seed=9, pool_pages=2048, sink=64, recent=128, staging=1024)
    rows, caches, stage = _run(case, device)
    _check_rotations(case, rows)
    _check_caches(case, caches)
    _check_window(case, stage)


def test_no_window(device):
    case = step_case([500, 9], [4, 2], bs=32, seed=11, window=False)
    rows, caches, stage = _run(case, device)
    assert stage is None
    _check_rotations(case, rows)
    _check_caches(case, caches)


def test_rejects_oversized_steps(device):
    case = step_case([10], [2], bs=32, seed=12)
    with pytest.raises(ValueError):
        step.step_write(case.q.to(device).repeat(600, 1, 1), case.k.to(device).repeat(600, 1, 1),
                        case.v.to(device).repeat(600, 1, 1), case.layer.R_k.to(device), case.layer.R_v.to(device),
                        torch.zeros(1200, dtype=torch.int64, device=device), [0, 1200], [1210],
                        case.layer.k_cache.to(device), case.layer.v_cache.to(device), -1, -1, 6, 1)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_decode_with_output_rotation(device, out_dtype):
    case = decode_case([5000, 333, 24], [4, 1, 3], bs=128, seed=13)
    L = case.layer
    q, k, v = case.rotated()
    stage = L.stage()
    want = oatt.paged_attention_ref(q, k, v, L.k_cache, L.v_cache, case.bt, case.qsl, case.seqs, L.scale,
                                    stage) @ L.R_v.t()
    dstage = tuple(t.to(device) for t in stage)
    n = q.shape[0]
    out = torch.full((n + 2, 6 * D), 7.0, dtype=out_dtype, device=device)
    decode.paged_attention(q.to(device), k.to(device), v.to(device), L.k_cache.to(device), L.v_cache.to(device),
                           case.bt.to(device), case.qsl, case.seqs, L.scale, dstage,
                           out_rotation=L.R_v.t().contiguous().to(device), out=out[:n])
    got = out.cpu().float()
    assert (got[n:] == 7.0).all(), "rows past the step's tokens must stay untouched"
    got = got[:n].view(n, 6, D)
    if out_dtype == torch.float32:
        err = (got - want).abs().max().item()
        assert err <= 1e-3 * want.abs().max().item(), f"max err {err:.3e}"
    else:
        assert ((got - want).abs() <= 2e-2 + 2.0 ** -8 * want.abs()).all()
