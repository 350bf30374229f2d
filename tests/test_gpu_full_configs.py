"""GPU parity at the full workload shapes the benchmarks are quoted on.

Every case builds its layer state with the CPU oracle's write path (rotate,
clip, INT2 store and FP32 window write of each request's history, then of the
step's new tokens), so the GPU read kernels and the oracle read the same
bytes.  Shapes:

* 32 concurrent requests x 4 MTP query tokens, histories U[2048, 16384], pages
  drawn from a shared 8192-page pool, window on (sink 128, recent 256,
  staging 8192), clip 0.96 / 0.92;
* 8 requests x 1 query token over 32768-token histories whose pages fill a
  2056-page pool (2048 history pages plus the new tokens' pages), through
  the MTP entry and through the DecodeOnly entry;
* prefill continuation of 9256 new tokens over a 15360-token INT2 history;
* the fused rotate + clip + quantize write of 65,536 bf16 tokens with random
  slots, about 1/16 of them skipped (-1).

Tolerances (stated, as in the smaller tests): fp32 decode outputs
max |gpu - oracle| <= 1e-3 * max |oracle|; prefill output elementwise
|gpu - oracle| <= 2e-2 + 2^-8 |oracle|; fused write >= 99.9 % of code bytes
identical, every dequantized value within one quantization step, meta scales
within 2 fp16 ulps, and no byte outside the valid slots touched.
"""
import pytest
import torch

from oracle import attention as oatt
from oracle import format as ofmt
from oracle import rotate as orot
from oracle import store as ostore
from oscar_amd import synthetic
from oscar_amd.kernels import decode, prefill, quant
from tests.scenarios import decode_case

pytestmark = pytest.mark.gpu

D = 256
REL_TOL = 1e-3


def _rel_err(got, want):
    return (got - want).abs().max().item() / max(want.abs().max().item(), 1e-6)


def test_concurrent_mtp_32_requests_8192_page_pool(device):
    g = torch.Generator().manual_seed(31)
    hist = torch.randint(2048, 16385, (32,), generator=g).tolist()
    case = decode_case(hist, [4] * 32, seed=32, pool_pages=8192)
    L = case.layer
    q, k, v = case.rotated()
    stage = L.stage()
    print(f"C3 shape: 32 x 4 tokens, history {min(hist)}..{max(hist)} (total {sum(hist)})", flush=True)
    want = oatt.paged_attention_ref(q, k, v, L.k_cache, L.v_cache, case.bt, case.qsl, case.seqs, L.scale, stage)
    got = decode.paged_attention(q.to(device), k.to(device), v.to(device), L.k_cache.to(device),
                                 L.v_cache.to(device), case.bt.to(device), case.qsl, case.seqs, L.scale,
                                 tuple(t.to(device) for t in stage)).cpu()
    assert torch.isfinite(got).all()
    err = _rel_err(got, want)
    assert err <= REL_TOL, f"rel err {err:.3e}"


@pytest.fixture(scope="module")
def long_context_case():
    # 8 x 32768-token histories: 2048 pages, plus one page per request for the new token.
    return decode_case([32768] * 8, [1] * 8, seed=51, pool_pages=2056)


def test_long_context_decode_8x32k_mtp_entry(device, long_context_case):
    case = long_context_case
    L = case.layer
    q, k, v = case.rotated()
    stage = L.stage()
    print("C5 decode shape through the MTP entry: 8 x 1 token over 32768", flush=True)
    want = oatt.paged_attention_ref(q, k, v, L.k_cache, L.v_cache, case.bt, case.qsl, case.seqs, L.scale, stage)
    got = decode.paged_attention(q.to(device), k.to(device), v.to(device), L.k_cache.to(device),
                                 L.v_cache.to(device), case.bt.to(device), case.qsl, case.seqs, L.scale,
                                 tuple(t.to(device) for t in stage)).cpu()
    assert torch.isfinite(got).all()
    err = _rel_err(got, want)
    assert err <= REL_TOL, f"rel err {err:.3e}"


def test_long_context_decode_8x32k_decode_only_entry(device, long_context_case):
    # The DecodeOnly read covers [0, seq) of every request (its new token was
    # written by the step, as the engine's write precedes the read).
    case = long_context_case
    L = case.layer
    q, _, _ = case.rotated()
    A = L.arena
    print("C5 decode shape through the DecodeOnly entry: 8 x 1 token over 32769", flush=True)
    want = oatt.decode_only_ref(q, L.k_cache, L.v_cache, case.bt, case.seqs, L.scale, 1, D,
                                (A.stage_k, A.stage_v, A.owner, A.sink_eff, L.recent))
    got = decode.decode_only(q.to(device), L.k_cache.to(device), L.v_cache.to(device), case.bt.to(device),
                             case.seqs, L.scale, tuple(t.to(device) for t in L.stage()), L.sink, L.recent).cpu()
    assert torch.isfinite(got).all()
    err = _rel_err(got, want)
    assert err <= REL_TOL, f"rel err {err:.3e}"


def test_prefill_continuation_15360_plus_9256(device):
    hist, new = 15360, 9256
    case = decode_case([hist], [new], seed=93)
    L = case.layer
    q, k, v = case.rotated()
    stage = L.stage()
    print(f"C4 shape: {hist} history + {new} new tokens", flush=True)
    kc, vc = ostore.full_dequant_ref(L.k_cache, L.v_cache, case.bt[0], hist, 1, D)
    kc, vc = L.arena.splice(case.bt[0], hist, kc, vc)
    want = oatt.prefill_ref(q, k, v, kc, vc, L.scale, 1, D)
    got = prefill.prefill_continuation(q.to(device), k.to(device), v.to(device), L.k_cache.to(device),
                                       L.v_cache.to(device), case.bt[0].to(device), hist, L.scale,
                                       tuple(t.to(device) for t in stage)).cpu()
    assert torch.isfinite(got).all()
    bad = ((got - want).abs() > 2e-2 + 2.0 ** -8 * want.abs()).sum().item()
    assert bad == 0, f"{bad} outputs outside the bf16 bar, max abs err {(got - want).abs().max().item():.3e}"


def test_fused_write_65536_tokens_with_skipped_slots(device):
    N, hk, bs = 65536, 1, 128
    pages = N // bs + 8
    g = torch.Generator().manual_seed(61)
    k, v = synthetic.kv(N, hk, D, seed=62)
    Rk, Rv = synthetic.rotations(D, seed=63)
    slots = torch.randperm(pages * bs, generator=g)[:N].to(torch.int64)
    slots[torch.rand(N, generator=g) < 1 / 16] = -1
    print("C5 write shape: 65536 tokens through the fused rotation entry", flush=True)
    caches = [torch.zeros(pages, bs, hk, D, dtype=torch.int8) for _ in range(2)]
    expect = [c.clone() for c in caches]
    ostore.store_ref(orot.rotate_clip(k, Rk, 0.96), orot.rotate_clip(v, Rv, 0.92), expect[0], expect[1], slots)
    dev = [c.to(device) for c in caches]
    ops = [quant.rotation_operand(R.to(device)) for R in (Rk, Rv)]
    quant.quant_write(k.to(device), v.to(device), ops[0], ops[1], dev[0], dev[1], slots.to(device),
                      quant.clip_index(0.96, D), quant.clip_index(0.92, D), hk, D)
    got_caches = [c.cpu() for c in dev]
    valid = slots[slots >= 0]
    got = ostore.logical_slots(got_caches[0], got_caches[1], valid, hk, D)
    want = ostore.logical_slots(expect[0], expect[1], valid, hk, D)
    codes = torch.cat([got[..., 32:96], got[..., 96:160]], -1)
    codes_w = torch.cat([want[..., 32:96], want[..., 96:160]], -1)
    same = (codes == codes_w).float().mean().item()
    assert same >= 0.999, f"only {same:.5f} of code bytes match"
    kg, vg = ofmt.parse_slot_bytes(got, D)
    kw, vw = ofmt.parse_slot_bytes(want, D)
    meta_g = [ofmt.f16_from_le(got[..., 2 * j:2 * j + 1], got[..., 2 * j + 1:2 * j + 2]) for j in range(4)]
    meta_w = [ofmt.f16_from_le(want[..., 2 * j:2 * j + 1], want[..., 2 * j + 1:2 * j + 2]) for j in range(4)]
    for (a, b), (sa, sb) in (((kg, kw), (meta_g[0], meta_w[0])), ((vg, vw), (meta_g[2], meta_w[2]))):
        step = torch.maximum(sa, sb)
        assert ((a - b).abs() <= step * 1.0001 + 1e-6).all()
        assert ((sa - sb).abs() <= 2 * 2.0 ** -10 * sb.abs()).all()
    for c in got_caches:
        flat = c.view(torch.uint8).reshape(pages * bs, -1)
        mask = torch.ones(pages * bs, dtype=torch.bool)
        mask[valid] = False
        assert not flat[mask].any()
