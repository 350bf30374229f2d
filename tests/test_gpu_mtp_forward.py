"""GPU parity of oscar_mtp_forward, the one-call forward of a short step.

The entry enqueues oscar_step_write and oscar_paged_decode_rotated with the
arguments its two structs hold, so on the same state it must give exactly
what the two entries give when called one after the other (both are checked
against the oracle in test_gpu_step_write.py): output, caches, window arena
and its images bit-exact.  The C2 case is also checked against the oracle
directly (the reference's write then read, oscar_ascend/backend.py:150-189,
273-303, 439-481): bf16 output within 2e-2 + 2^-8 |oracle|.  The step half is
shared by the layers of a step: two layers through one MtpStep give what
each gives alone.
"""
import pytest
import torch

from oracle import attention as oatt
from oscar_amd.kernels import _lib, decode, quant, staging, step
from tests.scenarios import step_case

pytestmark = pytest.mark.gpu
D = 256


def _state(case, device):
    """Device copies of the layer's caches and arena (stage_k, stage_v, owner, images)."""
    L = case.layer
    caches = (L.k_cache.to(device), L.v_cache.to(device))
    stage = None
    if L.arena is not None:
        kimg, vimg = staging.stage_images(L.arena.stage_k, L.arena.stage_v)
        stage = tuple(t.to(device) for t in (L.arena.stage_k, L.arena.stage_v, L.arena.owner, kimg, vimg))
    return caches, stage


def _inputs(case, device):
    L = case.layer
    q = case.q.to(device).reshape(case.q.shape[0], -1)
    k = case.k.to(device).reshape(case.k.shape[0], -1)
    v = case.v.to(device).reshape(case.v.shape[0], -1)
    rots = tuple(r.to(device).contiguous() for r in (L.R_k, L.R_v, L.R_v.t()))
    return q, k, v, rots


def _two_calls(case, device, out_dtype):
    L = case.layer
    caches, stage = _state(case, device)
    q, k, v, (rk, rv, rvt) = _inputs(case, device)
    sink_eff = L.arena.sink_eff if L.arena is not None else 0
    qr, kr, vr = step.step_write(q, k, v, rk, rv, case.md.slot_mapping.to(device), case.qsl, case.seqs, caches[0],
                                 caches[1], quant.clip_index(L.clip_k, D), quant.clip_index(L.clip_v, D),
                                 L.num_heads, L.num_kv_heads, stage, sink_eff, L.recent)
    n = q.shape[0]
    out = torch.full((n + 3, L.num_heads * D), 5.0, dtype=out_dtype, device=device)
    decode.paged_attention(qr, kr, vr, caches[0], caches[1], case.bt.to(device), case.qsl, case.seqs, L.scale, stage,
                           out_rotation=rvt, out=out[:n])
    return out, caches, stage


def _layer(case, device, caches, stage):
    L = case.layer
    _, _, _, (rk, rv, rvt) = _inputs(case, device)
    sink_eff = L.arena.sink_eff if L.arena is not None else 0
    return step.MtpLayer(rk, rv, rvt, caches[0], caches[1], L.num_heads, L.num_kv_heads,
                         quant.clip_index(L.clip_k, D), quant.clip_index(L.clip_v, D), L.scale, stage, sink_eff,
                         L.recent)


def _one_call(case, device, out_dtype, st=None):
    L = case.layer
    caches, stage = _state(case, device)
    q, k, v, _ = _inputs(case, device)
    stream = _lib.stream_handle(torch.device(device))
    if st is None:
        st = step.mtp_step(case.qsl, case.seqs, q.shape[0], case.md.slot_mapping.to(device), case.bt.to(device),
                           L.num_heads, L.num_kv_heads, D, 16, torch.device(device), stream, reuse=False)
    n = q.shape[0]
    out = torch.full((n + 3, L.num_heads * D), 5.0, dtype=out_dtype, device=device)
    step.mtp_forward(_layer(case, device, caches, stage), st, q, k, v, out, stream)
    return out, caches, stage


def _assert_same(a, b):
    out_a, caches_a, stage_a = a
    out_b, caches_b, stage_b = b
    torch.cuda.synchronize()
    assert torch.equal(out_a.view(torch.uint8) if out_a.dtype == torch.bfloat16 else out_a,
                       out_b.view(torch.uint8) if out_b.dtype == torch.bfloat16 else out_b)
    for x, y in zip(caches_a, caches_b):
        assert torch.equal(x.view(torch.uint8), y.view(torch.uint8))
    assert (stage_a is None) == (stage_b is None)
    if stage_a is not None:
        for x, y in zip(stage_a, stage_b):
            assert torch.equal(x, y)


CASES = {
    "c2": dict(history=[24579], q_lens=[4], seed=93),
    "collisions": dict(history=[37 + 64 * i for i in range(9)], q_lens=[3, 1, 4, 2, 1, 4, 3, 2, 1], bs=32, seed=3,
                       hq=8, hk=2, sink=32, recent=32, staging=64),
    "no_window": dict(history=[500, 9], q_lens=[4, 2], bs=32, seed=11, window=False),
    "long_requests": dict(history=[700, 3, 4000], q_lens=[16, 2, 9], bs=64, seed=5, clip=(0.0, 0.0), sink=64,
                          recent=128, staging=512),
}


@pytest.mark.parametrize("name", sorted(CASES))
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_matches_the_two_entries(device, name, out_dtype):
    kw = CASES[name]
    case = step_case(kw["history"], kw["q_lens"], **{k: v for k, v in kw.items() if k not in ("history", "q_lens")})
    _assert_same(_two_calls(case, device, out_dtype), _one_call(case, device, out_dtype))


def test_c2_against_the_oracle(device):
    case = step_case([24579], [4], seed=93)
    out, _, _ = _one_call(case, device, torch.bfloat16)
    L = case.layer
    L.write(case.k, case.v, case.md)                 # the oracle's write of the same step
    q, k, v = (case.q.float() @ L.R_k, case.k.float() @ L.R_k, case.v.float() @ L.R_v)
    want = oatt.paged_attention_ref(q, k, v, L.k_cache, L.v_cache, case.bt, case.qsl, case.seqs, L.scale,
                                    L.stage()) @ L.R_v.t()
    n = q.shape[0]
    got = out.cpu().float()
    assert (got[n:] == 5.0).all(), "rows past the step's tokens must stay untouched"
    got = got[:n].view(n, L.num_heads, D)
    assert ((got - want).abs() <= 2e-2 + 2.0 ** -8 * want.abs()).all()


def test_step_half_shared_by_layers(device):
    # Two layers (their own caches, rotations, arena, seeds) of one step
    # through a single MtpStep give what each gives with a step of its own.
    a = step_case([24579], [4], seed=93, identity_pages=True)
    b = step_case([24579], [4], seed=94, identity_pages=True)
    assert torch.equal(a.md.slot_mapping, b.md.slot_mapping) and torch.equal(a.bt, b.bt)
    dev = torch.device(device)
    stream = _lib.stream_handle(dev)
    slots, bt = a.md.slot_mapping.to(device), a.bt.to(device)
    st = step.mtp_step(a.qsl, a.seqs, 4, slots, bt, 6, 1, D, 16, dev, stream)
    assert step.mtp_step(a.qsl, a.seqs, 4, slots, bt, 6, 1, D, 16, dev, stream) is st
    assert step.mtp_step(a.qsl, a.seqs, 4, slots.clone(), bt, 6, 1, D, 16, dev, stream) is not st
    assert step.mtp_step(a.qsl, [a.seqs[0] + 1], 4, slots, bt, 6, 1, D, 16, dev, stream) is not st
    assert step.mtp_step([0, 17], [40], 17, slots, bt, 6, 1, D, 16, dev, stream) is None   # q_len > 16
    want_a = _one_call(a, device, torch.bfloat16)
    want_b = _one_call(b, device, torch.bfloat16)
    got_a = _one_call(a, device, torch.bfloat16, st)
    got_b = _one_call(b, device, torch.bfloat16, st)
    _assert_same(want_a, got_a)
    _assert_same(want_b, got_b)


def test_mismatched_halves_enqueue_nothing(device):
    case = step_case([300], [2], bs=32, seed=21, hq=8, hk=2)
    caches, stage = _state(case, device)
    before = [c.clone() for c in caches]
    q, k, v, _ = _inputs(case, device)
    dev = torch.device(device)
    stream = _lib.stream_handle(dev)
    st = step.mtp_step(case.qsl, case.seqs, 2, case.md.slot_mapping.to(device), case.bt.to(device), 6, 1, D, 16, dev,
                       stream, reuse=False)
    out = torch.zeros(2, 8 * D, dtype=torch.bfloat16, device=device)
    with pytest.raises(_lib.OscarKernelError, match="invalid argument"):
        step.mtp_forward(_layer(case, device, caches, stage), st, q, k, v, out, stream)
    torch.cuda.synchronize()
    for c, c0 in zip(caches, before):
        assert torch.equal(c.view(torch.uint8), c0.view(torch.uint8))
    assert (out == 0).all()
