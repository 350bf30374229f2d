"""GPU parity of the impl-level forward (write + window + read) against the
oracle composition (oracle/forward.py, restating oscar_ascend/backend.py:150-189,
239-319, 361-415, 418-498).

The fused write rotates on MFMA, so INT2 codes may differ from the oracle's at
bin edges.  The oracle runs in fp32 (the model's bf16 inputs upcast exactly),
as the reference's own gate does (delivery/probe_prefill.py:266-281); the
impl's output is bf16.  Stated tolerance: the bf16 contract's max-abs 2e-2
plus half a bf16 ulp of the oracle value,
    |gpu - oracle| <= 2e-2 + 2^-8 * |oracle|   (elementwise).
"""
import dataclasses
from types import SimpleNamespace as NS

import pytest
import torch

from oracle.forward import OracleLayer
from oracle.staging import Arena
from oscar_amd import synthetic
from oscar_amd.backend import OscarAttentionBackendImpl, metadata_batch_lists
from tests.scenarios import metadata

pytestmark = pytest.mark.gpu
D = 256
BF16_ABS = 2e-2
BF16_HALF_ULP = 2.0 ** -8


def within_bf16(got, want):
    return bool(((got - want).abs() <= BF16_ABS + BF16_HALF_ULP * want.abs()).all())


def make_impl(hq=6, hk=1, clip=(0.96, 0.92), sink=128, recent=256, staging=8192):
    impl = OscarAttentionBackendImpl.__new__(OscarAttentionBackendImpl)
    impl.head_size, impl.num_kv_heads, impl.num_heads = D, hk, hq
    impl.scale = D ** -0.5
    impl.key_cache = impl.value_cache = None
    impl._oscar_setup()
    impl._oscar_cfg = dataclasses.replace(impl._oscar, k_clip_ratio=clip[0], v_clip_ratio=clip[1],
                                          sink_tokens=sink, recent_tokens=recent, staging_tokens=staging)
    return impl


def run_steps(device, steps, pool, bs=128, hq=6, hk=1, seed=0, **cfg):
    """steps: list of (q_lens per request, seq_lens per request)."""
    impl = make_impl(hq, hk, **cfg)
    Rk, Rv = synthetic.rotations(D, seed + 1)
    layer = NS(layer_name="model.layers.3.self_attn.attn", _oscar_rots=(Rk.to(device), Rv.to(device)))
    caches = [torch.zeros(pool, bs, hk, D, dtype=torch.int8, device=device) for _ in range(2)]
    olayer = OracleLayer(torch.zeros(pool, bs, hk, D, dtype=torch.int8), torch.zeros(pool, bs, hk, D, dtype=torch.int8),
                         Rk, Rv, hq, hk, D, impl.scale, impl._oscar.k_clip_ratio, impl._oscar.v_clip_ratio,
                         impl._oscar.sink_tokens, impl._oscar.recent_tokens, impl._oscar.staging_tokens)
    perm = synthetic.page_permutation(pool, seed + 2)
    B = len(steps[0][0])
    per = pool // B
    bt = torch.stack([perm[i * per:(i + 1) * per] for i in range(B)])
    outs = []
    for si, (q_lens, seqs) in enumerate(steps):
        n = sum(q_lens)
        k, v = synthetic.kv(n, hk, D, seed=seed * 100 + si)
        q = synthetic.queries(n, hq, D, seed=seed * 100 + 50 + si)
        qsl = [0]
        slots = []
        for i, (ql, s) in enumerate(zip(q_lens, seqs)):
            qsl.append(qsl[-1] + ql)
            slots.append(synthetic.slots_for(bt[i], s - ql, ql, bs))
        md = metadata(torch.cat(slots), qsl, seqs, bt)
        mdd = NS(**{**vars(md), "slot_mapping": md.slot_mapping.to(device), "block_tables": bt.to(device)})
        out = impl.forward(layer, q.to(device), k.to(device), v.to(device), caches, mdd,
                           output=torch.empty(n, hq, D, dtype=torch.bfloat16, device=device))
        torch.cuda.synchronize()
        want = olayer.forward(q.float(), k.float(), v.float(), md)
        outs.append((out.cpu().float(), want.float()))
    return impl, layer, caches, olayer, outs


def test_prefill_then_mtp_steps_match_oracle(device):
    steps = [([600], [600]), ([4], [604]), ([4], [608]), ([3], [611])]
    _, _, _, _, outs = run_steps(device, steps, pool=8, seed=1)
    for i, (got, want) in enumerate(outs):
        err = (got - want).abs().max().item()
        assert within_bf16(got, want), f"step {i}: max abs err {err:.3e}"


def test_mixed_batch_long_and_short_requests(device):
    steps = [([300, 40], [300, 40]), ([2, 20], [302, 60]), ([4, 1], [306, 61])]
    _, _, _, _, outs = run_steps(device, steps, pool=16, seed=2)
    for i, (got, want) in enumerate(outs):
        assert within_bf16(got, want), i


def test_window_disabled(device):
    steps = [([200], [200]), ([4], [204])]
    _, _, _, _, outs = run_steps(device, steps, pool=4, seed=3, staging=0)
    for got, want in outs:
        assert within_bf16(got, want)


def test_padding_rows_stay_zero(device):
    impl = make_impl()
    Rk, Rv = synthetic.rotations(D, 9)
    layer = NS(layer_name="model.layers.0.self_attn.attn", _oscar_rots=(Rk.to(device), Rv.to(device)))
    caches = [torch.zeros(4, 128, 1, D, dtype=torch.int8, device=device) for _ in range(2)]
    q = synthetic.queries(6, 6, D, 1).to(device)
    k, v = (t.to(device) for t in synthetic.kv(6, 1, D, 2))
    bt = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32)
    md = metadata(torch.tensor([0, 1, 2, 3, 256]), [0, 4, 5], [4, 1], bt)
    md.num_actual_tokens = 5
    md.slot_mapping = torch.tensor([0, 1, 2, 3, 256, -1], device=device)
    md.block_tables = bt.to(device)
    out = impl.forward(layer, q, k, v, caches, md, output=torch.full((6, 6, D), 7.0, dtype=torch.bfloat16, device=device))
    torch.cuda.synchronize()
    assert torch.count_nonzero(out[5]) == 0
    assert torch.isfinite(out.float()).all()
