"""Pin the oracle against vectors recorded from the reference implementation.

The fixtures under tests/golden/ were written by tests/golden/make_golden.py
(run in the build container, where the reference tree is readable) from the
reference's own AscendOscarAttentionBackendImpl (oscar_ascend/backend.py):

* staging_*.npz — owner tags and staged fp32 K/V after each multi-request
  window write (backend.py:418-481), including seat collisions, a padding
  request, a skipped slot (-1) and recycled pages;
* forward_*.npz — the impl-level forward (rotate + clip + INT2 store + window +
  read, backend.py:150-415) over a prefill step and three MTP steps, through
  the reference's default dense route and its paged route, with and without
  the window and clipping, plus the INT2 cache bytes after the last step;
* decode_only_*.npz — the windowed DecodeOnly read (backend.py:500-586) on
  arenas with planted gaps: a lost sink seat, an unstaged position inside the
  recent window, an unstaged last position, a request no longer than the
  sink.  The oracle's window bounds and LSE merge are replayed on the same
  caches and arena.

Tolerances: owner tags and INT2 cache bytes are compared bit-exactly; staged
fp32 vectors and attention outputs (fp32 on both sides, different summation
orders) within 1e-5 absolute.
"""
from pathlib import Path
from types import SimpleNamespace as NS

import numpy as np
import pytest
import torch

from oracle.forward import OracleLayer
from oracle.staging import Arena

GOLDEN = Path(__file__).resolve().parent / "golden"
FP32_ABS = 1e-5


def load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def metadata(slots, qsl, seqs, bt):
    qsl = [int(x) for x in qsl]
    seqs = [int(x) for x in seqs]
    return NS(num_actual_tokens=len(slots), slot_mapping=torch.as_tensor(slots, dtype=torch.int64),
              query_start_loc=torch.tensor(qsl), actual_seq_lengths_q=qsl[1:],
              seq_lens=torch.tensor(seqs), seq_lens_cpu=torch.tensor(seqs), seq_lens_list=seqs,
              block_tables=bt)


@pytest.mark.parametrize("name", ["staging_bs4.npz", "staging_bs16.npz"])
def test_window_arena_matches_reference(name):
    z = load(name)
    bs, hk, d = int(z["bs"]), z["s0_k"].shape[1], z["s0_k"].shape[2]
    arena = Arena.create(bs, hk, d, int(z["sink"]), int(z["recent"]), int(z["staging"]))
    rk, rv = torch.from_numpy(z["rk"]), torch.from_numpy(z["rv"])
    assert arena.owner.shape == z["s0_owner"].shape
    for i in range(int(z["steps"])):
        md = metadata(z[f"s{i}_slots"], z[f"s{i}_qsl"], z[f"s{i}_seqs"], torch.zeros(1, 1, dtype=torch.int32))
        arena.write(torch.from_numpy(z[f"s{i}_k"]), torch.from_numpy(z[f"s{i}_v"]), md, rk, rv)
        assert np.array_equal(arena.owner.numpy(), z[f"s{i}_owner"]), f"step {i}: owner tags differ"
        np.testing.assert_allclose(arena.stage_k.numpy(), z[f"s{i}_stage_k"], rtol=0, atol=FP32_ABS)
        np.testing.assert_allclose(arena.stage_v.numpy(), z[f"s{i}_stage_v"], rtol=0, atol=FP32_ABS)


FORWARD = [f"forward_{r}_w{w}_c{c}.npz" for r in ("dense", "paged") for w in (0, 1) for c in (0, 1)]


@pytest.mark.parametrize("name", FORWARD)
def test_forward_matches_reference(name):
    z = load(name)
    bs, pool, d, hk, hq = (int(z[k]) for k in ("bs", "pool", "d", "hk", "hq"))
    window = bool(z["window"])
    clip_k, clip_v = (float(x) for x in z["clip"])
    route = str(z["route"])
    kc = torch.zeros(pool, bs, hk, d, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    layer = OracleLayer(kc, vc, torch.from_numpy(z["rk"]), torch.from_numpy(z["rv"]), hq, hk, d, d ** -0.5,
                        clip_k, clip_v, 16 if window else 0, 16 if window else 0, 64 if window else 0,
                        paged_max_qlen=16 if route == "paged" else 0)
    bt = torch.from_numpy(z["bt"])
    for i in range(int(z["steps"])):
        md = metadata(z[f"s{i}_slots"], z[f"s{i}_qsl"], z[f"s{i}_seqs"], bt)
        out = layer.forward(torch.from_numpy(z[f"s{i}_q"]), torch.from_numpy(z[f"s{i}_k"]),
                            torch.from_numpy(z[f"s{i}_v"]), md)
        np.testing.assert_allclose(out.numpy(), z[f"s{i}_out"], rtol=0, atol=FP32_ABS,
                                   err_msg=f"{name} step {i}")
    assert np.array_equal(kc.view(torch.uint8).numpy(), z["kcache"]), "K cache bytes differ"
    assert np.array_equal(vc.view(torch.uint8).numpy(), z["vcache"]), "V cache bytes differ"


@pytest.mark.parametrize("name", ["decode_only_gaps.npz", "decode_only_bs8.npz"])
def test_decode_only_windowed_matches_reference(name):
    from oracle import attention as oatt

    z = load(name)
    d, hk, bs = int(z["d"]), int(z["hk"]), int(z["bs"])
    kc = torch.from_numpy(z["kcache"]).view(torch.bfloat16).view(-1, bs, hk, d)
    vc = torch.from_numpy(z["vcache"]).view(torch.bfloat16).view(-1, bs, hk, d)
    rk, rv = torch.from_numpy(z["rk"]), torch.from_numpy(z["rv"])
    q = torch.from_numpy(z["q"])
    seqs = [int(x) for x in z["seqs"]]
    arena = (torch.from_numpy(z["stage_k"]), torch.from_numpy(z["stage_v"]), torch.from_numpy(z["owner"]),
             int(z["sink_eff"]), int(z["recent"]))
    got = oatt.decode_only_ref(q.float() @ rk, kc, vc, torch.from_numpy(z["bt"]), seqs, d ** -0.5, hk, d,
                               arena) @ rv.t()
    want = torch.from_numpy(z["out"])
    assert (got - want).abs().max().item() <= FP32_ABS
    # A plausible misreading, taking the staged value wherever the owner tag
    # matches (the MTP read's rule), does not reproduce the reference here.
    naive = torch.zeros_like(want)
    for b, seq in enumerate(seqs):
        hk_, hv_ = oatt.history(kc, vc, torch.from_numpy(z["bt"])[b], seq, hk, d, arena[:3])
        qr = (q[b].float() @ rk).view(hk, -1, d)                     # [Hk, group, D]
        p = torch.softmax(torch.einsum("kgd,tkd->kgt", qr, hk_) * d ** -0.5, -1)
        naive[b] = torch.einsum("kgt,tkd->kgd", p, hv_).reshape(-1, d) @ rv.t()
    assert (naive - want).abs().max().item() > 1e-3
