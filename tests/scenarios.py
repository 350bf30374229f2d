"""Seeded scenario builders shared by the parity tests.

A scenario is the state one FULL layer holds right before its attention read:
INT2 caches and FP32 window arena after a prefill write of each request's
history and the write of the current step's new tokens, all produced by the
CPU oracle's impl-level write path (oracle/forward.py), plus the step's
rotated q/k/v.
"""
from __future__ import annotations

from dataclasses import dataclass
from types import SimpleNamespace as NS

import torch

from oracle.forward import OracleLayer
from oscar_amd import synthetic

D = 256


@dataclass
class DecodeCase:
    layer: OracleLayer
    q: torch.Tensor          # [n, Hq, D] model dtype (unrotated)
    k: torch.Tensor          # [n, Hk, D]
    v: torch.Tensor
    qsl: list
    seqs: list
    bt: torch.Tensor         # [B, T] int32
    md: NS                   # metadata of the decode step

    def rotated(self):
        L = self.layer
        return (self.q.float() @ L.R_k, self.k.float() @ L.R_k, self.v.float() @ L.R_v)


def metadata(slots, qsl, seqs, bt):
    return NS(num_actual_tokens=len(slots), slot_mapping=torch.as_tensor(slots, dtype=torch.int64),
              query_start_loc=torch.tensor(qsl), actual_seq_lengths_q=list(qsl[1:]),
              seq_lens=torch.tensor(seqs), seq_lens_cpu=torch.tensor(seqs), seq_lens_list=list(seqs),
              block_tables=bt)


@dataclass
class StepCase:
    """A layer's state after its requests' history was written, and the
    step that comes next (not yet written)."""
    layer: OracleLayer
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    qsl: list
    seqs: list
    bt: torch.Tensor
    md: NS


def step_case(history, q_lens, *, hq=6, hk=1, bs=128, pool_pages=None, seed=0,
              clip=(0.96, 0.92), sink=128, recent=256, staging=8192, window=True,
              cache_dtype=torch.int8, identity_pages=False, fill_bytes=False) -> StepCase:
    """Requests with the given history lengths write their history in one
    prefill step; the returned case holds the next step's q_lens new tokens.
    fill_bytes: the caches start as random bytes (an engine's caches are not
    cleared), so slots nothing wrote hold arbitrary meta, NaN and inf included."""
    B = len(history)
    need = [(h + n + bs - 1) // bs for h, n in zip(history, q_lens)]
    pool = pool_pages or sum(need)
    if pool < sum(need):
        raise ValueError("page pool too small")
    perm = torch.arange(pool, dtype=torch.int32) if identity_pages else synthetic.page_permutation(pool, seed + 1)
    T = max(need)
    bt = torch.zeros(B, T, dtype=torch.int32)
    off = 0
    for i, n in enumerate(need):
        bt[i, :n] = perm[off:off + n]
        off += n
    Rk, Rv = synthetic.rotations(D, seed + 2)
    caches = [torch.zeros(pool, bs, hk, D, dtype=cache_dtype) for _ in range(2)]
    if fill_bytes:
        g = torch.Generator().manual_seed(seed + 77)
        for c in caches:
            raw = c.view(torch.uint8)
            raw.copy_(torch.randint(0, 256, raw.shape, generator=g, dtype=torch.uint8))
            raw.view(-1)[1::7] = 0x7C      # fp16 inf / NaN high bytes scattered over the meta
    layer = OracleLayer(caches[0], caches[1], Rk, Rv, hq, hk, D, D ** -0.5, clip[0], clip[1],
                        sink if window else 0, recent if window else 0, staging if window else 0)
    # Prefill step: every request writes its whole history.
    hk_all, hv_all, slots, qsl = [], [], [], [0]
    for i, h in enumerate(history):
        k, v = synthetic.kv(h, hk, D, seed=seed * 1000 + 17 * i + 3)
        hk_all.append(k)
        hv_all.append(v)
        slots.append(synthetic.slots_for(bt[i], 0, h, bs))
        qsl.append(qsl[-1] + h)
    if sum(history):
        md = metadata(torch.cat(slots), qsl, list(history), bt)
        layer.write(torch.cat(hk_all), torch.cat(hv_all), md)
    # The next step's new tokens.
    n_tot = sum(q_lens)
    k, v = synthetic.kv(n_tot, hk, D, seed=seed * 1000 + 999)
    q = synthetic.queries(n_tot, hq, D, seed=seed * 1000 + 998)
    qsl, slots = [0], []
    for i, (h, n) in enumerate(zip(history, q_lens)):
        slots.append(synthetic.slots_for(bt[i], h, n, bs))
        qsl.append(qsl[-1] + n)
    seqs = [h + n for h, n in zip(history, q_lens)]
    md = metadata(torch.cat(slots), qsl, seqs, bt)
    return StepCase(layer, q, k, v, qsl, seqs, bt, md)


def decode_case(history, q_lens, **kw) -> DecodeCase:
    """step_case, then the step's new tokens written (store + stage): the
    state right before the step's read."""
    c = step_case(history, q_lens, **kw)
    c.layer.write(c.k, c.v, c.md)
    return DecodeCase(c.layer, c.q, c.k, c.v, c.qsl, c.seqs, c.bt, c.md)
