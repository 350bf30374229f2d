"""Oracle: impl-level forward (write, stage, read) of one FULL-attention layer.

Restates the composition in AscendOscarAttentionBackendImpl.forward /
do_kv_cache_update / _prefill_attention (oscar_ascend/backend.py:150-189,
239-319, 361-415).  Test infrastructure only; every tensor stays on the CPU.

Routing mirrors the reference's paged route (backend.py:273-303): requests
with 0 < q_len <= paged_max_qlen (16) use the fp32 paged MTP semantics; longer
requests use the dense continuation semantics (history dequant + staged
splice, attention in the query dtype; backend.py:361-412).  paged_max_qlen = 0
gives the reference's default dense route (OSCAR_ASCEND_USE_PAGED unset,
backend.py:306-307), where every request takes the dense semantics.  Padding
rows stay zero.
"""
from __future__ import annotations

import itertools
from dataclasses import dataclass, field

import torch

from . import attention, rotate, store
from .staging import Arena, host_lists

PAGED_MAX_QLEN = 16           # backend.py:277


@dataclass
class OracleLayer:
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    R_k: torch.Tensor
    R_v: torch.Tensor
    num_heads: int
    num_kv_heads: int
    head_size: int
    scale: float
    clip_k: float = 0.0
    clip_v: float = 0.0
    sink: int = 64
    recent: int = 256
    staging: int = 8192
    paged_max_qlen: int = PAGED_MAX_QLEN
    arena: Arena | None = field(default=None)

    @property
    def window_enabled(self) -> bool:
        """config.py:89 — staging > 0 and (sink > 0 or recent > 0)."""
        return self.staging > 0 and (self.sink > 0 or self.recent > 0)

    def do_kv_cache_update(self, key, value, slot_mapping) -> None:
        """backend.py:150-189 — rotate + clip + INT2 store of N new tokens."""
        N = slot_mapping.shape[0]
        if N <= 0 or key is None:
            return
        Hk, D = self.num_kv_heads, self.head_size
        k_rot = rotate.rotate_clip(key[:N].reshape(N, Hk, D), self.R_k, self.clip_k)
        v_rot = rotate.rotate_clip(value[:N].reshape(N, Hk, D), self.R_v, self.clip_v)
        store.store_ref(k_rot, v_rot, self.k_cache, self.v_cache, slot_mapping)

    def ensure_arena(self) -> Arena:
        if self.arena is None:
            self.arena = Arena.create(self.k_cache.shape[1], self.num_kv_heads, self.head_size,
                                      self.sink, self.recent, self.staging)
        return self.arena

    def write(self, key, value, md) -> None:
        """backend.py:261-269 — store, then (window on) stage."""
        self.do_kv_cache_update(key, value, md.slot_mapping[:md.num_actual_tokens])
        if self.window_enabled:
            self.ensure_arena().write(key, value, md, self.R_k, self.R_v)

    def stage(self):
        return self.arena.triple() if (self.window_enabled and self.arena is not None) else None

    def read(self, query, key, value, md) -> torch.Tensor:
        """backend.py:271-319 — per-request attention, output in query dtype."""
        N, Hq, D = query.shape
        Hk = self.num_kv_heads
        qsl, seqs = host_lists(md)
        actual = min(N, md.num_actual_tokens)
        out = torch.zeros(N, Hq, D, dtype=query.dtype)
        Rk, Rv = self.R_k.float(), self.R_v.float()
        for i, (a, b) in enumerate(itertools.pairwise(qsl)):
            if a >= actual:
                continue
            b = min(b, actual)
            n = b - a
            if n <= 0:
                continue
            bt_row = md.block_tables[i]
            if n <= self.paged_max_qlen:
                res = attention.paged_attention_ref(
                    query[a:b].float() @ Rk, key[a:b].float() @ Rk, value[a:b].float() @ Rv,
                    self.k_cache, self.v_cache, bt_row.unsqueeze(0), [0, n], [seqs[i]],
                    self.scale, self.stage()) @ Rv.t()
            else:
                cached = seqs[i] - n
                if cached <= 0:
                    empty = torch.zeros(0, Hk, D)
                    res = attention.prefill_ref(query[a:b], key[a:b], value[a:b], empty, empty,
                                                self.scale, Hk, D)
                else:
                    kc, vc = store.full_dequant_ref(self.k_cache, self.v_cache, bt_row, cached, Hk, D)
                    if self.stage() is not None:
                        kc, vc = self.arena.splice(bt_row, cached, kc, vc)
                    dt = query.dtype
                    res = attention.prefill_ref(
                        (query[a:b].float() @ Rk).to(dt), (key[a:b].float() @ Rk).to(dt),
                        (value[a:b].float() @ Rv).to(dt), kc.to(dt), vc.to(dt), self.scale, Hk, D)
                    res = res.float() @ Rv.t()
            out[a:b] = res.to(query.dtype)
        return out

    def forward(self, query, key, value, md) -> torch.Tensor:
        self.write(key, value, md)
        return self.read(query, key, value, md)
