"""Oracle: FP32 sink/recent window arena (owner-tagged hash seats).

Restates AscendOscarAttentionBackendImpl._ensure_staging / _staging_write /
_stage_splice and staging_order (oscar_ascend/backend.py:87-92, 418-498).
Test infrastructure only.

The arena has ``rows`` rows of ``bs`` seats.  Physical cache slot ``s`` hashes
to seat (row ``(s // bs) % rows``, column ``s % bs``).  ``owner[row, col]``
holds the physical page that currently owns the seat (or -1); the staged K/V
are the *unclipped, unquantized* rotated fp32 vectors.
"""
from __future__ import annotations

import itertools
from dataclasses import dataclass

import torch


def host_lists(md):
    """backend.py:25-55 — (query_start_loc, seq_lens) as Python lists.

    Preference order follows the reference: query_start_loc_cpu, then
    [0] + actual_seq_lengths_q, then query_start_loc; seq_lens_list, then
    seq_lens_cpu / _seq_lens_cpu, then seq_lens.
    """
    def as_list(x, name):
        if x is None:
            raise RuntimeError(f"attn_metadata.{name} missing")
        return x.tolist() if hasattr(x, "tolist") else list(x)

    qsl_cpu = getattr(md, "query_start_loc_cpu", None)
    ends = getattr(md, "actual_seq_lengths_q", None)
    if qsl_cpu is not None:
        qsl = as_list(qsl_cpu, "query_start_loc_cpu")
    elif ends is not None:
        qsl = [0] + as_list(ends, "actual_seq_lengths_q")
    else:
        qsl = as_list(md.query_start_loc, "query_start_loc")
    seq_cpu = getattr(md, "seq_lens_cpu", None)
    if seq_cpu is None:
        seq_cpu = getattr(md, "_seq_lens_cpu", None)
    seq_list = getattr(md, "seq_lens_list", None)
    src = seq_list if seq_list is not None else (seq_cpu if seq_cpu is not None else md.seq_lens)
    return qsl, as_list(src, "seq_lens")


def staging_order(seats: torch.Tensor, capacity: int) -> torch.Tensor:
    """backend.py:87-92 — stable argsort of seat ids (fp32 keys below 2^24)."""
    keys = seats.float() if capacity <= 2 ** 24 else seats
    return torch.argsort(keys, stable=True)


def arena_geometry(bs: int, sink: int, recent: int, staging: int):
    """backend.py:421-430 — (sink_eff, sink_pages, tail_pages, rows)."""
    sink_eff = (sink // bs) * bs
    sink_pages = sink_eff // bs
    tail_pages = (recent + bs - 1) // bs + 1
    rows = max((staging + bs - 1) // bs, sink_pages + tail_pages + 2)
    return sink_eff, sink_pages, tail_pages, rows


@dataclass
class Arena:
    stage_k: torch.Tensor     # [rows, bs, Hk, D] fp32
    stage_v: torch.Tensor
    owner: torch.Tensor       # [rows, bs] int64, -1 = empty
    bs: int
    sink_eff: int
    recent: int

    @property
    def rows(self) -> int:
        return self.owner.shape[0]

    @classmethod
    def create(cls, bs: int, hk: int, D: int, sink: int, recent: int, staging: int):
        """backend.py:418-437 — zeroed arena, all owners -1."""
        sink_eff, _, _, rows = arena_geometry(bs, sink, recent, staging)
        sk = torch.zeros(rows, bs, hk, D)
        return cls(sk, torch.zeros_like(sk), torch.full((rows, bs), -1, dtype=torch.int64),
                   bs, sink_eff, recent)

    def write(self, key, value, md, R_k, R_v) -> None:
        """backend.py:439-481 — record window tokens; last writer per seat wins.

        Tokens outside both windows still claim their seat, with owner -1, so a
        recycled page can never be read back from a stale seat.
        """
        N = md.num_actual_tokens
        if N == 0:
            return
        slot = md.slot_mapping[:N].to(torch.int64).cpu()
        qsl, seqs = host_lists(md)
        lengths = [max(0, min(b, N) - min(a, N)) for a, b in itertools.pairwise(qsl)]
        req = torch.repeat_interleave(torch.arange(len(lengths)), torch.tensor(lengths), output_size=N)
        seq = torch.tensor(seqs[:len(lengths)])
        ends = torch.tensor(qsl[1:])
        pos = seq[req] - ends[req] + torch.arange(N)
        keep = (pos >= seq[req] - self.recent) | (pos < self.sink_eff)
        bs = self.bs
        valid = torch.nonzero(slot >= 0, as_tuple=True)[0]
        seats = (slot[valid] // bs % self.rows) * bs + slot[valid] % bs
        order = staging_order(seats, self.rows * bs)
        ordered = seats[order]
        last = torch.cat([ordered[1:] != ordered[:-1],
                          torch.ones(min(1, ordered.numel()), dtype=torch.bool)])
        chosen = valid[order[last]]
        seats = ordered[last]
        rows, cols = seats // bs, seats % bs
        self.owner[rows, cols] = torch.where(keep[chosen], slot[chosen] // bs, -1)
        kept = keep[chosen]
        chosen, rows, cols = chosen[kept], rows[kept], cols[kept]
        if chosen.numel() == 0:
            return
        hk, D = self.stage_k.shape[2], self.stage_k.shape[3]
        k = key[:N].reshape(N, hk, D)[chosen].float().cpu()
        v = value[:N].reshape(N, hk, D)[chosen].float().cpu()
        self.stage_k[rows, cols] = k @ R_k.float().cpu()
        self.stage_v[rows, cols] = v @ R_v.float().cpu()

    def splice(self, bt_row, cached_len: int, k_cached, v_cached):
        """backend.py:483-498 — replace owned history positions by staged fp32."""
        bs = self.bs
        npg = (cached_len + bs - 1) // bs
        page = bt_row[:npg].to(torch.int64)
        rows = page % self.rows
        owned = self.owner[rows] == page.unsqueeze(-1)
        pos = (torch.arange(npg) * bs).unsqueeze(-1) + torch.arange(bs)
        owned = (owned & (pos < cached_len)).reshape(-1)[:cached_len]
        hk = self.stage_k.shape[2]
        ks = self.stage_k[rows].reshape(npg * bs, hk, -1)[:cached_len]
        vs = self.stage_v[rows].reshape(npg * bs, hk, -1)[:cached_len]
        m = owned.view(-1, 1, 1)
        return (torch.where(m, ks.to(k_cached.dtype), k_cached),
                torch.where(m, vs.to(v_cached.dtype), v_cached))

    def triple(self):
        return self.stage_k, self.stage_v, self.owner
