"""Oracle: paged MTP attention, chunked causal SDPA, decode and split reducer.

Restates oscar_ascend/kernels/paged_attention.py:20-64 and
oscar_ascend/kernels/decode_kernel.py:41-117, 250-293 (torch semantics only).
Test infrastructure only.

All tensors are in the rotated domain: q = query @ R_k, k = key @ R_k,
v = value @ R_v; outputs are in the rotated-V domain (the caller applies R_v^T).
"""
from __future__ import annotations

import itertools
import math

import torch
import torch.nn.functional as F

from . import store

PREFILL_QBLOCK = 512          # decode_kernel.py:20 default


def query_layout(qsl, seqs):
    """paged_attention.py:20-38 — (req per token, prefix per request,
    start per request, causal end per token)."""
    lengths = [b - a for a, b in itertools.pairwise(qsl)]
    if len(seqs) != len(lengths) or any(n < 0 or s < n for n, s in zip(lengths, seqs)):
        raise ValueError("Invalid OSCAR query/sequence lengths")
    req = torch.tensor([i for i, n in enumerate(lengths) for _ in range(n)], dtype=torch.int32)
    prefix = torch.tensor([s - n for s, n in zip(seqs, lengths)], dtype=torch.int32)
    starts = torch.tensor(qsl[:-1], dtype=torch.int32)
    ends = torch.tensor([s - n + j + 1 for s, n in zip(seqs, lengths) for j in range(n)], dtype=torch.int32)
    return req, prefix, starts, ends


def prefill_ref(q, k_new, v_new, k_cached, v_cached, scale: float, hk: int, D: int,
                qblock: int = PREFILL_QBLOCK):
    """decode_kernel.py:70-117 — causal SDPA of N new queries over C cached + N new keys.

    Computes in q's dtype.  Query i (absolute position C + i) sees keys
    0 .. C + i.  GQA: head h uses kv-head h // (Hq / Hk).
    """
    N, Hq = q.shape[0], q.shape[1]
    C = k_cached.shape[0]
    g = Hq // hk
    dt = q.dtype
    k_all = torch.cat([k_cached.to(dt), k_new.to(dt)], 0).transpose(0, 1).unsqueeze(0)
    v_all = torch.cat([v_cached.to(dt), v_new.to(dt)], 0).transpose(0, 1).unsqueeze(0)
    out = torch.empty(N, Hq, D, dtype=dt)
    if C <= 0 and N <= qblock:
        o = F.scaled_dot_product_attention(q.transpose(0, 1).unsqueeze(0), k_all, v_all,
                                           is_causal=True, scale=scale, enable_gqa=g > 1)
        out.copy_(o[0].transpose(0, 1))
        return out
    key_pos = torch.arange(C + N)
    for q0 in range(0, N, qblock):
        q1 = min(q0 + qblock, N)
        visible = key_pos.unsqueeze(0) <= torch.arange(C + q0, C + q1).unsqueeze(1)
        o = F.scaled_dot_product_attention(q[q0:q1].transpose(0, 1).unsqueeze(0), k_all, v_all,
                                           attn_mask=visible, scale=scale, enable_gqa=g > 1)
        out[q0:q1] = o[0].transpose(0, 1)
    return out


def history(kc, vc, bt_row, count: int, hk: int, D: int, stage=None):
    """Dequantized history of one request, with owner-matched staged override
    (paged_attention.py:48-60)."""
    bs = kc.shape[1]
    pos = torch.arange(count)
    pages = bt_row[pos // bs].long()
    k, v = store.dequant_split_ref(kc.view(torch.uint8), vc.view(torch.uint8), pages, pos % bs, hk, D)
    if stage is not None:
        sk, sv, owner = stage
        rows = pages % owner.shape[0]
        m = (owner[rows, pos % bs] == pages).view(-1, 1, 1)
        k = torch.where(m, sk[rows, pos % bs], k)
        v = torch.where(m, sv[rows, pos % bs], v)
    return k, v


def paged_attention_ref(q, k, v, kc, vc, bt, qsl, seqs, scale: float, stage=None):
    """paged_attention.py:41-64 — MTP oracle.

    Request i owns query rows [a, b); its history is positions
    0 .. seqs[i] - (b - a) - 1 read through block-table row i, and new token j
    additionally sees new tokens 0 .. j.
    """
    out = torch.zeros_like(q)
    hk, D = k.shape[1:]
    for i, (a, b) in enumerate(itertools.pairwise(qsl)):
        if a == b:
            continue
        hk_hist, hv_hist = history(kc, vc, bt[i], seqs[i] - (b - a), hk, D, stage)
        out[a:b] = prefill_ref(q[a:b], k[a:b], v[a:b], hk_hist, hv_hist, scale, hk, D)
    return out


def decode_ref(q, kc, vc, bt, seq_lens, scale: float, hk: int, D: int):
    """decode_kernel.py:41-67 — one query per sequence over its INT2 history.
    Returns (out [B, Hq, D], lse [B, Hq]) in fp32."""
    ks, vs = store.gather_kv_ref(kc, vc, bt, seq_lens, hk, D)
    B, Hq = q.shape[:2]
    g = Hq // hk
    out = torch.empty(B, Hq, D)
    lse = torch.empty(B, Hq)
    for b in range(B):
        kr = ks[b].repeat_interleave(g, dim=1)
        vr = vs[b].repeat_interleave(g, dim=1)
        s = torch.einsum("hd,lhd->hl", q[b].float(), kr) * scale
        out[b] = torch.einsum("hl,lhd->hd", torch.softmax(s, -1), vr)
        lse[b] = torch.logsumexp(s, -1)
    return out, lse


def merge_splits(outs: torch.Tensor, lses: torch.Tensor):
    """decode_kernel.py:250-293 — LSE-weighted merge of per-split (out, lse).

    outs [S, D], lses [S]; a split with lse = -inf is empty and skipped.
    All splits empty -> (zeros, -inf).
    """
    m = -math.inf
    total = 0.0
    acc = torch.zeros(outs.shape[-1])
    for o, c in zip(outs, lses.tolist()):
        if c == -math.inf:
            continue
        m_new = max(m, c)
        old = math.exp(m - m_new) if m != -math.inf else 0.0
        w = math.exp(c - m_new)
        acc = acc * old + w * o
        total = total * old + w
        m = m_new
    if total <= 0.0:
        return torch.zeros_like(acc), -math.inf
    return acc / total, m + math.log(total)


def window_bounds(owner, bt_row, seq: int, bs: int, sink_eff: int, recent: int):
    """backend.py:514-551 — (sink_active, cut) of one DecodeOnly request.

    The sink counts only when the request is longer than it and every seat of
    its sink pages holds that page; the tail is the longest run of staged
    positions ending at seq - 1 inside [max(seq - recent, sink end), seq);
    cut is where that run starts (seq when position seq - 1 is not staged).
    """
    rows = owner.shape[0]

    def staged(pos):
        page = int(bt_row[pos // bs])
        return int(owner[page % rows, pos % bs]) == page

    sink_pages = sink_eff // bs
    sink_active = sink_pages > 0 and seq > sink_eff and all(staged(p) for p in range(sink_pages * bs))
    t0 = max(seq - recent, sink_eff if sink_active else 0)
    cut = seq
    while cut > t0 and staged(cut - 1):
        cut -= 1
    return sink_active, cut


def _segment(q, k, v, scale: float, g: int):
    """Softmax attention of q [Hq, D] over k, v [L, Hk, D]: (out [Hq, D], lse [Hq]);
    an empty segment gives (0, -inf)."""
    if k.shape[0] == 0:
        return torch.zeros_like(q), torch.full((q.shape[0],), -math.inf)
    s = torch.einsum("hd,lhd->hl", q, k.repeat_interleave(g, dim=1)) * scale
    return torch.einsum("hl,lhd->hd", torch.softmax(s, -1), v.repeat_interleave(g, dim=1)), torch.logsumexp(s, -1)


def decode_only_ref(q, kc, vc, bt, seqs, scale: float, hk: int, D: int, arena=None):
    """backend.py:321-358, 500-586 — the DecodeOnly read (no fresh K/V): one
    rotated query per request [B, Hq, D] over its whole history [0, seq).

    Without a window arena: decode_ref over the INT2 caches.  With one
    (``arena``: stage_k, stage_v, owner, sink_eff, recent): the INT2 middle
    [si*bs, cut), read through the block table shifted by si sink pages, and
    the FP32 segment (sink positions when the sink is active, tail [cut, seq))
    are attended separately and merged through their log-sum-exps.
    Output fp32 in the rotated-V domain.
    """
    B, Hq, _ = q.shape
    g = Hq // hk
    if arena is None:
        return decode_ref(q, kc, vc, bt, torch.tensor(seqs), scale, hk, D)[0]
    sk, sv, owner, sink_eff, recent = arena
    bs = kc.shape[1]
    rows = owner.shape[0]
    out = torch.zeros(B, Hq, D)
    for b, seq in enumerate(seqs):
        row = bt[b].long()
        sink_active, cut = window_bounds(owner, row, seq, bs, sink_eff, recent)
        si = sink_eff // bs if sink_active else 0
        # INT2 middle
        n_mid = cut - si * bs
        if n_mid > 0:
            shifted = row[torch.clamp(torch.arange(row.numel()) + si, max=row.numel() - 1)]
            o1, l1 = decode_ref(q[b:b + 1].float(), kc, vc, shifted[None], [n_mid], scale, hk, D)
            o1, l1 = torch.nan_to_num(o1[0]), l1[0]
            l1 = torch.where(torch.isfinite(l1), l1, torch.full_like(l1, -math.inf))
        else:
            o1, l1 = torch.zeros(Hq, D), torch.full((Hq,), -math.inf)
        # FP32 sink + tail from the arena
        pos = list(range(sink_eff)) if sink_active else []
        pos += list(range(cut, seq))
        p = torch.tensor(pos, dtype=torch.long)
        pages = row[p // bs] if pos else p
        ks = sk[pages % rows, p % bs] if pos else torch.zeros(0, hk, D)
        vs = sv[pages % rows, p % bs] if pos else torch.zeros(0, hk, D)
        o2, l2 = _segment(q[b].float(), ks.float(), vs.float(), scale, g)
        lse = torch.logaddexp(l1, l2)
        safe = torch.where(torch.isfinite(lse), lse, torch.zeros_like(lse))
        out[b] = o1 * torch.exp(l1 - safe)[:, None] + torch.nan_to_num(o2) * torch.exp(l2 - safe)[:, None]
    return out
