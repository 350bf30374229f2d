"""OSCAR INT2 FULL-attention impl for MI355X (drop-in for the reference impl).

Same surface as the reference's AscendOscarAttentionBackendImpl
(oscar_ascend/backend.py:95-611): the plugin swaps a FULL layer impl's class
to a subclass of (this class, the native impl class) and calls
``_oscar_setup()``; vLLM then calls ``forward`` / ``do_kv_cache_update``.

Write path (every step with fresh K/V):
  short steps        -> one fused step write (kernels/step.py, with the read)
  other steps        -> do_kv_cache_update + _staging_write in one library
                        call (kernels/quant.py): a seat-winner pass, then the
                        fused HIP kernel: rotate (MFMA) + clip + INT2 quantize
                        + pack + paged-slot write, whose epilogue writes the
                        window (owner tags, unclipped fp32 rotated values and
                        their fp16 operand images) from the same values
Read path, per request (backend.py:273-313 routing):
  0 < q_len <= 16    -> paged MTP decode kernel over INT2 history + window
  q_len > 16         -> prefill-continuation kernel (f16 MFMA over dequantized
                        history tiles + the new tokens, right-aligned causal)
Both read kernels work in the rotated domain; q/k/v are rotated with one
fp32 matmul each and the output is mapped back with R_v^T.

There is no fallback path: a missing library or a kernel error raises.
"""
from __future__ import annotations

import itertools
from enum import Enum

import torch

from .config import OscarConfig
from .format import HEAD_DIM, K_IDX_OFF, VALUES_PER_BYTE, check_d
from .kernels import _lib, decode, prefill, quant, staging, step
from .rotation import get_layer_rotation


def metadata_batch_lists(attn_metadata) -> tuple[list, list]:
    """(query_start_loc, seq_lens) as host lists (backend.py:25-55).

    Never uses a tensor as a boolean.  Preference: query_start_loc_cpu, then
    [0] + actual_seq_lengths_q, then query_start_loc; seq_lens_list, then
    seq_lens_cpu / _seq_lens_cpu, then seq_lens.
    """

    def as_list(x, name: str) -> list:
        if x is None:
            raise RuntimeError(f"attn_metadata.{name} is missing")
        return x.tolist() if hasattr(x, "tolist") else list(x)

    qsl_cpu = getattr(attn_metadata, "query_start_loc_cpu", None)
    ends = getattr(attn_metadata, "actual_seq_lengths_q", None)
    if qsl_cpu is not None:
        qsl = as_list(qsl_cpu, "query_start_loc_cpu")
    elif ends is not None:
        qsl = [0] + as_list(ends, "actual_seq_lengths_q")
    else:
        qsl = as_list(attn_metadata.query_start_loc, "query_start_loc")
    seq_cpu = getattr(attn_metadata, "seq_lens_cpu", None)
    if seq_cpu is None:
        seq_cpu = getattr(attn_metadata, "_seq_lens_cpu", None)
    seq_list = getattr(attn_metadata, "seq_lens_list", None)
    seqs = as_list(seq_list if seq_list is not None else (
        seq_cpu if seq_cpu is not None else attn_metadata.seq_lens), "seq_lens")
    return qsl, seqs


class OscarAttentionState(Enum):
    """Attention states accepted in metadata (backend.py:57-64); routing only
    looks at per-request query lengths."""

    PrefillNoCache = 0
    PrefillCacheHit = 1
    DecodeOnly = 2
    ChunkedPrefill = 3
    SpecDecoding = 4


def _is_decode_only(state) -> bool:
    """The DecodeOnly member of any engine's attention-state enum (or its value 2)."""
    if state is None:
        return False
    return getattr(state, "name", None) == "DecodeOnly" or state == OscarAttentionState.DecodeOnly.value


def _capturing(t: torch.Tensor) -> bool:
    """True while t's device stream is being captured into a graph."""
    return t.is_cuda and torch.cuda.is_current_stream_capturing()


class OscarAttentionBackendImpl:
    """Mixed into the native FULL-attention impl class by the plugin."""

    # ------------------------------------------------------------------ setup
    def _oscar_setup(self) -> None:
        """backend.py:99-122 — config, geometry checks, library load."""
        if getattr(self, "_oscar_cfg", None) is not None:
            return
        cfg = OscarConfig.from_env(head_dim=self.head_size)
        check_d(cfg.head_dim)
        if self.head_size != HEAD_DIM:
            raise ValueError(f"OSCAR MI355X kernels are written for head_size {HEAD_DIM}, got {self.head_size}")
        if self.num_heads % self.num_kv_heads:
            raise ValueError("OSCAR requires Hq divisible by Hk")
        _lib.load()
        self._oscar_cfg = cfg
        self._oscar_stage_ready = False
        self._oscar_stats = {"writes": 0, "kv_bytes_written": 0, "reads": 0}
        self._oscar_fixed_step_capture = False
        if cfg.verbose:
            print(f"[oscar-amd] OSCAR impl active: D={self.head_size}, slot=160B (K 96B + V 64B), "
                  f"Hq={self.num_heads}, Hk={self.num_kv_heads}, clip={cfg.k_clip_ratio}/{cfg.v_clip_ratio}, "
                  f"window(sink={cfg.sink_tokens}, recent={cfg.recent_tokens}, staging={cfg.staging_tokens})")

    @property
    def _oscar(self) -> OscarConfig:
        return self._oscar_cfg

    def allow_fixed_step_capture(self, allow: bool = True) -> None:
        """Let forward run under HIP graph capture.  Its launch arguments are
        built from the step's host-side request lengths (query_start_loc_cpu,
        seq_lens), so a replay repeats the captured step exactly: valid only
        when every replay is that same step (a benchmark), never for an
        engine's decode graphs, whose replays carry new lengths."""
        self._oscar_fixed_step_capture = bool(allow)

    # ------------------------------------------------------------------ caches / rotations
    def _set_caches(self, kv_cache) -> None:
        """backend.py:191-226 — split (K, V) caches; per-head slot width must be
        D bytes (int8 geometry) or 2D bytes (bf16 geometry)."""
        if isinstance(kv_cache, (tuple, list)) and len(kv_cache) >= 2:
            self.key_cache, self.value_cache = kv_cache[0], kv_cache[1]
        elif isinstance(kv_cache, torch.Tensor) and kv_cache.dim() > 0:
            self.key_cache, self.value_cache = kv_cache[0], kv_cache[1]
        if getattr(self, "key_cache", None) is None or getattr(self, "value_cache", None) is None:
            raise ValueError("OSCAR needs K and V caches")
        if not getattr(self, "_oscar_geo_ok", False):
            k8 = self.key_cache.view(torch.uint8)
            v8 = self.value_cache.view(torch.uint8)
            if k8.ndim != 4 or v8.ndim != 4 or not k8.is_contiguous() or not v8.is_contiguous():
                raise ValueError("OSCAR requires contiguous [blocks, tokens, heads, bytes] caches")
            slot_k, slot_v = int(k8.stride(2)), int(v8.stride(2))
            need_k = K_IDX_OFF + self.head_size // VALUES_PER_BYTE
            need_v = self.head_size // VALUES_PER_BYTE
            if slot_k not in (self.head_size, 2 * self.head_size):
                raise ValueError(f"OSCAR K slot width {slot_k}B must be {self.head_size} or {2 * self.head_size}")
            if need_k > slot_k or need_v > slot_v:
                raise ValueError(f"OSCAR slot too small: K needs {need_k}B, V needs {need_v}B")
            self._oscar_geo_ok = True

    def _layer_rots(self, layer, device):
        """backend.py:228-236 — (R_k, R_v) cached on the layer, plus their MFMA
        operands (rebuilt when the cached rotations are replaced)."""
        if not getattr(layer, "_oscar_rots", None):
            cfg = self._oscar
            rk = get_layer_rotation(cfg.k_rotation_path, layer.layer_name, self.head_size, device, mode="k", strict=True)
            rv = get_layer_rotation(cfg.v_rotation_path, layer.layer_name, self.head_size, device, mode="v", strict=True)
            layer._oscar_rots = (rk, rv)
        rk, rv = layer._oscar_rots
        if rk.device != torch.device(device) or rk.dtype != torch.float32:
            rk = rk.to(device=device, dtype=torch.float32).contiguous()
            rv = rv.to(device=device, dtype=torch.float32).contiguous()
            layer._oscar_rots = (rk, rv)
        cached = getattr(layer, "_oscar_rot_ops", None)
        if cached is None or cached[0] is not rk or cached[1] is not rv:
            layer._oscar_rkT = rk.t().contiguous()
            layer._oscar_rvT = rv.t().contiguous()
            layer._oscar_rot_ops = (rk, rv, quant.rotation_operand(rk), quant.rotation_operand(rv))
            # the output rotation of the prefill route (out @ R_v^T) on MFMA
            layer._oscar_rvT_op = quant.rotation_operand(layer._oscar_rvT)
        return layer._oscar_rots

    # ------------------------------------------------------------------ write path
    def do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping) -> None:
        """backend.py:150-189 — rotate + clip + INT2 store of the step's tokens."""
        self._kv_write(layer, key, value, kv_cache, slot_mapping, None)

    def _kv_write(self, layer, key, value, kv_cache, slot_mapping, window) -> None:
        if key is None or value is None:
            return
        slot_mapping = slot_mapping.to(device=key.device, dtype=torch.int64)
        N = slot_mapping.shape[0]
        if N <= 0:
            return
        self._set_caches(kv_cache)
        self._layer_rots(layer, key.device)
        _, _, op_k, op_v = layer._oscar_rot_ops
        cfg = self._oscar
        D = self.head_size
        quant.quant_write(key, value, op_k, op_v, self.key_cache, self.value_cache, slot_mapping,
                          quant.clip_index(cfg.k_clip_ratio, D), quant.clip_index(cfg.v_clip_ratio, D),
                          self.num_kv_heads, D, window=window)
        self._oscar_stats["writes"] += 1
        self._oscar_stats["kv_bytes_written"] += N * self.num_kv_heads * 160

    def _write_step(self, layer, key, value, kv_cache, attn_metadata) -> None:
        """The step's INT2 write and, with the window on, its window write
        (backend.py:277-282: do_kv_cache_update, then _staging_write) in one
        library call: a seat-winner pass and the fused quantize-write kernel,
        whose epilogue writes the window from the same rotated values."""
        N = attn_metadata.num_actual_tokens
        slot_mapping = attn_metadata.slot_mapping[:N]
        if not self._oscar.window_enabled:
            self.do_kv_cache_update(layer, key, value, kv_cache, slot_mapping)
            return
        self._ensure_staging(layer, kv_cache)
        if N <= 0:
            return
        self._kv_write(layer, key, value, kv_cache, slot_mapping, self._window_args(layer, key.device, attn_metadata))

    def _window_args(self, layer, dev, attn_metadata):
        """The step's request layout and the layer's arena, as the window
        writes take them."""
        N = attn_metadata.num_actual_tokens
        qsl, seqs = metadata_batch_lists(attn_metadata)
        lengths = [max(0, min(b, N) - min(a, N)) for a, b in itertools.pairwise(qsl)]
        if sum(lengths) != N:
            raise ValueError("query_start_loc does not cover the step's tokens")
        B = len(lengths)
        meta = torch.tensor(list(qsl[:B + 1]) + list(seqs[:B]), dtype=torch.int32).to(dev, non_blocking=True)
        _, sink_eff = self._stage_params(layer)
        return (meta[:B + 1], meta[B + 1:], B, sink_eff, self._oscar.recent_tokens, layer._oscar_stage_k,
                layer._oscar_stage_v, layer._oscar_slot_owner, layer._oscar_seat_winner, layer._oscar_stage_kimg,
                layer._oscar_stage_vimg)

    def _ensure_staging(self, layer, kv_cache) -> None:
        """backend.py:418-437 — persistent per-layer FP32 window arena."""
        if getattr(layer, "_oscar_stage_ready", False):
            self._oscar_stage_ready = True
            return
        bs = kv_cache[0].shape[1]
        cfg = self._oscar
        self.stage_block = bs
        self.sink_eff, self.sink_pages, self.tail_pages, rows = staging.arena_geometry(
            bs, cfg.sink_tokens, cfg.recent_tokens, cfg.staging_tokens)
        dev = kv_cache[0].device
        layer._oscar_stage_k = torch.zeros(rows, bs, self.num_kv_heads, self.head_size, dtype=torch.float32, device=dev)
        layer._oscar_stage_v = torch.zeros_like(layer._oscar_stage_k)
        layer._oscar_slot_owner = torch.full((rows, bs), -1, dtype=torch.int64, device=dev)
        layer._oscar_seat_winner = staging.winner_buffer(rows, bs, dev)
        # fp16 operand images of the window for the paged decode (32-token tiles)
        layer._oscar_stage_kimg = layer._oscar_stage_vimg = None
        if bs % 32 == 0:
            layer._oscar_stage_kimg = torch.zeros(staging.k_image_shape(rows, bs, self.num_kv_heads),
                                                  dtype=torch.float16, device=dev)
            layer._oscar_stage_vimg = torch.zeros(staging.image_shape(rows, bs, self.num_kv_heads),
                                                  dtype=torch.float16, device=dev)
        layer._oscar_stage_rows = rows
        layer._oscar_stage_ready = True
        self._oscar_stage_ready = True

    def _stage_params(self, layer):
        bs = layer._oscar_stage_k.shape[1]
        cfg = self._oscar
        sink_eff = (cfg.sink_tokens // bs) * bs
        return bs, sink_eff

    def _staging_write(self, layer, key, value, attn_metadata) -> None:
        """backend.py:439-481 — record the step's window tokens (last writer per
        seat wins; tokens outside both windows invalidate their seat)."""
        N = attn_metadata.num_actual_tokens
        if N == 0:
            return
        dev = key.device
        qsl, seqs, B, sink_eff, recent, sk, sv, owner, winner, kimg, vimg = self._window_args(layer, dev, attn_metadata)
        rk, rv = self._layer_rots(layer, dev)
        bs, _ = self._stage_params(layer)
        staging.staging_write(key, value, attn_metadata.slot_mapping[:N].to(dev), qsl, seqs, B, self.num_kv_heads,
                              self.head_size, bs, sink_eff, recent, rk, rv, sk, sv, owner, winner, kimg, vimg)

    def _stage(self, layer):
        if self._oscar.window_enabled and getattr(layer, "_oscar_stage_ready", False):
            return (layer._oscar_stage_k, layer._oscar_stage_v, layer._oscar_slot_owner,
                    layer._oscar_stage_kimg, layer._oscar_stage_vimg)
        return None

    # ------------------------------------------------------------------ forward
    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None,
                output_scale=None, output_block_scale=None):
        """backend.py:239-319 — write, then read per request; padding rows stay 0."""
        if output is None:
            raise ValueError("Output tensor must be provided.")
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError("OSCAR fused output quantization is unsupported")
        num_tokens = query.shape[0]
        if attn_metadata is None:
            return output.fill_(0)
        capturing = _capturing(query)
        if capturing and not getattr(self, "_oscar_fixed_step_capture", False):
            # The reference plugin likewise runs eagerly (delivery/serve_oscar.sh:54-55).
            raise RuntimeError("OSCAR attention cannot be captured into an engine's graphs: its launch arguments "
                               "come from the step's host-side request lengths, which every replay would reuse; "
                               "serve with --enforce-eager")
        self._set_caches(kv_cache)
        if key is None or value is None:
            # backend.py:304-309: without fresh K/V only the DecodeOnly state
            # has a read path (the reference's dense route needs the keys)
            if not _is_decode_only(getattr(attn_metadata, "attn_state", None)):
                raise NotImplementedError("OSCAR reads without fresh K/V need the DecodeOnly attention state")
            attn_out = self._decode_attention(layer, query, attn_metadata)
            self._oscar_stats["reads"] += 1
            output[:num_tokens] = attn_out.reshape(output[:num_tokens].shape).to(output.dtype)
            return output

        if self._short_step(layer, query, key, value, kv_cache, attn_metadata, output, capturing):
            self._oscar_stats["reads"] += 1
            return output
        self._write_step(layer, key, value, kv_cache, attn_metadata)

        attn_out = self._read(layer, query, key, value, attn_metadata)
        self._oscar_stats["reads"] += 1
        if output.ndim == 3:
            output[:num_tokens] = attn_out[:num_tokens].to(output.dtype)
        else:
            output[:num_tokens] = attn_out.reshape(num_tokens, -1).to(output.dtype)
        return output

    def _short_step(self, layer, query, key, value, kv_cache, attn_metadata, output, capturing: bool) -> bool:
        """The whole forward of a step whose requests all take the paged read
        (0 < q_len <= 16, backend.py:273-303) in one library call: the fused
        step write (q/k/v rotation, INT2 write, window write) and the decode
        with R_v^T and the cast to the output dtype in its merge.  The layer's
        arguments are packed once per layer and the step's once per step.
        Returns False (nothing done) when the step does not qualify."""
        cfg = self._oscar
        N = attn_metadata.num_actual_tokens
        if not cfg.use_paged or N <= 0 or N > step.MAX_STEP_TOKENS or query.shape[0] < N or output.shape[0] < N:
            return False
        if output.dtype not in (torch.bfloat16, torch.float32) or query.dtype != torch.bfloat16 \
                or key.dtype != torch.bfloat16 or value.dtype != torch.bfloat16:
            return False
        if self.key_cache.shape[1] % 32:
            return False
        qsl, seqs = metadata_batch_lists(attn_metadata)
        dev = query.device
        stream = _lib.stream_handle(dev)
        st = step.mtp_step(qsl, seqs, N, attn_metadata.slot_mapping, attn_metadata.block_tables, self.num_heads,
                           self.num_kv_heads, self.head_size, cfg.paged_max_q_len, dev, stream, reuse=not capturing)
        if st is None:
            return False
        step.mtp_forward(self._mtp_layer(layer, kv_cache, dev), st, query, key, value, output, stream)
        self._oscar_stats["writes"] += 1
        self._oscar_stats["kv_bytes_written"] += N * self.num_kv_heads * 160
        if output.shape[0] > N:
            output[N:].zero_()
        return True

    def _mtp_layer(self, layer, kv_cache, dev) -> step.MtpLayer:
        """The layer half of the short-step forward, kept on the layer and
        rebuilt only when its rotations, caches or window arena are replaced."""
        cfg = self._oscar
        if cfg.window_enabled:
            self._ensure_staging(layer, kv_cache)
        rots = getattr(layer, "_oscar_rots", None)
        if not rots:
            rots = self._layer_rots(layer, dev)
        arena = (layer._oscar_stage_k, layer._oscar_stage_v, layer._oscar_slot_owner, layer._oscar_stage_kimg,
                 layer._oscar_stage_vimg) if cfg.window_enabled else (None,) * 5
        ml = getattr(layer, "_oscar_mtp", None)
        rvT = getattr(layer, "_oscar_rvT", None)
        if ml is not None and ml.bound_to(rots[0], rots[1], rvT, self.key_cache, self.value_cache, *arena):
            return ml
        rk, rv = self._layer_rots(layer, dev)
        D = self.head_size
        bs = self.key_cache.shape[1]
        ml = step.MtpLayer(rk, rv, layer._oscar_rvT, self.key_cache, self.value_cache, self.num_heads,
                           self.num_kv_heads, quant.clip_index(cfg.k_clip_ratio, D),
                           quant.clip_index(cfg.v_clip_ratio, D), self.scale,
                           arena if cfg.window_enabled else None, (cfg.sink_tokens // bs) * bs, cfg.recent_tokens)
        layer._oscar_mtp = ml
        return ml

    def _decode_attention(self, layer, query, attn_metadata) -> torch.Tensor:
        """backend.py:321-358, 500-586 — one query token per request over its
        whole history, staged values only in the windowed segments; output
        in the query dtype."""
        qsl, seqs = metadata_batch_lists(attn_metadata)
        N = query.shape[0]
        B = len(seqs)
        if N != B or any(b - a != 1 for a, b in itertools.pairwise(qsl[:B + 1])):
            raise ValueError("DecodeOnly needs exactly one query token per request")
        dev = query.device
        rk, _ = self._layer_rots(layer, dev)
        cfg = self._oscar
        q = query.reshape(N, self.num_heads, self.head_size)
        out_rot = decode.decode_only(q.float() @ rk, self.key_cache, self.value_cache, attn_metadata.block_tables,
                                     seqs, self.scale, self._stage(layer), cfg.sink_tokens, cfg.recent_tokens)
        return (out_rot @ layer._oscar_rvT).to(query.dtype)

    def _read(self, layer, query, key, value, attn_metadata) -> torch.Tensor:
        N, Hq, D = query.shape
        dev = query.device
        Hk = self.num_kv_heads
        qsl, seqs = metadata_batch_lists(attn_metadata)
        actual = min(N, attn_metadata.num_actual_tokens)
        pairs = [(i, a, min(b, actual), seqs[i]) for i, (a, b) in enumerate(itertools.pairwise(qsl)) if a < actual]
        limit = self._oscar.paged_max_q_len if self._oscar.use_paged else 0
        short = [p for p in pairs if 0 < p[2] - p[1] <= limit]
        large = [p for p in pairs if p[2] - p[1] > limit]
        rk, rv = self._layer_rots(layer, dev)
        rvT = layer._oscar_rvT
        stage = self._stage(layer)
        attn_out = torch.zeros(N, Hq, D, device=dev, dtype=query.dtype)
        bt = attn_metadata.block_tables
        q3 = query.view(N, Hq, D)
        k3 = key.view(-1, Hk, D)
        v3 = value.view(-1, Hk, D)
        if short:
            token_ids = [t for _, a, b, _ in short for t in range(a, b)]
            contiguous = token_ids == list(range(token_ids[0], token_ids[0] + len(token_ids)))
            if contiguous:
                sl = slice(token_ids[0], token_ids[0] + len(token_ids))
                qs, ks, vs = q3[sl], k3[sl], v3[sl]
            else:
                idx = torch.tensor(token_ids, device=dev)
                qs, ks, vs = q3[idx], k3[idx], v3[idx]
            starts = [0]
            for _, a, b, _ in short:
                starts.append(starts[-1] + b - a)
            req_idx = torch.tensor([i for i, _, _, _ in short], device=bt.device)
            out_rot = decode.paged_attention(qs.float() @ rk, ks.float() @ rk, vs.float() @ rv,
                                             self.key_cache, self.value_cache, bt[req_idx], starts,
                                             [s for _, _, _, s in short], self.scale, stage)
            res = (out_rot @ rvT).to(query.dtype)
            if contiguous:
                attn_out[sl] = res
            else:
                attn_out[idx] = res
        # bf16 models rotate on MFMA (oscar_rotate_rows: about 2^-16 of each
        # product, below the fp16 rounding the prefill kernel's operands take
        # and the bf16 output's); other dtypes keep the fp32 matmuls.
        mfma_rot = query.dtype == key.dtype == value.dtype == torch.bfloat16
        _, _, op_k, op_v = layer._oscar_rot_ops
        for i, a, b, seq in large:
            cached = seq - (b - a)
            if mfma_rot:
                qr, kr, vr = (quant.rotate_rows(q3[a:b], op_k), quant.rotate_rows(k3[a:b], op_k),
                              quant.rotate_rows(v3[a:b], op_v))
            else:
                qr, kr, vr = q3[a:b].float() @ rk, k3[a:b].float() @ rk, v3[a:b].float() @ rv
            out_rot = prefill.prefill_continuation(qr, kr, vr, self.key_cache, self.value_cache, bt[i],
                                                   max(cached, 0), self.scale, stage)
            if mfma_rot:
                quant.rotate_rows(out_rot, layer._oscar_rvT_op, torch.bfloat16, out=attn_out[a:b])
            else:
                attn_out[a:b] = (out_rot @ rvT).to(query.dtype)
        return attn_out


# The reference's class name, kept for drop-in imports.
AscendOscarAttentionBackendImpl = OscarAttentionBackendImpl
