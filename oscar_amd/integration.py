"""Memory budgeting of the persistent OSCAR buffers (MI355X, 288 GB HBM3E).

Mirrors oscar_ascend/integration.py:17-44, 89-114: the KV-cache budget the
engine may allocate is what remains after the fixed per-layer buffers, in
whole cache blocks.  Per OSCAR layer the fixed buffers here are
  * R_k, R_v and their transposes, fp32       4 * D^2 * 4
  * the MFMA rotation operands of R_k, R_v      3 * oscar_rotation_operand_bytes(D)
    and R_v^T
  * the FP32 window arena                      rows * bs * (2 * Hk * D * 4 + 8)
  * its fp16 MFMA operand images (high and    rows * bs * 4 * Hk * D * 2
    low parts of K and of V)
  * the arena's seat-winner buffer             rows * bs * 8 + 16
and, once per device, the split-decode workspace of the largest batch and
the library's no-allocation decode array (32 MiB, a static device array every
GPU that loads the library holds whether or not that entry is called).

The engine seams (``install_runner_hooks``) apply that budget before vLLM
allocates its caches and print one READY manifest per rank after it did;
``validate_ready`` checks a server log's manifests.
"""
from __future__ import annotations

import hashlib
import json
from copy import deepcopy
from pathlib import Path

MI355X_HBM_BYTES = 288 * 10 ** 9
ROTATION_OPERAND_BYTES = 524288        # oscar_rotation_operand_bytes(256): MFMA tiles + fp32 R
NOALLOC_SCRATCH_BYTES = 32 << 20       # OSCAR_DECODE_NOALLOC_SCRATCH_BYTES: resident once per device


def memory_budget(available: int, native_per_block: int, shadow_per_block: int, fixed_bytes: int) -> int:
    """integration.py:17-23 — KV bytes = whole blocks that fit after the fixed buffers."""
    if native_per_block <= 0 or available <= fixed_bytes:
        raise ValueError("Insufficient memory for OSCAR persistent buffers")
    blocks = (available - fixed_bytes) // (native_per_block + shadow_per_block)
    if blocks < 1:
        raise ValueError("OSCAR memory budget cannot hold one cache block")
    return blocks * native_per_block


def arena_rows(block_size: int, sink: int, recent: int, staging: int) -> int:
    """integration.py:99-113 — rows reserved at the engine page size."""
    return max((staging + block_size - 1) // block_size,
               sink // block_size + (recent + block_size - 1) // block_size + 3)


def fixed_bytes_per_layer(head_dim: int, num_kv_heads: int, block_size: int, sink: int, recent: int,
                          staging: int, window: bool) -> int:
    fixed = 4 * head_dim * head_dim * 4 + 3 * ROTATION_OPERAND_BYTES
    if window:
        rows = arena_rows(block_size, sink, recent, staging)
        fixed += rows * block_size * (2 * num_kv_heads * head_dim * 4 + 4 * num_kv_heads * head_dim * 2 + 8 + 8) + 16
    return fixed


DECODE_TILE = 32                       # history tokens per decode tile
DECODE_ROWS = 32                       # (query, head) rows per partial
DECODE_PARTIAL_FLOATS = DECODE_ROWS * 256 + 2 * DECODE_ROWS
DECODE_LAUNCH_ITEMS = 128              # (request, kv head) items carried in one launch's kernel arguments
DECODE_MAX_SPLITS = 1023               # history splits per item (the fresh-token partial makes 1024)
DECODE_MAX_TILES_PER_SPLIT = 256


DECODE_RESIDENT_SPLITS = 512          # split workgroups resident at once (two per CU, 256 CUs)
DECODE_STEP = 128                      # history tokens per decode step (4 tiles)
DECODE_MAX_STEPS_PER_SPLIT = 64


def decode_partial_slots(items: int, max_history: int, tiles_per_split: int = 0) -> int:
    """Partial slots of one launch chunk of `items` (request, kv head) items,
    one fresh-token slot each.  Explicit tiles per split: ceil(tiles / tps)
    splits per item.  Automatic: per-item split counts that keep the chunk
    within one round of resident workgroups (or one split per 64 steps of
    each item when that is more), never more than the items' steps."""
    if tiles_per_split:
        tiles = -(-max_history // DECODE_TILE) if max_history > 0 else 0
        return items * (-(-tiles // tiles_per_split) + 1)
    steps = -(-max_history // DECODE_STEP) if max_history > 0 else 0
    bound = max(items * -(-steps // DECODE_MAX_STEPS_PER_SPLIT), DECODE_RESIDENT_SPLITS)
    return min(items * steps, bound) + items


def decode_split_plan(query_lens, histories, max_history: int, tiles_per_split: int = 0, fresh: int = 1):
    """The library's per-item history splits of one launch chunk (items in
    order, one per (request, kv head)): returns (nsplit, pbase) lists.
    Explicit tiles per split: ceil(tiles / tps) splits per item.  Automatic:
    the smallest common number T of 128-token steps per split (T <= 64) that
    keeps the history splits within one round of resident workgroups, and
    ceil(steps / T) splits per item, where a last step of at most one tile
    (32 tokens) goes uncounted when that lowers T; never more splits than
    steps."""
    steps = [-(-h // DECODE_STEP) if q > 0 and h > 0 else 0 for q, h in zip(query_lens, histories)]
    if tiles_per_split:
        tiles = -(-max_history // DECODE_TILE) if max_history > 0 else 0
        per = [-(-tiles // tiles_per_split)] * len(steps)
    else:
        def least_t(cnt):
            t = max(1, -(-sum(cnt) // DECODE_RESIDENT_SPLITS))
            while sum(-(-n // t) for n in cnt) > DECODE_RESIDENT_SPLITS and t < DECODE_MAX_STEPS_PER_SPLIT:
                t += 1
            return t
        # a last step of at most one tile's tokens may go uncounted when that lowers T
        cut = [s - (1 if s > 1 and 0 < h % DECODE_STEP <= DECODE_TILE else 0) for s, h in zip(steps, histories)]
        T, Tc = least_t(steps), least_t(cut)
        cnt = cut if Tc < T else steps
        T = min(T, Tc)
        per = [max(-(-n // T), -(-s // DECODE_MAX_STEPS_PER_SPLIT)) for n, s in zip(cnt, steps)]
    nsplit, pbase, slot = [], [], 0
    for n, st in zip(per, steps):
        n = min(n, st)
        nsplit.append(n)
        pbase.append(slot)
        slot += n + fresh
    return nsplit, pbase


def decode_workspace_bytes(max_requests: int, num_kv_heads: int, num_heads: int, max_query_len: int,
                           max_history: int, tiles_per_split: int = 0) -> int:
    """Same value as oscar_paged_decode_workspace_bytes (no library needed):
    one fp32 partial (32 rows x 256 + max + sum) per partial slot and row tile
    of one launch chunk (requests of a launch share one workspace)."""
    row_tiles = -(-(max_query_len * (num_heads // num_kv_heads)) // DECODE_ROWS)
    per_launch = DECODE_LAUNCH_ITEMS // num_kv_heads
    chunk = min(max_requests, per_launch)
    return decode_partial_slots(chunk * num_kv_heads, max_history, tiles_per_split) * row_tiles * \
        DECODE_PARTIAL_FLOATS * 4


def kv_block_bytes(block_size: int, num_kv_heads: int, slot_width: int, layers: int) -> int:
    """Native bytes of one cache block across the OSCAR layers (K and V caches)."""
    return 2 * block_size * num_kv_heads * slot_width * layers


def plan_capacity(available: int, layers: int, head_dim: int = 256, num_kv_heads: int = 1,
                  num_heads: int = 6, block_size: int = 128, slot_width: int = 256, sink: int = 128,
                  recent: int = 256, staging: int = 8192, window: bool = True, max_requests: int = 256,
                  max_query_len: int = 4, max_history: int = 262144) -> dict:
    """Budget one GPU: how many cache blocks (and INT2 tokens) fit."""
    fixed = layers * fixed_bytes_per_layer(head_dim, num_kv_heads, block_size, sink, recent, staging, window)
    fixed += decode_workspace_bytes(max_requests, num_kv_heads, num_heads, max_query_len, max_history)
    fixed += NOALLOC_SCRATCH_BYTES
    native = kv_block_bytes(block_size, num_kv_heads, slot_width, layers)
    budget = memory_budget(available, native, 0, fixed)
    blocks = budget // native
    return {"available": available, "fixed": fixed, "native_per_block": native, "budget": budget,
            "blocks": blocks, "tokens": blocks * block_size}


def source_fingerprint() -> str:
    """integration.py:26-32 — sha256 over the package's Python and HIP sources."""
    root = Path(__file__).parent
    digest = hashlib.sha256()
    for path in sorted(list(root.rglob("*.py")) + list(root.rglob("*.hip")) + list(root.rglob("*.h"))):
        digest.update(str(path.relative_to(root)).encode())
        digest.update(path.read_bytes())
    return digest.hexdigest()


def verify_layers(layer_types, actual_ids) -> None:
    """integration.py:35-44 — every full-attention layer must run OSCAR."""
    expected = {i for i, kind in enumerate(layer_types) if kind in ("full_attention", "attention")}
    if not expected or set(actual_ids) != expected or len(actual_ids) != len(expected):
        raise RuntimeError(f"Incomplete OSCAR layers: expected={sorted(expected)}, actual={sorted(actual_ids)}")


# vLLM v1 worker classes on ROCm (the reference hooks vllm_ascend's
# NPUWorker / NPUModelRunner at the same two methods).
WORKER_CLASS = ("vllm.v1.worker.gpu_worker", "Worker")
RUNNER_CLASS = ("vllm.v1.worker.gpu_model_runner", "GPUModelRunner")
KV_CACHE_UTILS = "vllm.v1.core.kv_cache_utils"
READY_MARKER = "[oscar-amd] READY "
INJECTION_FAILED = "[oscar-amd] injection failed"


def _import_attr(module: str, name: str):
    mod = __import__(module, fromlist=[name])
    return getattr(mod, name)


def _oscar_modules(ctx: dict) -> dict:
    return {name: m for name, m in ctx.items() if getattr(getattr(m, "impl", None), "_oscar_cfg", None) is not None}


def oscar_fixed_bytes(runner, specs: dict, targets: dict) -> int:
    """Persistent bytes the OSCAR layers allocate after profiling (rotations,
    MFMA operands, window arena and its images, at the engine page size),
    plus, once per device, the split-decode workspace of the largest batch
    and the library's 32 MiB no-allocation decode array."""
    fixed = 0
    hk = heads = 1
    for name, module in targets.items():
        impl = module.impl
        c = impl._oscar
        bs = specs[name].block_size
        fixed += fixed_bytes_per_layer(impl.head_size, impl.num_kv_heads, bs, c.sink_tokens, c.recent_tokens,
                                       c.staging_tokens, c.window_enabled)
        hk, heads = impl.num_kv_heads, impl.num_heads
    cfg = runner.vllm_config
    max_reqs = int(getattr(cfg.scheduler_config, "max_num_seqs", 256) or 256)
    max_len = int(getattr(cfg.model_config, "max_model_len", 0) or 0)
    spec_cfg = getattr(cfg, "speculative_config", None)
    max_q = 1 + int(getattr(spec_cfg, "num_speculative_tokens", 0) or 0) if spec_cfg is not None else 1
    if targets and max_len > 0:
        fixed += decode_workspace_bytes(max_reqs, hk, heads, max_q, max_len)
    if targets:
        fixed += NOALLOC_SCRATCH_BYTES
    return fixed


def install_runner_hooks() -> None:
    """integration.py:47-195 — the two engine seams around cache allocation.

    * ``Worker.determine_available_memory``: the KV budget the engine may
      allocate shrinks to whole native blocks that fit after the OSCAR
      persistent buffers (``memory_budget``); the plan is kept on the runner.
    * ``GPUModelRunner.initialize_kv_cache_tensors``: after the engine built
      its caches, every OSCAR layer binds them, loads its rotations (and MFMA
      operands) and allocates its window arena; the actual persistent bytes
      must stay inside the profiled budget, every full-attention layer must
      run OSCAR (``verify_layers``), and one READY manifest line is printed.

    The reference's MTP draft shadow caches (``mtp_shadow``) are not part of
    this build, so the shadow term is zero.  Idempotent."""
    try:
        Worker = _import_attr(*WORKER_CLASS)
        Runner = _import_attr(*RUNNER_CLASS)
    except Exception as e:  # noqa: BLE001 - no vLLM in this process
        raise RuntimeError(f"OSCAR runner hooks need vLLM's v1 worker ({e})") from e
    if getattr(Worker, "_oscar_memory_hook", False):
        return
    original_memory = Worker.determine_available_memory
    original_caches = Runner.initialize_kv_cache_tensors

    def determine_available_memory(worker):
        available = original_memory(worker)
        runner = worker.model_runner
        ctx = runner.compilation_config.static_forward_context
        targets = _oscar_modules(ctx)
        if not targets:
            return available
        get_groups = _import_attr(KV_CACHE_UTILS, "get_kv_cache_groups")
        get_config = _import_attr(KV_CACHE_UTILS, "get_kv_cache_config_from_groups")
        cfg = runner.vllm_config
        if getattr(cfg.cache_config, "num_gpu_blocks_override", None) is not None:
            raise ValueError("num_gpu_blocks_override bypasses OSCAR memory budgeting")
        if getattr(cfg.parallel_config, "data_parallel_size", 1) != 1:
            raise ValueError("OSCAR manifest validation supports DP=1")
        if getattr(cfg.parallel_config, "pipeline_parallel_size", 1) != 1:
            raise ValueError("OSCAR memory accounting supports PP=1")
        specs = deepcopy(runner.get_kv_cache_spec())
        groups = get_groups(cfg, deepcopy(specs))
        provisional = get_config(cfg, groups, available)
        if provisional.num_blocks < 1:
            raise ValueError("No native cache blocks fit")
        native = sum(t.size for t in provisional.kv_cache_tensors) // provisional.num_blocks
        fixed = oscar_fixed_bytes(runner, specs, targets)
        budget = memory_budget(available, native, 0, fixed)
        runner._oscar_memory_plan = {"available": available, "native": native, "shadow": 0, "fixed": fixed,
                                     "budget": budget}
        worker.available_kv_cache_memory_bytes = budget
        print("[oscar-amd] MEMORY " + json.dumps(runner._oscar_memory_plan, sort_keys=True), flush=True)
        return budget

    def initialize_kv_cache_tensors(runner, kv_cache_config, *args, **kwargs):
        caches = original_caches(runner, kv_cache_config, *args, **kwargs)
        from .rotation import layer_index_from_name

        ctx = runner.compilation_config.static_forward_context
        names, ids = [], []
        persistent = 0
        for name, module in _oscar_modules(ctx).items():
            impl = module.impl
            cache = caches[name]
            impl._set_caches(cache)
            k_cache = impl.key_cache
            impl._layer_rots(module, k_cache.device)
            persistent += 4 * impl.head_size ** 2 * 4 + 3 * ROTATION_OPERAND_BYTES
            if impl._oscar.window_enabled:
                impl._ensure_staging(module, (impl.key_cache, impl.value_cache))
                for attr in ("_oscar_stage_k", "_oscar_stage_v", "_oscar_slot_owner", "_oscar_seat_winner",
                             "_oscar_stage_kimg", "_oscar_stage_vimg"):
                    t = getattr(module, attr, None)
                    if t is not None:
                        persistent += t.numel() * t.element_size()
            names.append(name)
            ids.append(layer_index_from_name(name))
        if names:
            plan = getattr(runner, "_oscar_memory_plan", None)
            if plan is None:
                raise RuntimeError("OSCAR caches were initialised without the OSCAR memory plan")
            native_bytes = sum(t.size for t in kv_cache_config.kv_cache_tensors)
            if native_bytes + persistent > plan["available"]:
                raise RuntimeError("Actual OSCAR persistent allocation exceeds profiled budget")
            hf = runner.model_config.hf_text_config
            verify_layers(getattr(hf, "layer_types", []), ids)
            rank = 0
            try:
                import torch.distributed as dist

                rank = dist.get_rank() if dist.is_initialized() else 0
            except Exception:  # noqa: BLE001 - no process group
                rank = 0
            manifest = {
                "rank": rank,
                "world_size": runner.vllm_config.parallel_config.tensor_parallel_size,
                "layers": sorted(names),
                "layer_ids": sorted(ids),
                "shadow_layers": [],
                "native_bytes": native_bytes,
                "persistent_bytes": persistent,
                "source": str(Path(__file__).parent.resolve()),
                "sha256": source_fingerprint(),
                "verified": True,
            }
            runner._oscar_manifest = manifest
            print(READY_MARKER + json.dumps(manifest, sort_keys=True), flush=True)
        return caches

    Worker.determine_available_memory = determine_available_memory
    Runner.initialize_kv_cache_tensors = initialize_kv_cache_tensors
    Worker._oscar_memory_hook = True



def validate_ready(log: str, expected_sha: str | None = None) -> dict:
    """delivery/check_ready.py:8-29 — the READY manifests of a server log, by rank.

    Every tensor-parallel rank must have printed one verified, non-empty
    manifest; the ranks must agree on world size and layer coverage; each
    manifest's source fingerprint must equal ``expected_sha`` (or the first
    rank's); and the log must hold no injection failure or traceback."""
    records = {}
    for line in log.splitlines():
        at = line.find(READY_MARKER)
        if at < 0:
            continue
        record = json.loads(line[at + len(READY_MARKER):])
        if not record.get("verified") or not record.get("layers"):
            raise ValueError("Unverified or empty layer manifest")
        records[record["rank"]] = record
    if not records:
        raise ValueError("No verified cache initialization manifests")
    first = next(iter(records.values()))
    if set(records) != set(range(first["world_size"])):
        raise ValueError("Missing tensor-parallel rank manifests")
    want_sha = expected_sha or first["sha256"]
    for record in records.values():
        if record["world_size"] != first["world_size"] or record["layers"] != first["layers"]:
            raise ValueError("Ranks disagree about model coverage")
        if record["sha256"] != want_sha:
            raise ValueError("Worker source does not match this checkout")
    if INJECTION_FAILED in log or "Traceback (most recent call last)" in log:
        raise ValueError("Server log contains initialization/runtime failure")
    return records
