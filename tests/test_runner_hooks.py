"""The engine seams around cache allocation, with vLLM's v1 worker classes
replaced by fakes (tests/fake_engine.py), restating the reference's
tests/test_backend.py:218-243 (READY manifests) and 255-317 (the hook bodies):
the memory hook shrinks the KV budget to whole blocks after the OSCAR
persistent buffers, the cache hook binds caches, rotations and window arenas,
checks the actual bytes against the plan and prints one verified manifest.

CPU only: the MFMA rotation operand (a kernel call) is replaced by an empty
buffer of the library's operand size; tests/test_gpu_runner_hooks.py runs the
same hooks with real device caches and operands."""
import json
from types import SimpleNamespace as NS

import pytest
import torch

from oscar_amd import integration, plugin
from oscar_amd.kernels import quant
from tests.fake_engine import HEAD, Engine


@pytest.fixture
def no_operand_kernel(monkeypatch):
    monkeypatch.setattr(quant, "rotation_operand",
                        lambda R: torch.zeros(integration.ROTATION_OPERAND_BYTES, dtype=torch.uint8))


def start(engine, monkeypatch):
    engine.install(monkeypatch)
    integration.install_runner_hooks()
    return engine.Worker()


def expected_fixed(engine, num_layers=1, hk=1, heads=6, window=True):
    per_layer = integration.fixed_bytes_per_layer(HEAD, hk, engine.block_size, 64, 64, 256, window)
    workspace = integration.decode_workspace_bytes(4, hk, heads, 4, 4096)
    return num_layers * per_layer + workspace + integration.NOALLOC_SCRATCH_BYTES


def test_hooks_budget_then_initialize_and_report(monkeypatch, capsys, no_operand_kernel):
    engine = Engine("cpu")
    worker = start(engine, monkeypatch)
    budget = worker.determine_available_memory()
    out = capsys.readouterr().out
    plan = worker.model_runner._oscar_memory_plan
    fixed = expected_fixed(engine)
    assert plan == {"available": 200 * 10 ** 6, "native": engine.block_bytes, "shadow": 0, "fixed": fixed,
                    "budget": budget}
    assert budget % engine.block_bytes == 0 and budget + fixed <= plan["available"]
    assert plan["available"] - fixed - budget < engine.block_bytes
    assert worker.available_kv_cache_memory_bytes == budget
    assert json.loads(out.split("[oscar-amd] MEMORY ", 1)[1]) == plan
    # the spec dict handed to vLLM's grouping is a copy holding every layer
    assert engine.groups_calls == [sorted(engine.specs)]

    caches = worker.model_runner.initialize_kv_cache_tensors(engine.kv_config(budget))
    name = next(iter(engine.layers))
    layer = engine.layers[name]
    assert layer.impl.key_cache is caches[name][0] and layer.impl.value_cache is caches[name][1]
    assert layer._oscar_stage_ready and layer._oscar_stage_k.shape[1] == engine.block_size
    assert torch.equal(layer._oscar_rots[0], torch.eye(HEAD))
    assert not hasattr(engine.Runner.compilation_config.static_forward_context[engine.native_name], "_oscar_rots")
    records = integration.validate_ready(capsys.readouterr().out, integration.source_fingerprint())
    record = records[0]
    assert record["layers"] == [name] and record["layer_ids"] == [0] and record["shadow_layers"] == []
    assert record["native_bytes"] == engine.kv_config(budget).kv_cache_tensors[0].size
    per_layer = integration.fixed_bytes_per_layer(HEAD, 1, engine.block_size, 64, 64, 256, True)
    assert record["persistent_bytes"] == per_layer
    assert worker.model_runner._oscar_manifest == record


@pytest.mark.parametrize("hk,heads", [(1, 6), (2, 12)])
def test_budget_covers_several_layers_without_window(monkeypatch, capsys, no_operand_kernel, hk, heads):
    engine = Engine("cpu", layer_ids=(3, 7), layer_types=["linear_attention"] * 3 + ["full_attention"]
                    + ["linear_attention"] * 3 + ["full_attention"], num_kv_heads=hk, num_heads=heads,
                    window=False)
    worker = start(engine, monkeypatch)
    budget = worker.determine_available_memory()
    assert worker.model_runner._oscar_memory_plan["fixed"] == expected_fixed(engine, 2, hk, heads, False)
    worker.model_runner.initialize_kv_cache_tensors(engine.kv_config(budget))
    record = integration.validate_ready(capsys.readouterr().out)[0]
    assert record["layer_ids"] == [3, 7]
    assert record["persistent_bytes"] == 2 * integration.fixed_bytes_per_layer(HEAD, hk, 32, 0, 0, 0, False)
    assert not getattr(next(iter(engine.layers.values())), "_oscar_stage_ready", False)


def test_no_oscar_layers_leaves_budget_alone(monkeypatch, capsys):
    engine = Engine("cpu", layer_ids=())
    worker = start(engine, monkeypatch)
    assert worker.determine_available_memory() == 200 * 10 ** 6
    worker.model_runner.initialize_kv_cache_tensors(engine.kv_config(10 ** 6))
    assert "[oscar-amd]" not in capsys.readouterr().out


def test_hooks_install_once(monkeypatch):
    engine = Engine("cpu")
    engine.install(monkeypatch)
    integration.install_runner_hooks()
    hooked = (engine.Worker.determine_available_memory, engine.Runner.initialize_kv_cache_tensors)
    integration.install_runner_hooks()
    assert (engine.Worker.determine_available_memory, engine.Runner.initialize_kv_cache_tensors) == hooked
    assert engine.Worker._oscar_memory_hook


def test_hooks_need_the_v1_worker(monkeypatch):
    import sys

    monkeypatch.setitem(sys.modules, "vllm.v1.worker.gpu_worker", None)
    with pytest.raises(RuntimeError, match="v1 worker"):
        integration.install_runner_hooks()


@pytest.mark.parametrize("override,match", [
    ({"cache_config.num_gpu_blocks_override": 64}, "num_gpu_blocks_override"),
    ({"parallel_config.data_parallel_size": 2}, "DP=1"),
    ({"parallel_config.pipeline_parallel_size": 2}, "PP=1"),
])
def test_unsupported_engine_settings_rejected(monkeypatch, override, match):
    worker = start(Engine("cpu", overrides=override), monkeypatch)
    with pytest.raises(ValueError, match=match):
        worker.determine_available_memory()


def test_budget_that_holds_no_block_rejected(monkeypatch):
    engine = Engine("cpu", free_bytes=3 * 10 ** 6)
    worker = start(engine, monkeypatch)
    with pytest.raises(ValueError, match="OSCAR"):
        worker.determine_available_memory()
    engine.provisional = NS(kv_cache_tensors=[], num_blocks=0)
    with pytest.raises(ValueError, match="No native cache blocks"):
        worker.determine_available_memory()


def test_initialize_without_plan_or_over_budget_fails(monkeypatch, no_operand_kernel):
    engine = Engine("cpu")
    worker = start(engine, monkeypatch)
    with pytest.raises(RuntimeError, match="memory plan"):
        worker.model_runner.initialize_kv_cache_tensors(engine.kv_config(10 ** 6))
    budget = worker.determine_available_memory()
    worker.model_runner._oscar_memory_plan["available"] = budget
    with pytest.raises(RuntimeError, match="exceeds profiled budget"):
        worker.model_runner.initialize_kv_cache_tensors(engine.kv_config(budget))


def test_initialize_with_a_layer_left_native_fails(monkeypatch, no_operand_kernel):
    engine = Engine("cpu", layer_types=["full_attention", "full_attention"])
    worker = start(engine, monkeypatch)
    budget = worker.determine_available_memory()
    with pytest.raises(RuntimeError, match="Incomplete OSCAR layers"):
        worker.model_runner.initialize_kv_cache_tensors(engine.kv_config(budget))


# ---------------------------------------------------------------- READY manifests
def ready_line(record):
    return integration.READY_MARKER + json.dumps(record)


def test_incomplete_layer_and_rank_manifests_fail():
    record = {"rank": 0, "world_size": 2, "layers": ["layer.1"], "verified": True, "sha256": "a"}
    with pytest.raises(ValueError, match="Missing tensor-parallel rank"):
        integration.validate_ready(ready_line(record))
    logs = ready_line(record) + "\n" + ready_line(dict(record, rank=1))
    assert sorted(integration.validate_ready(logs, "a")) == [0, 1]
    with pytest.raises(ValueError, match="does not match"):
        integration.validate_ready(logs, "stale")
    with pytest.raises(ValueError, match="disagree"):
        integration.validate_ready(ready_line(record) + "\n" + ready_line(dict(record, rank=1, layers=["x"])))
    with pytest.raises(ValueError, match="Unverified"):
        integration.validate_ready(ready_line(dict(record, verified=False)))
    with pytest.raises(ValueError, match="No verified"):
        integration.validate_ready("engine started\n")
    with pytest.raises(ValueError, match="failure"):
        integration.validate_ready(logs + "\nTraceback (most recent call last):\n")
    with pytest.raises(ValueError, match="failure"):
        integration.validate_ready(logs + "\n[oscar-amd] injection failed: model.layers.0: boom\n")
    # the marker may follow a logger prefix
    assert integration.validate_ready("(Worker pid=7) " + ready_line(dict(record, world_size=1)))[0]["rank"] == 0


# ---------------------------------------------------------------- plugin -> hooks
def test_plugin_injects_impl_and_installs_hooks(monkeypatch, capsys, no_operand_kernel):
    """Attention.__init__ after-hook (plugin.py:73-181): the impl class is swapped,
    then the runner hooks are installed; a second layer does not wrap them twice."""
    import sys
    from types import ModuleType

    from oscar_amd.backend import OscarAttentionBackendImpl

    engine = Engine("cpu")
    engine.install(monkeypatch)

    class NativeImpl:
        def __init__(self):
            self.head_size, self.num_kv_heads, self.num_heads = HEAD, 1, 6
            self.scale = HEAD ** -0.5
            self.attn_type = "decoder"
            self.sliding_window = self.sinks = None

    class Attention:
        def __init__(self, layer_name):
            self.layer_name = layer_name
            self.impl = NativeImpl()

    model_config = NS(hf_text_config=NS(layer_types=["full_attention", "linear_attention"]))
    for name, attrs in {"vllm.attention.layer": {"Attention": Attention},
                        "vllm.config": {"get_current_vllm_config": lambda: NS(model_config=model_config)}}.items():
        module = ModuleType(name)
        vars(module).update(attrs)
        monkeypatch.setitem(sys.modules, name, module)
    monkeypatch.setattr(plugin, "_PATCHED", False)
    monkeypatch.setattr(plugin, "_HEARTBEAT", {"loaded": 0, "layers": [], "errors": []})
    monkeypatch.delenv("OSCAR_ASCEND_ENABLE", raising=False)
    plugin.load_plugin()
    first = Attention("model.layers.0.self_attn.attn")
    hooked = engine.Worker.determine_available_memory
    second = Attention("model.layers.2.self_attn.attn")
    assert isinstance(first.impl, OscarAttentionBackendImpl) and isinstance(second.impl, NativeImpl)
    assert engine.Worker._oscar_memory_hook and engine.Worker.determine_available_memory is hooked
    assert plugin._HEARTBEAT["loaded"] == 2 and not plugin._HEARTBEAT["errors"]

    # without vLLM's worker module the injection fails loudly, as it does for a failed class swap
    monkeypatch.setattr(engine.Worker, "_oscar_memory_hook", False)
    monkeypatch.setitem(sys.modules, "vllm.v1.worker.gpu_worker", None)
    with pytest.raises(RuntimeError, match="injection failed"):
        Attention("model.layers.4.self_attn.attn")
    assert plugin._HEARTBEAT["errors"]
