"""The engine seams around cache allocation on the device: the memory hook's
plan, then the cache hook over device caches, with the library building the
MFMA rotation operands and the window arena living in HBM (reference
tests/test_backend.py:255-317 with real buffers).  The persistent bytes the
cache hook counts must equal the budget's per-layer term, and one verified
READY manifest is printed."""
import pytest
import torch

from oscar_amd import integration
from tests.fake_engine import HEAD, Engine

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("block_size,hk,heads", [(32, 1, 6), (128, 2, 12)])
def test_hooks_on_device_caches(monkeypatch, capsys, device, block_size, hk, heads):
    engine = Engine(device, layer_ids=(1, 3), layer_types=["linear_attention", "full_attention"] * 2,
                    block_size=block_size, num_kv_heads=hk, num_heads=heads)
    engine.install(monkeypatch)
    integration.install_runner_hooks()
    worker = engine.Worker()
    budget = worker.determine_available_memory()
    caches = worker.model_runner.initialize_kv_cache_tensors(engine.kv_config(budget))
    torch.cuda.synchronize()
    record = integration.validate_ready(capsys.readouterr().out, integration.source_fingerprint())[0]
    per_layer = integration.fixed_bytes_per_layer(HEAD, hk, block_size, 64, 64, 256, True)
    assert record["layer_ids"] == [1, 3] and record["persistent_bytes"] == 2 * per_layer
    for name, layer in engine.layers.items():
        assert layer.impl.key_cache is caches[name][0]
        rk, rv, op_k, op_v = layer._oscar_rot_ops
        assert rk.device.type == "cuda" and op_k.numel() == integration.ROTATION_OPERAND_BYTES
        assert torch.count_nonzero(op_k).item() > 0 and torch.equal(op_k, op_v)
        assert layer._oscar_stage_k.device.type == "cuda"
        assert layer._oscar_stage_kimg is not None
        assert (layer._oscar_slot_owner == -1).all().item()
