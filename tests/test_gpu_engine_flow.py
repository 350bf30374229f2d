"""The drop-in end to end, with vLLM replaced by fakes (tests/fake_engine.py
and a fake Attention class): the plugin swaps the impl of a decoder
full-attention layer as vLLM builds it, the worker hooks budget memory and
bind the engine's device caches (READY manifest), then the engine's forward
calls run a prefill step (dense route, K4), an MTP step (paged route, K3) and
a DecodeOnly read without fresh K/V, each checked against the oracle layer
fed the same inputs (reference plugin.py:73-181, integration.py:47-195,
backend.py:239-319).  Tolerance: the bf16 contract |gpu - oracle| <= 2e-2 +
2^-8 |oracle| elementwise (the oracle runs in fp32)."""
import dataclasses
import sys
from types import ModuleType
from types import SimpleNamespace as NS

import pytest
import torch

from oracle import attention as oatt
from oracle.forward import OracleLayer
from oscar_amd import integration, plugin
from oscar_amd.backend import OscarAttentionBackendImpl, OscarAttentionState
from tests.fake_engine import HEAD, Engine
from tests.test_gpu_backend import within_bf16

pytestmark = pytest.mark.gpu
BS, HQ, HK = 32, 6, 1


class NativeImpl:
    def __init__(self):
        self.head_size, self.num_kv_heads, self.num_heads = HEAD, HK, HQ
        self.scale = HEAD ** -0.5
        self.attn_type = "decoder"
        self.sliding_window = self.sinks = None


class Attention(torch.nn.Module):
    def __init__(self, layer_name):
        super().__init__()
        self.layer_name = layer_name
        self.impl = NativeImpl()


def fake_vllm(monkeypatch):
    model_config = NS(hf_text_config=NS(layer_types=["linear_attention", "full_attention"]))
    for name, attrs in {"vllm.attention.layer": {"Attention": Attention},
                        "vllm.config": {"get_current_vllm_config": lambda: NS(model_config=model_config)}}.items():
        module = ModuleType(name)
        vars(module).update(attrs)
        monkeypatch.setitem(sys.modules, name, module)
    monkeypatch.setattr(plugin, "_PATCHED", False)
    monkeypatch.setattr(plugin, "_HEARTBEAT", {"loaded": 0, "layers": [], "errors": []})
    for key in ("OSCAR_ASCEND_ENABLE", "OSCAR_ASCEND_CALIB", "OSCAR_ASCEND_K_ROTATION_PATH",
                "OSCAR_ASCEND_V_ROTATION_PATH"):
        monkeypatch.delenv(key, raising=False)
    monkeypatch.setenv("OSCAR_ASCEND_SINK_TOKENS", "32")
    monkeypatch.setenv("OSCAR_ASCEND_RECENT_TOKENS", "64")
    monkeypatch.setenv("OSCAR_ASCEND_STAGING_TOKENS", "256")


def step_md(device, bt, qsl, seqs, slots, state=None):
    md = NS(num_actual_tokens=qsl[-1], slot_mapping=torch.tensor(slots, dtype=torch.int64),
            query_start_loc=torch.tensor(qsl), actual_seq_lengths_q=list(qsl[1:]), seq_lens=torch.tensor(seqs),
            seq_lens_cpu=torch.tensor(seqs), seq_lens_list=list(seqs), block_tables=bt)
    dev = NS(**{**vars(md), "slot_mapping": md.slot_mapping.to(device), "block_tables": bt.to(device)})
    if state is not None:
        md.attn_state = dev.attn_state = state
    return md, dev


def test_plugin_hooks_and_forward_routes(monkeypatch, capsys, device):
    fake_vllm(monkeypatch)
    engine = Engine(device, layer_ids=(), layer_types=["linear_attention", "full_attention"], block_size=BS,
                    blocks=16)
    engine.install(monkeypatch)
    plugin.load_plugin()
    attn = Attention("model.layers.1.self_attn.attn")
    assert isinstance(attn.impl, OscarAttentionBackendImpl) and engine.Worker._oscar_memory_hook
    attn.impl._oscar_cfg = dataclasses.replace(attn.impl._oscar, k_clip_ratio=0.96, v_clip_ratio=0.92)
    engine.add_module(attn)
    worker = engine.Worker()
    budget = worker.determine_available_memory()
    caches = worker.model_runner.initialize_kv_cache_tensors(engine.kv_config(budget))
    record = integration.validate_ready(capsys.readouterr().out, integration.source_fingerprint())[0]
    assert record["layer_ids"] == [1]

    rk, rv = attn._oscar_rots
    assert torch.equal(rk.cpu(), torch.eye(HEAD))
    olayer = OracleLayer(torch.zeros(16, BS, HK, HEAD, dtype=torch.int8), torch.zeros(16, BS, HK, HEAD, dtype=torch.int8),
                         torch.eye(HEAD), torch.eye(HEAD), HQ, HK, HEAD, attn.impl.scale, 0.96, 0.92, 32, 64, 256)
    bt = torch.tensor([[3, 9, 1, 14, 6, 0, 11, 2], [5, 12, 7, 4, 10, 8, 13, 15]], dtype=torch.int32)
    g = torch.Generator().manual_seed(61)
    kv_cache = caches[attn.layer_name]

    def run(q_lens, seqs, state=None, fresh=True):
        n = sum(q_lens)
        q = torch.randn(n, HQ, HEAD, generator=g).to(torch.bfloat16)
        k = torch.randn(n, HK, HEAD, generator=g).to(torch.bfloat16) if fresh else None
        v = torch.randn(n, HK, HEAD, generator=g).to(torch.bfloat16) if fresh else None
        qsl, slots = [0], []
        for i, (ql, s) in enumerate(zip(q_lens, seqs)):
            qsl.append(qsl[-1] + ql)
            slots += [int(bt[i][p // BS]) * BS + p % BS for p in range(s - ql, s)]
        md, mdd = step_md(device, bt, qsl, seqs, slots, state)
        out = attn.impl.forward(attn, q.to(device), None if k is None else k.to(device),
                                None if v is None else v.to(device), kv_cache, mdd,
                                output=torch.empty(n, HQ * HEAD, dtype=torch.bfloat16, device=device))
        torch.cuda.synchronize()
        if fresh:
            want = olayer.forward(q.float(), k.float(), v.float(), md)
        else:
            A = olayer.arena
            want = oatt.decode_only_ref(q.float(), olayer.k_cache, olayer.v_cache, bt, seqs, olayer.scale, HK, HEAD,
                                        (A.stage_k, A.stage_v, A.owner, A.sink_eff, olayer.recent))
        return out.cpu().float().view(n, HQ, HEAD), want.float()

    for got, want in (run([150, 90], [150, 90]),                     # prefill (dense route)
                      run([4, 3], [154, 93]),                        # MTP step (paged route)
                      run([1, 1], [154, 93], OscarAttentionState.DecodeOnly, fresh=False)):
        assert within_bf16(got, want)
