"""A stand-in for the two vLLM v1 worker classes the OSCAR runner hooks wrap
(``vllm.v1.worker.gpu_worker.Worker``, ``vllm.v1.worker.gpu_model_runner.GPUModelRunner``)
and the two ``vllm.v1.core.kv_cache_utils`` functions the memory hook calls,
shaped like the reference's fakes (tests/test_backend.py:255-317): a runner
whose static forward context holds OSCAR layers and a native layer, a worker
whose profiler reports a fixed number of free bytes, and an engine allocator
that hands each layer its (K, V) cache pair."""
from __future__ import annotations

import dataclasses
import sys
from types import ModuleType
from types import SimpleNamespace as NS

import torch

from oscar_amd.backend import OscarAttentionBackendImpl

HEAD = 256


def make_impl(num_kv_heads=1, num_heads=6, sink=64, recent=64, staging=256, window=True):
    impl = OscarAttentionBackendImpl.__new__(OscarAttentionBackendImpl)
    impl.head_size, impl.num_kv_heads, impl.num_heads = HEAD, num_kv_heads, num_heads
    impl.scale = HEAD ** -0.5
    impl.key_cache = impl.value_cache = None
    impl._oscar_setup()
    impl._oscar_cfg = dataclasses.replace(impl._oscar, sink_tokens=sink, recent_tokens=recent,
                                          staging_tokens=staging if window else 0)
    return impl


class Engine:
    """One worker/runner pair over ``layer_ids`` OSCAR layers (plus one native
    layer the hooks must leave alone), ``blocks`` cache blocks of
    ``block_size`` tokens on ``device``."""

    def __init__(self, device, layer_ids=(0,), layer_types=("full_attention", "linear_attention"),
                 block_size=32, blocks=8, free_bytes=200 * 10 ** 6, num_kv_heads=1, num_heads=6,
                 window=True, tp=1, overrides=None, modules=None):
        """modules: {layer name: attention module} built elsewhere (by the
        plugin, say) to use instead of fresh OSCAR layers."""
        self.device = torch.device(device)
        self.block_size, self.blocks = block_size, blocks
        self.layers = {}
        for i in layer_ids if modules is None else ():
            name = f"model.layers.{i}.self_attn.attn"
            self.layers[name] = NS(layer_name=name, impl=make_impl(num_kv_heads, num_heads, window=window))
        self.layers.update(modules or {})
        self.native_name = "model.layers.99.linear_attn"
        ctx = dict(self.layers)
        ctx[self.native_name] = NS(layer_name=self.native_name, impl=NS())
        self.specs = {name: NS(block_size=block_size, num_kv_heads=num_kv_heads, head_size=HEAD,
                               head_size_v=HEAD) for name in ctx}
        # int8-geometry slots: D bytes per (token, kv head), K and V, every layer
        self.block_bytes = 2 * block_size * num_kv_heads * HEAD * len(ctx)
        self.provisional = NS(kv_cache_tensors=[NS(size=self.block_bytes * blocks)], num_blocks=blocks)
        self.allocated = None
        engine = self
        cfg = NS(
            cache_config=NS(num_gpu_blocks_override=None),
            parallel_config=NS(pipeline_parallel_size=1, data_parallel_size=1, tensor_parallel_size=tp),
            scheduler_config=NS(max_num_seqs=4),
            model_config=NS(max_model_len=4096),
            speculative_config=NS(num_speculative_tokens=3),
        )
        for key, value in (overrides or {}).items():
            section, field = key.split(".")
            setattr(getattr(cfg, section), field, value)

        class GPUModelRunner:
            compilation_config = NS(static_forward_context=ctx)
            vllm_config = cfg
            model_config = NS(hf_text_config=NS(layer_types=list(layer_types)))

            def get_kv_cache_spec(self):
                return engine.specs

            def initialize_kv_cache_tensors(self, kv_cache_config, kernel_block_sizes=None):
                engine.allocated = kv_cache_config
                shape = (engine.blocks, engine.block_size, num_kv_heads, HEAD)
                caches = {}
                for name in ctx:
                    caches[name] = tuple(torch.zeros(shape, dtype=torch.int8, device=engine.device)
                                         for _ in range(2))
                return caches

        class Worker:
            def __init__(self):
                self.model_runner = GPUModelRunner()

            def determine_available_memory(self):
                return free_bytes

        self.Runner, self.Worker = GPUModelRunner, Worker
        self.groups_calls = []
        self._ctx, self._heads = ctx, num_kv_heads

    def add_module(self, module):
        """Register one more attention module (e.g. built by the plugin after
        the fake worker modules were installed)."""
        self.layers[module.layer_name] = module
        self._ctx[module.layer_name] = module
        self.specs[module.layer_name] = NS(block_size=self.block_size, num_kv_heads=self._heads, head_size=HEAD,
                                           head_size_v=HEAD)
        self.block_bytes = 2 * self.block_size * self._heads * HEAD * len(self._ctx)
        self.provisional = NS(kv_cache_tensors=[NS(size=self.block_bytes * self.blocks)], num_blocks=self.blocks)

    def modules(self):
        engine = self

        def get_kv_cache_groups(cfg, specs):
            engine.groups_calls.append(sorted(specs))
            return ["group"]

        def get_kv_cache_config_from_groups(cfg, groups, available):
            return engine.provisional

        return {
            "vllm.v1.worker.gpu_worker": {"Worker": self.Worker},
            "vllm.v1.worker.gpu_model_runner": {"GPUModelRunner": self.Runner},
            "vllm.v1.core.kv_cache_utils": {
                "get_kv_cache_groups": get_kv_cache_groups,
                "get_kv_cache_config_from_groups": get_kv_cache_config_from_groups,
            },
        }

    def install(self, monkeypatch):
        """Put the fake modules into ``sys.modules`` for the test's duration."""
        for name, attrs in self.modules().items():
            module = ModuleType(name)
            vars(module).update(attrs)
            monkeypatch.setitem(sys.modules, name, module)

    def kv_config(self, budget):
        blocks = budget // self.block_bytes
        return NS(kv_cache_tensors=[NS(size=blocks * self.block_bytes)], num_blocks=blocks)
