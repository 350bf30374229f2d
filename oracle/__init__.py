"""CPU oracle for the OSCAR INT2 KV-cache path — TEST INFRASTRUCTURE ONLY.

This package restates, in plain torch-CPU / numpy, the algorithm the reference
plugin (`oscar_ascend`) runs on its torch path.  It is the checker the HIP
kernels are compared against.  Nothing in the product package (`oscar_amd`)
imports it; only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline`
leg of `bench.py` may use it, and only as the checker or the timed CPU
baseline — never as the thing measured or shipped.

Modules (each function cites the reference file:line it follows):

* ``format``    — slot layout, per-vector INT2 quantize / pack / dequant,
                  fp16 little-endian meta (oscar_ascend/format.py).
* ``store``     — paged-slot scatter write and gather/dequant
                  (oscar_ascend/kernels/store_kernel.py).
* ``rotate``    — fp32 rotation + sort-based clip (oscar_ascend/backend.py).
* ``staging``   — FP32 sink/recent window arena: ensure / write / splice
                  (oscar_ascend/backend.py).
* ``attention`` — query layout, paged MTP oracle, chunked causal SDPA oracle,
                  single-query decode oracle, split reducer
                  (oscar_ascend/kernels/{paged_attention,decode_kernel}.py).
* ``forward``   — the impl-level composition: write, stage, read
                  (oscar_ascend/backend.py forward / _prefill_attention).
* ``quant_ref.c`` — an independent C restatement of the quantizer, built into
                  ``oracle/_build`` and cross-checked against ``format``.

Parity pinning: every function here is checked in ``tests/test_oracle_*.py``
against closed forms, the restated reference tests, brute force on tiny
inputs, and the golden vectors under ``tests/golden/`` (written by importing
the reference in the build container for the two functions nothing else
pins: the staging arena state and the impl-level forward composition).
"""
