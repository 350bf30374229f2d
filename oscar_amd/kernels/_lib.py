"""ctypes binding of the gfx950 HIP library (C ABI in include/oscar_amd.h).

The library is built in-tree (``oscar_amd/_oscar_hip.so``).  torch is imported
before the library is opened so that the library's ``libamdhip64.so.7``
dependency resolves to the HIP runtime torch already loaded: both then share
one runtime, one device context and torch's streams.

There is no fallback: a missing library, a failed load or a non-zero status
raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL load, see module doc)

LIB_PATH = Path(__file__).resolve().parents[1] / "_oscar_hip.so"

_c_i32, _c_i64, _c_sz, _c_p, _c_f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_float

# name -> (restype, argtypes); must list every symbol declared in include/oscar_amd.h.
SIGNATURES = {
    "oscar_rotation_operand_bytes": (_c_sz, [_c_i32]),
    "oscar_rotation_operand": (_c_i32, [_c_p, _c_p, _c_i32, _c_p]),
    "oscar_rotate_rows": (_c_i32, [_c_p, _c_i32, _c_i64, _c_i64, _c_i32, _c_p, _c_p, _c_i32, _c_i64, _c_p]),
    "oscar_quant_write": (_c_i32, [_c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_i64, _c_p, _c_p, _c_p,
                                   _c_p, _c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                   _c_i64, _c_i64, _c_i32, _c_i32, _c_p]),
    "oscar_quant_write_prerotated": (_c_i32, [_c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_i64, _c_p,
                                              _c_p, _c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64,
                                              _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_p]),
    "oscar_paged_decode_workspace_bytes": (_c_sz, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i64, _c_i32]),
    "oscar_paged_decode": (_c_i32, [_c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_i32, _c_p, _c_p,
                                    _c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                    _c_p, _c_i64, _c_i32, _c_p, _c_p, _c_i32, _c_i32, _c_i64,
                                    _c_p, _c_p, _c_p, _c_i32, _c_f32, _c_i32, _c_p, _c_p, _c_sz,
                                    _c_p]),
    "oscar_paged_decode_noalloc": (_c_i32, [_c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_i32, _c_p, _c_p,
                                            _c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                            _c_p, _c_i64, _c_i32, _c_p, _c_p, _c_i32, _c_i32, _c_i64,
                                            _c_p, _c_p, _c_p, _c_i32, _c_f32, _c_i32, _c_p, _c_p]),
    "oscar_paged_decode_rotated": (_c_i32, [_c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_i32, _c_p, _c_p,
                                            _c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                            _c_p, _c_i64, _c_i32, _c_p, _c_p, _c_i32, _c_i32, _c_i64,
                                            _c_p, _c_p, _c_p, _c_i32, _c_f32, _c_i32, _c_p, _c_p, _c_i64,
                                            _c_i32, _c_p, _c_sz, _c_p]),
    "oscar_step_write": (_c_i32, [_c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_p,
                                  _c_p, _c_p, _c_p, _c_p, _c_i32, _c_p, _c_p, _c_i32, _c_i64, _c_i64, _c_i64,
                                  _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_p, _c_p, _c_p, _c_p,
                                  _c_p, _c_i32, _c_i32, _c_i32, _c_p, _c_p, _c_p, _c_p]),
    "oscar_mtp_forward": (_c_i32, [_c_p, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_i32, _c_p]),
    "oscar_decode_only_workspace_bytes": (_c_sz, [_c_i32, _c_i32, _c_i32, _c_i64, _c_i32]),
    "oscar_decode_only": (_c_i32, [_c_p, _c_i32, _c_i32, _c_i32, _c_p, _c_p, _c_i32, _c_i64, _c_i64,
                                   _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i32,
                                   _c_p, _c_i32, _c_i64, _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32,
                                   _c_f32, _c_i32, _c_p, _c_p, _c_sz, _c_p]),
    "oscar_prefill_continuation": (_c_i32, [_c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_i32, _c_p,
                                            _c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                            _c_i64, _c_i64, _c_p, _c_i32, _c_i64, _c_p, _c_p, _c_p,
                                            _c_i32, _c_f32, _c_p, _c_p]),
    "oscar_staging_write": (_c_i32, [_c_p, _c_p, _c_i64, _c_p, _c_i32, _c_p, _c_p, _c_i32, _c_i32,
                                     _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_p, _c_p, _c_p, _c_p,
                                     _c_p, _c_p, _c_p, _c_p, _c_p]),
    "oscar_quant_write_window": (_c_i32, [_c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_i64, _c_p, _c_p, _c_p,
                                          _c_p, _c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                          _c_i64, _c_i64, _c_i32, _c_i32, _c_p, _c_p, _c_i32, _c_i32, _c_i32,
                                          _c_i32, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p]),
}

STATUS = {
    0: "ok",
    -1: "invalid argument",
    -2: "unsupported head size (kernels are written for D = 256)",
    -3: "workspace too small",
    -4: "kernel launch failed",
    -5: "unsupported cache geometry (slot widths, strides or alignment)",
}

_lib = None


class OscarKernelError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Open the library once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise OscarKernelError(
                f"OSCAR HIP library missing at {LIB_PATH}; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'`")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    status = getattr(load(), name)(*args)
    if status != 0:
        raise OscarKernelError(f"{name} failed: {STATUS.get(status, status)}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """The hipStream_t of the device's current stream (torch's own raw-stream
    query where it exists: no Stream object is built per call)."""
    if _raw_stream is not None:
        idx = device.index
        return _raw_stream(torch.cuda.current_device() if idx is None else idx)
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()
