"""oscar_amd — MI355X-native OSCAR INT2 KV-cache path.

Drop-in for the reference plugin's FULL-attention impl (oscar_ascend):

  plugin.py      vLLM general-plugin entry point (impl class surgery)
  config.py      OSCAR_ASCEND_* configuration
  format.py      160-byte logical slot layout constants
  rotation.py    per-layer orthogonal K/V rotation loading
  backend.py     the attention impl (write path, window arena, read path)
  integration.py memory budgeting of the persistent per-layer buffers
  kernels/       ctypes boundary to the gfx950 HIP library (_oscar_hip.so)
"""
from . import config, format  # noqa: F401

__version__ = "0.1.0"
__all__ = ["config", "format", "__version__"]
