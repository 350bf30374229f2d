"""vLLM general-plugin entry point (zero-edit runtime injection).

Entry point (pyproject): ``vllm.general_plugins: oscar_amd = oscar_amd.plugin:load_plugin``,
the same seam as the reference (oscar_ascend/plugin.py:73-181, pyproject.toml:12-13):

1. ``load_plugin()`` post-hooks ``Attention.__init__`` (idempotent);
2. after each Attention is built, ``_should_oscar`` selects the decoder
   FULL-attention layers of a hybrid model (MTP draft layers, sliding-window
   and sink layers are left native);
3. ``install_impl`` swaps the impl's class to a subclass of
   (OscarAttentionBackendImpl, native impl class) and runs ``_oscar_setup``;
   on any error the original class and ``__dict__`` are restored and the
   construction fails loudly;
4. the worker hooks (``integration.install_runner_hooks``) are installed
   once; failing to install them fails the construction the same way.

With ``OSCAR_ASCEND_CALIB=1`` (rotation calibration, ``oscar_amd.gen_rotations``)
no impl is swapped: every decoder full-attention module gets the capture
hook of ``oscar_amd.calib`` instead, whatever ``OSCAR_ASCEND_ENABLE`` says.

The reference's Ascend platform bootstrap (plugin.py:27-57) has no MI355X
counterpart: vLLM resolves the ROCm platform itself.
"""
from __future__ import annotations

import os

_HEARTBEAT: dict = {"loaded": 0, "layers": [], "errors": []}
_PATCHED = False
_SKIP_REASONS_LOGGED: set = set()
_COMBINED: dict = {}


def install_impl(impl, target_class) -> None:
    """plugin.py:60-70 — commit the class swap only if setup succeeds."""
    old_class, old_state = impl.__class__, impl.__dict__.copy()
    try:
        impl.__class__ = target_class
        impl._oscar_setup()
    except Exception:
        impl.__class__ = old_class
        impl.__dict__.clear()
        impl.__dict__.update(old_state)
        raise


def oscar_class_for(native_cls):
    """The OSCAR impl class mixed over a native impl class (cached)."""
    from .backend import OscarAttentionBackendImpl

    if issubclass(native_cls, OscarAttentionBackendImpl):
        return native_cls
    cls = _COMBINED.get(native_cls)
    if cls is None:
        cls = type(f"Oscar{native_cls.__name__}", (OscarAttentionBackendImpl, native_cls), {})
        _COMBINED[native_cls] = cls
    return cls


def _attention_class():
    for mod, name in (("vllm.attention.layer", "Attention"),
                      ("vllm.model_executor.layers.attention.attention", "Attention")):
        try:
            module = __import__(mod, fromlist=[name])
            return getattr(module, name)
        except Exception:  # noqa: BLE001 - try the next known location
            continue
    return None


def load_plugin() -> None:
    """plugin.py:73-181 — install the Attention.__init__ after-hook once."""
    global _PATCHED
    if _PATCHED:
        return
    if os.environ.get("OSCAR_ASCEND_ENABLE", "auto") == "0" and not _calibrating():
        print("[oscar-amd] OSCAR_ASCEND_ENABLE=0 -> native attention kept")
        _PATCHED = True
        return
    Attention = _attention_class()
    if Attention is None:
        _HEARTBEAT["errors"].append("vLLM Attention class not found")
        print("[oscar-amd] vLLM Attention class not found; OSCAR not injected")
        _PATCHED = True
        return
    orig_init = Attention.__init__

    def _patched_init(self, *args, **kwargs):
        orig_init(self, *args, **kwargs)
        if _calibrating():
            # plugin.py:103-111: calibration keeps the native impl and only
            # captures the unquantized Q/K/V of the engine's forward passes
            try:
                from .calib import register_attention_hook

                register_attention_hook(self)
            except Exception as e:  # noqa: BLE001 - a layer without captures is reported by finalize_cov
                print(f"[oscar-amd] calibration hook not registered on {getattr(self, 'layer_name', '?')}: {e}")
            return None
        impl = getattr(self, "impl", None)
        if impl is None or not _should_oscar(self, impl):
            return None
        try:
            install_impl(impl, oscar_class_for(type(impl)))
            from .integration import install_runner_hooks

            install_runner_hooks()
        except Exception as e:
            _HEARTBEAT["errors"].append(str(e))
            raise RuntimeError(f"[oscar-amd] injection failed: {getattr(self, 'layer_name', '?')}: {e}") from e
        _HEARTBEAT["loaded"] += 1
        _HEARTBEAT["layers"].append(
            f"{getattr(self, 'layer_name', '?')}:heads={impl.num_heads}/kv={impl.num_kv_heads}/d={impl.head_size}")
        return None

    Attention.__init__ = _patched_init
    _PATCHED = True
    print("[oscar-amd] plugin loaded: Attention.__init__ after-hook installed")


def _calibrating() -> bool:
    return os.environ.get("OSCAR_ASCEND_CALIB", "0") == "1"


def _is_hybrid_config(model_config) -> bool:
    """plugin.py:184-196 — is_hybrid, or layer_types containing non-attention layers."""
    if getattr(model_config, "is_hybrid", False):
        return True
    hf = getattr(model_config, "hf_text_config", None) or getattr(model_config, "hf_config", None)
    layer_types = getattr(hf, "layer_types", None) or []
    return any(lt != "attention" for lt in layer_types)


def _should_oscar(layer, impl) -> bool:
    """plugin.py:202-253 — decoder FULL-attention layers of hybrid models only."""
    layer_name = getattr(layer, "layer_name", "") or ""
    if ".mtp." in layer_name or layer_name.startswith("mtp."):
        if "mtp-draft" not in _SKIP_REASONS_LOGGED:
            _SKIP_REASONS_LOGGED.add("mtp-draft")
            print(f"[oscar-amd][SKIP] {layer_name}: MTP draft layer keeps its native KV")
        return False
    try:
        from vllm.config import get_current_vllm_config

        mc = get_current_vllm_config().model_config
        reasons = []
        if not _is_hybrid_config(mc):
            reasons.append("not-hybrid")
        at = getattr(impl, "attn_type", "decoder")
        if str(getattr(at, "value", at)) != "decoder":
            reasons.append(f"attn_type={at!r}")
        if getattr(impl, "sliding_window", None) is not None:
            reasons.append("sliding-window")
        if getattr(impl, "sinks", None) is not None:
            reasons.append("sinks")
        if reasons:
            key = ",".join(reasons)
            if key not in _SKIP_REASONS_LOGGED:
                _SKIP_REASONS_LOGGED.add(key)
                print(f"[oscar-amd][SKIP] {layer_name}: {key}")
            return False
        return True
    except Exception as e:  # noqa: BLE001 - no engine config: leave the layer native
        print(f"[oscar-amd][SKIP] _should_oscar: {e}")
        return False


def heartbeat() -> dict:
    """plugin.py:265-267."""
    return dict(_HEARTBEAT)
