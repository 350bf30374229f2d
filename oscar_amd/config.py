"""Plugin settings, read once per layer from ``OSCAR_ASCEND_*`` variables.

The variable names, defaults and rejections are the plugin surface a
deployment already sets (reference: oscar_ascend/config.py:71-97); the code
is written from that list of variables, defaults and rejections.

Variables (an unset, empty or unparsable numeric value means its default):

  OSCAR_ASCEND_HEAD_DIM          int    256   only when the caller gives none
  OSCAR_ASCEND_K_CLIP_RATIO      float  0.0   must lie in [0, 1]
  OSCAR_ASCEND_V_CLIP_RATIO      float  0.0   must lie in [0, 1]
  OSCAR_ASCEND_K_ROTATION_PATH   str    ""    empty: identity rotation
  OSCAR_ASCEND_V_ROTATION_PATH   str    ""
  OSCAR_ASCEND_SINK_TOKENS       int    64    negative counts as 0
  OSCAR_ASCEND_RECENT_TOKENS     int    256   negative counts as 0
  OSCAR_ASCEND_STAGING_TOKENS    int    8192  negative counts as 0
  OSCAR_ASCEND_GROUP_SIZE        int    0     anything else is rejected
  OSCAR_ASCEND_VERBOSE           flag   on    "0" turns it off
  OSCAR_ASCEND_USE_PAGED         switch on    when set, only "1" turns it on
                                              (as the reference reads it); any
                                              other value: every request takes
                                              the prefill-continuation kernel

USE_PAGED defaults to on here when the variable is unset (the reference
defaults it off until its NPU kernel was probed): short requests then take
the paged HIP decode kernel.  A set value is read as the reference reads it,
so OSCAR_ASCEND_USE_PAGED=0, =false or =off all turn the paged route off.
OSCAR_ASCEND_USE_TRITON, OSCAR_ASCEND_FUSED_PREP and OSCAR_ASCEND_ENABLE
select between the reference's own kernel variants; they are accepted and
have no effect, as there is a single HIP path.
"""
from __future__ import annotations

import math
import os
from dataclasses import dataclass
from typing import Callable, Mapping

from .format import BITS, HEAD_DIM, LEVELS, SLOT_SIZE

PREFIX = "OSCAR_ASCEND_"
PAGED_MAX_Q_LEN = 16          # longest request the paged decode takes (backend.py:277)


def _number(env: Mapping[str, str], name: str, parse: Callable[[str], float], default):
    text = env.get(PREFIX + name, "").strip()
    if not text:
        return default
    try:
        return parse(text)
    except ValueError:
        return default


def _count(env: Mapping[str, str], name: str, default: int) -> int:
    return max(0, _number(env, name, int, default))


def _flag(env: Mapping[str, str], name: str, default: bool) -> bool:
    """On unless set to "0" (config.py:90, VERBOSE)."""
    text = env.get(PREFIX + name)
    return default if text is None else text != "0"


def _switch(env: Mapping[str, str], name: str, default: bool) -> bool:
    """Off unless set to "1" (config.py:93, USE_PAGED); `default` when unset."""
    text = env.get(PREFIX + name)
    return default if text is None else text == "1"


@dataclass(frozen=True)
class OscarConfig:
    head_dim: int = HEAD_DIM
    k_clip_ratio: float = 0.0
    v_clip_ratio: float = 0.0
    k_rotation_path: str = ""
    v_rotation_path: str = ""
    sink_tokens: int = 64
    recent_tokens: int = 256
    staging_tokens: int = 8192
    use_paged: bool = True
    verbose: bool = True
    paged_max_q_len: int = PAGED_MAX_Q_LEN

    def __post_init__(self):
        for which, ratio in (("K", self.k_clip_ratio), ("V", self.v_clip_ratio)):
            if not (math.isfinite(ratio) and 0.0 <= ratio <= 1.0):
                raise ValueError(f"OSCAR {which} clip ratio {ratio!r} is outside [0, 1]")

    @property
    def window_enabled(self) -> bool:
        """The FP32 window exists when it has room and something to keep."""
        return self.staging_tokens > 0 and (self.sink_tokens > 0 or self.recent_tokens > 0)

    @property
    def levels(self) -> int:
        return LEVELS

    @property
    def data_bytes(self) -> int:
        """Packed code bytes of one vector (64 at D = 256)."""
        return (self.head_dim * BITS + 7) // 8

    @property
    def slot_bytes(self) -> int:
        return SLOT_SIZE            # 96 B in the K cache + 64 B in the V cache

    @classmethod
    def from_env(cls, head_dim: int | None = None, env: Mapping[str, str] | None = None) -> "OscarConfig":
        env = os.environ if env is None else env
        group = _number(env, "GROUP_SIZE", int, 0)
        if group != 0:
            raise ValueError(f"OSCAR quantizes whole vectors; OSCAR_ASCEND_GROUP_SIZE={group} is unsupported")
        return cls(
            head_dim=head_dim if head_dim is not None else _number(env, "HEAD_DIM", int, HEAD_DIM),
            k_clip_ratio=_number(env, "K_CLIP_RATIO", float, 0.0),
            v_clip_ratio=_number(env, "V_CLIP_RATIO", float, 0.0),
            k_rotation_path=env.get(PREFIX + "K_ROTATION_PATH", ""),
            v_rotation_path=env.get(PREFIX + "V_ROTATION_PATH", ""),
            sink_tokens=_count(env, "SINK_TOKENS", 64),
            recent_tokens=_count(env, "RECENT_TOKENS", 256),
            staging_tokens=_count(env, "STAGING_TOKENS", 8192),
            use_paged=_switch(env, "USE_PAGED", True),
            verbose=_flag(env, "VERBOSE", True),
        )
