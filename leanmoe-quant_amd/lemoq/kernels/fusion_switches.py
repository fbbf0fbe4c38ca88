"""The decode path's fusion switches, as this build has them.

Mirrors the reference's ``src/lemoq/kernels/fusion_switches.py`` (the switch
names, their ``LEMOQ_*`` environment overrides, ``fusion_enabled`` /
``fusion_states`` / ``fusion_payload_fields``) so that code which queries or
records the switches keeps working.  The difference is what a switch can
select here.  The reference keeps both arms of every candidate (fused or the
ATen/HF original) for its A/B rounds; this build's decode step is one native
launch sequence with every candidate fused in, so only ``kv_int8`` has two
built arms (the KV-INT8 cache or the fp16 cache, ``DecodeSession(kv_cache=...)``).
Asking for an arm that is not built (``LEMOQ_PACKED_QKV=0``, say) is refused
with ``NotImplementedError`` by ``require_built`` -- which ``DecodeSession``
calls -- instead of being ignored.
"""

from __future__ import annotations

import os
from typing import Any

__all__ = [
    "BUILT_ARMS",
    "ENV_VARS",
    "FUSION_DEFAULTS",
    "fusion_enabled",
    "fusion_payload_fields",
    "fusion_states",
    "require_built",
]

# switch -> environment override (the reference's names, fusion_switches.py:42-50)
ENV_VARS: dict[str, str] = {
    "fused_rope": "LEMOQ_FUSED_ROPE",
    "fused_route": "LEMOQ_FUSED_ROUTE",
    "skip_mask_fill": "LEMOQ_SKIP_MASK_FILL",
    "packed_qkv": "LEMOQ_PACKED_QKV",
    "kv_direct_write": "LEMOQ_KV_DIRECT_WRITE",
    "lm_head_w8": "LEMOQ_LMHEAD_W8",
    "kv_int8": "LEMOQ_KV_INT8",
}

# every switch defaults to on, as the reference adopted them (:52-60)
FUSION_DEFAULTS: dict[str, bool] = {name: True for name in ENV_VARS}

# the states each switch can take in this build, and where the fused form lives
BUILT_ARMS: dict[str, tuple[bool, ...]] = {
    "fused_rope": (True,),       # RoPE inside the attention launch
    "fused_route": (True,),      # router logits launch + routing inside gate/up
    "skip_mask_fill": (True,),   # the split-KV kernels read only [0, filled)
    "packed_qkv": (True,),       # one q|k|v GEMV with the input norm
    "kv_direct_write": (True,),  # the new row written by the attention launch
    "lm_head_w8": (True,),       # W8 lm_head GEMV with the argmax partials
    "kv_int8": (True, False),    # KV-INT8 cache, or the fp16 cache
}


def fusion_enabled(name: str, env: dict[str, str] | None = None) -> bool:
    """Requested state: the environment override if set ("1" on, anything else
    off), else the default."""
    if name not in ENV_VARS:
        raise KeyError("unknown fusion switch %r; declared: %s" % (name, sorted(ENV_VARS)))
    source = os.environ if env is None else env
    raw = source.get(ENV_VARS[name])
    return FUSION_DEFAULTS[name] if raw is None else raw == "1"


def fusion_states(env: dict[str, str] | None = None) -> dict[str, bool]:
    """Requested state of every switch."""
    return {name: fusion_enabled(name, env) for name in ENV_VARS}


def fusion_payload_fields(env: dict[str, str] | None = None) -> dict[str, Any]:
    """One field per switch for a result's ``config`` block."""
    return fusion_states(env)


def require_built(env: dict[str, str] | None = None) -> dict[str, bool]:
    """The requested states, after checking that this build has each of them;
    raises ``NotImplementedError`` naming every switch whose arm is not built."""
    states = fusion_states(env)
    missing = sorted(n for n, v in states.items() if v not in BUILT_ARMS[n])
    if missing:
        raise NotImplementedError(
            "fusion switch(es) %s set off, but this build has only the fused form of %s (the unfused "
            "arms are the reference's A/B baselines); unset %s"
            % (missing, "it" if len(missing) == 1 else "them", ", ".join(ENV_VARS[n] for n in missing)))
    return states
