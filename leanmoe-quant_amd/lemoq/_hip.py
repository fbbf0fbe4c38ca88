"""ctypes binding of ``liblemoq_hip.so`` (the C-ABI declared in ``include/lemoq_hip.h``).

The library is built in-tree by ``lemoq.build.build_library()`` (hipcc,
``--offload-arch=gfx950``) into ``lemoq/_lib/liblemoq_hip.so``.  Loading it is
cheap and works without a GPU (the CPU test-suite checks the exported
symbols); every compute call needs a ROCm device.

There is deliberately no fallback: when the library is missing or a tensor is
not on a ROCm device, the operators raise instead of computing on the CPU.
"""

from __future__ import annotations

import ctypes
import os
from typing import Any

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib")
LIB_NAME = "liblemoq_hip.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)

ABI_VERSION = 8

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float


class LemoqOlmoeLayer(ctypes.Structure):
    """Mirror of ``LemoqOlmoeLayer`` in include/lemoq_hip.h (field order matters)."""

    _fields_ = [
        (name, _P)
        for name in (
            "ln_in",
            "ln_post",
            "q_norm",
            "k_norm",
            "qkv_codes",
            "qkv_scale",
            "o_codes",
            "o_scale",
            "router",
            "gu_codes",
            "gu_scale",
            "dn_codes",
            "dn_scale",
            "kc",
            "ks",
            "vc",
            "vs",
        )
    ]


class LemoqOlmoeStep(ctypes.Structure):
    """Mirror of ``LemoqOlmoeStep`` in include/lemoq_hip.h (field order matters)."""

    _fields_ = [
        ("hidden", _I64),
        ("heads", _I64),
        ("head_dim", _I64),
        ("ffn", _I64),
        ("num_experts", _I64),
        ("top_k", _I64),
        ("vocab", _I64),
        ("group", _I64),
        ("num_layers", _I64),
        ("max_seq", _I64),
        ("num_splits", _I64),
        ("norm_topk_prob", _I64),
        ("eps", _F),
        ("qk_scale", _F),
        ("clip_qkv", _F),
        ("layers", ctypes.POINTER(LemoqOlmoeLayer)),
        ("embed", _P),
        ("final_norm", _P),
        ("lm_codes", _P),
        ("lm_scale", _P),
        ("cos_tab", _P),
        ("sin_tab", _P),
        ("token", _P),
        ("pos", _P),
        ("filled", _P),
        ("prompt", _P),
        ("prompt_len", _I64),
        ("history", _P),
        ("history_len", _I64),
        ("h", _P),
        ("xn", _P),
        ("qkv", _P),
        ("q_rot", _P),
        ("attn", _P),
        ("part_m", _P),
        ("part_l", _P),
        ("part_acc", _P),
        ("router_logits", _P),
        ("top_w", _P),
        ("top_i", _P),
        ("act", _P),
        ("logits", _P),
        ("am_val", _P),
        ("am_idx", _P),
        ("am_len", _I64),
        ("o_part", _P),
        ("h_mid", _P),
        ("kv_fp16", _I64),
        ("weight_bits", _I64),
        ("lm_f16", _P),
    ]


# name -> (restype, argtypes); every symbol the header declares.
SIGNATURES: dict[str, tuple[Any, list[Any]]] = {
    "lemoq_status_string": (ctypes.c_char_p, [_I]),
    "lemoq_abi_version": (_I, []),
    "lemoq_rtn_quantize_w8": (_I, [_P, _I64, _I64, _I64, _P, _P, _P, _P]),
    "lemoq_rtn_quantize": (_I, [_P, _I64, _I64, _I64, _I, _I, _P, _P, _P, _P, _P, _P]),
    "lemoq_mxfp4_quantize": (_I, [_P, _I64, _I64, _P, _P, _P]),
    "lemoq_gemv_q": (_I, [_P, _I64, _I64, _P, _I, _P, _P, _I, _I64, _I64, _I64, _P, _I, _P]),
    "lemoq_gemv_q_x32": (_I, [_P, _I64, _I64, _P, _I, _P, _P, _I, _I64, _I64, _I64, _P, _I, _P]),
    "lemoq_dequant_q": (_I, [_P, _I, _P, _P, _I, _I64, _I64, _I64, _P, _I64, _I64, _I, _P]),
    "lemoq_fake_quant_rows": (_I, [_P, _I64, _I64, _P, _P]),
    "lemoq_moe_gate_up_w4": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P]),
    "lemoq_moe_gate_up_w4_routed": (
        _I, [_P, _P, _P, _P, _I64, _I, _I64, _I64, _I64, _I64, _P, _P, _P, _P]),
    "lemoq_gemv_q_residual": (_I, [_P, _I64, _I64, _P, _I, _P, _P, _I, _I64, _I64, _I64, _P, _P, _P]),
    "lemoq_gemv_q_rmsnorm": (
        _I, [_P, _P, _I64, _I64, _I64, _P, _F, _P, _P, _I, _P, _P, _I, _I64, _I64, _I64, _P, _I, _P]),
    "lemoq_attn_merge_o_proj_w4": (_I, [_P, _P, _P, _I64, _I64, _I64, _P, _P, _I64, _I64, _P, _P]),
    "lemoq_moe_down_w4": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "lemoq_gemv_w8": (_I, [_P, _I64, _I64, _P, _P, _I64, _I64, _I64, _P, _I, _P]),
    "lemoq_gemv_w8_fused": (
        _I,
        [_P, _P, _I64, _P, _F, _P, _P, _P, _I64, _I64, _I64, _P, _P, _P],
    ),
    "lemoq_moe_gate_up_w8": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P]),
    "lemoq_moe_down_w8": (
        _I,
        [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P],
    ),
    "lemoq_attn_merge_o_proj_w8": (_I, [_P, _P, _P, _I64, _I64, _I64, _P, _P, _I64, _I64, _P, _P]),
    "lemoq_router_logits_resid": (_I, [_P, _I64, _P, _P, _F, _I64, _P, _I64, _P, _P, _P, _P]),
    "lemoq_attn_split_f16": (
        _I,
        [_P, _P, _P, _I64, _P, _I64, _I64, _I64, _F, _P, _P, _P, _P],
    ),
    "lemoq_attn_split_i8": (
        _I,
        [_P, _P, _P, _P, _P, _I64, _I64, _P, _I64, _I64, _I64, _F, _P, _P, _P, _P],
    ),
    "lemoq_attn_merge": (_I, [_P, _P, _P, _I64, _I64, _I64, _P, _P]),
    "lemoq_rmsnorm": (_I, [_P, _I64, _I64, _P, _F, _P, _P]),
    "lemoq_rope": (
        _I,
        [_P, _I64, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _I64, _P],
    ),
    "lemoq_kv_write_f16": (_I, [_P, _P, _I64, _P, _P, _I64, _P, _I64, _I64, _P]),
    "lemoq_kv_write_i8": (_I, [_P, _P, _I64, _I64, _P, _P, _P, _P, _I64, _I64, _P, _P]),
    "lemoq_kv_quantize_rows": (_I, [_P, _I64, _I64, _P, _P, _P]),
    "lemoq_route_topk": (_I, [_P, _I, _I64, _I64, _I64, _I64, _I, _P, _P, _P]),
    "lemoq_route_topk_splitk": (_I, [_P, _I64, _I64, _I64, _I64, _I, _P, _P, _P]),
    "lemoq_router_topk_fused": (
        _I,
        [_P, _P, _F, _I64, _P, _I64, _I64, _I, _P, _P, _P, _P, _P, _P],
    ),
    "lemoq_qk_norm_rope_kv_i8": (
        _I,
        [
            _P, _I64, _I64, _P, _P, _F, _P, _P, _P, _P, _P, _P, _P, _P,
            _I64, _I64, _P, _P, _I64, _P, _F, _P,
        ],
    ),
    "lemoq_argmax_advance": (_I, [_P, _I64, _P, _P, _P, _P, _I64, _P, _I64, _P]),
    "lemoq_olmoe_decode_step": (_I, [ctypes.POINTER(LemoqOlmoeStep), _P]),
    "lemoq_read_probe": (_I, [_P, _I64, _P, _I64, _P]),
    "lemoq_copy_probe": (_I, [_P, _P, _I64, _I64, _P]),
    "lemoq_lm_head_argmax_w8": (
        _I,
        [_P, _P, _F, _P, _P, _I64, _I64, _I64, _P, _P, _P, _I64, _P, _P, _P, _P, _I64, _P, _I64, _P],
    ),
    "lemoq_lm_head_argmax_w8_dq": (
        _I,
        [_P, _P, _F, _P, _P, _I64, _I64, _I64, _P, _P, _P, _I64, _P, _P, _P, _P, _I64, _P, _I64, _P],
    ),
    "lemoq_lm_head_argmax_f16": (
        _I,
        [_P, _P, _F, _P, _I64, _I64, _P, _P, _P, _I64, _P, _P, _P, _P, _I64, _P, _I64, _P],
    ),
    "lemoq_lm_head_argmax_parts": (_I64, [_I64]),
    "lemoq_router_logits": (_I, [_P, _P, _F, _I64, _P, _I64, _P, _P, _P]),
    "lemoq_attn_split_fused_i8": (
        _I,
        [_P, _I64, _I64, _P, _P, _F, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _F, _P, _P, _P, _F, _P],
    ),
    "lemoq_attn_split_fused_f16": (
        _I,
        [_P, _I64, _I64, _P, _P, _F, _P, _P, _P, _P, _P, _I64, _I64, _I64, _F, _P, _P, _P, _F, _P],
    ),
    "lemoq_moe_gate_up_w8_routed": (
        _I,
        [_P, _P, _P, _P, _I64, _I, _I64, _I64, _I64, _I64, _P, _P, _P, _P],
    ),
    "lemoq_gemm_w8": (_I, [_P, _I64, _I64, _I64, _P, _P, _P, _I64, _I64, _P, _I64, _P, _I64, _P]),
    "lemoq_gemm_f16": (_I, [_P, _I64, _I64, _I64, _P, _I64, _P, _I64, _P]),
    "lemoq_gemm_f16_splitk": (_I, [_P, _I64, _I64, _I64, _P, _I64, _P, _I64, _I64, _P, _P]),
    "lemoq_gemm_f16_splitk_noalloc": (_I, [_P, _I64, _I64, _I64, _P, _I64, _P, _I64, _I64, _P]),
    "lemoq_gather_rows": (_I, [_P, _I64, _I64, _P, _I64, _P, _P]),
    "lemoq_qk_norm_rope_kv_i8_rows": (
        _I,
        [_P, _I64, _I64, _I64, _P, _P, _F, _P, _P, _I64, _P, _P, _P, _P, _P, _I64, _I64, _P, _P, _I64, _F, _P],
    ),
    "lemoq_attn_prefill_f16": (_I, [_P, _I64, _P, _P, _I64, _I64, _I64, _I64, _F, _P, _I64, _P]),
    "lemoq_moe_prefill_max_tiles": (_I64, [_I64, _I64]),
    "lemoq_moe_prefill_sort": (_I, [_P, _P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _I64, _P]),
    "lemoq_moe_prefill_gate_up": (_I, [_P, _I64, _P, _P, _I64, _P, _P, _I64, _I64, _P, _P]),
    "lemoq_moe_prefill_down": (_I, [_P, _I64, _P, _P, _P, _I64, _P, _P, _I64, _I64, _P, _P]),
    "lemoq_moe_prefill_combine": (_I, [_P, _P, _I64, _I64, _I64, _P, _P, _P]),
    "lemoq_moe_prefill_combine_norm": (_I, [_P, _P, _I64, _I64, _I64, _P, _P, _P, _F, _P, _P]),
}


class HipLibraryError(RuntimeError):
    """The native library is missing, stale or reported an error."""


_LIB: ctypes.CDLL | None = None


def library_available() -> bool:
    return os.path.exists(LIB_PATH)


def unavailable_reason() -> str | None:
    """Why the HIP operators cannot run here, or None when they can (the library is
    built, loads with this ABI, and a ROCm device is visible).  Never raises."""
    if not os.path.exists(LIB_PATH):
        return "lemoq HIP library not built (%s missing)" % LIB_PATH
    try:
        load()
    except Exception as exc:  # noqa: BLE001
        return "lemoq HIP library does not load: %s" % exc
    try:
        import torch  # noqa: PLC0415

        if not torch.cuda.is_available() or torch.version.hip is None:
            return "no ROCm device is visible"
    except Exception as exc:  # noqa: BLE001
        return "torch is unavailable (%s)" % type(exc).__name__
    return None


def load() -> ctypes.CDLL:
    """Load (once) and type the C-ABI library.  Raises when it is missing."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise HipLibraryError(
            "lemoq HIP library not built: %s is missing. Run "
            "`python -c 'import __graft_entry__ as g; g.build()'` (hipcc, gfx950)." % LIB_PATH
        )
    # torch first: its bundled libamdhip64 (soname libamdhip64.so.7) must be
    # the runtime our library binds to, so both share one HIP context.
    import torch  # noqa: F401,PLC0415

    lib = ctypes.CDLL(LIB_PATH)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    ver = int(lib.lemoq_abi_version())
    if ver != ABI_VERSION:
        raise HipLibraryError("liblemoq_hip ABI %d != expected %d; rebuild" % (ver, ABI_VERSION))
    _LIB = lib
    return lib


def call(name: str, *args: Any) -> None:
    """Call a status-returning entry point; non-zero status -> exception."""
    lib = load()
    rc = int(getattr(lib, name)(*args))
    if rc != 0:
        msg = lib.lemoq_status_string(rc)
        text = msg.decode() if msg else "?"
        if rc in (-1, -2):
            raise ValueError("%s rejected its arguments: %s (status %d)" % (name, text, rc))
        if rc == -3:
            raise NotImplementedError("%s: %s (status %d)" % (name, text, rc))
        if rc == -4:
            raise ValueError("%s: %s (status %d)" % (name, text, rc))
        raise HipLibraryError("%s failed: %s (hipError %d)" % (name, text, rc))


def ptr(t: Any) -> int | None:
    """Device address of a tensor (None for None)."""
    if t is None:
        return None
    return int(t.data_ptr())


def stream_of(device: Any = None) -> int:
    """Raw hipStream_t of torch's current stream on `device`."""
    import torch  # noqa: PLC0415

    return int(torch.cuda.current_stream(device).cuda_stream)


def require_rocm(*tensors: Any, what: str) -> None:
    """Loud refusal for CPU tensors: the operators have no CPU path."""
    import torch  # noqa: PLC0415

    for t in tensors:
        if t is None:
            continue
        if not torch.is_tensor(t):
            raise TypeError("%s: expected a tensor, got %s" % (what, type(t).__name__))
        if not t.is_cuda:
            raise RuntimeError(
                "%s needs ROCm device tensors (got %s); this build has no CPU fallback"
                % (what, t.device)
            )
    dev = {t.device for t in tensors if t is not None}
    if len(dev) > 1:
        raise ValueError("%s: tensors on different devices %s" % (what, sorted(map(str, dev))))
