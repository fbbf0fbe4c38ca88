"""OLMoE checkpoints in and out of the decode step's packed W8 layout.

The reference quantises a loaded HF model in place: RTN w8 per group of 128
along K for the attention linears and the fused experts, router kept fp16
(``benchmarks/runner.py:452-483``, ``moe_grouped_quant.quantize_fused_experts``
``src/lemoq/kernels/moe_grouped_quant.py:191-244``), or takes pre-packed
experts (``moe_static.py:467-504``).  This module does the same from the
checkpoint files, with no HF modules in between:

* ``shape_from_hf_config(cfg)``: ``OlmoeShape`` from an HF OLMoE ``config.json``.
* ``read_hf_state(path)``: the tensors of ``*.safetensors`` in a local
  checkpoint directory (host memory, no pickle).
* ``quantize_state_dict(sd, shape, device=..., quantizer=None)``: HF OLMoE
  state dict -> ``OlmoeW8Weights``.  Both expert layouts are accepted:
  transformers 5 (``mlp.experts.gate_up_proj`` (E, 2F, H), ``down_proj``
  (E, H, F)) and 4.x (``mlp.experts.{e}.gate_proj/up_proj/down_proj.weight``).
  q|k|v rows are concatenated (the ``PackedQKV`` order), gate rows precede up
  rows per expert, the lm_head is W8 (the embedding when tied).  The default
  quantizer is the device RTN kernel (``lemoq.quant.rtn.quantize_rtn``).
* ``load_hf_olmoe(path, device)``: the two above on a local directory.
* ``save_packed(w, path)`` / ``load_packed(path, device)``: the packed layout
  as safetensors plus ``lemoq_olmoe.json`` (the shape), loaded back bit for bit.
"""

from __future__ import annotations

import json
import os
from dataclasses import asdict, fields
from typing import Any, Callable, Mapping

import torch

from lemoq.model.olmoe import LayerW8, OlmoeShape, OlmoeW8Weights

__all__ = ["shape_from_hf_config", "read_hf_state", "quantize_state_dict", "load_hf_olmoe", "save_packed",
           "load_packed", "PACKED_META"]

PACKED_META = "lemoq_olmoe.json"
PACKED_TENSORS = "lemoq_olmoe.safetensors"
_FORMAT = "lemoq-olmoe-w8a16-g128-v1"

Quantizer = Callable[[Any, int], "tuple[Any, Any]"]


def shape_from_hf_config(cfg: Mapping[str, Any], *, group_size: int = 128) -> OlmoeShape:
    """``OlmoeShape`` from an HF OLMoE config dict; configurations the decode
    step does not implement raise ``NotImplementedError``."""
    heads = int(cfg["num_attention_heads"])
    kv_heads = int(cfg.get("num_key_value_heads") or heads)
    if kv_heads != heads:
        raise NotImplementedError("grouped-query attention (num_key_value_heads != num_attention_heads)")
    hidden = int(cfg["hidden_size"])
    head_dim = int(cfg.get("head_dim") or hidden // heads)
    theta = cfg.get("rope_theta")
    if theta is None:
        theta = (cfg.get("rope_parameters") or {}).get("rope_theta", 10000.0)
    return OlmoeShape(
        hidden=hidden,
        heads=heads,
        head_dim=head_dim,
        layers=int(cfg["num_hidden_layers"]),
        num_experts=int(cfg["num_experts"]),
        top_k=int(cfg["num_experts_per_tok"]),
        ffn=int(cfg["intermediate_size"]),
        vocab=int(cfg["vocab_size"]),
        eps=float(cfg.get("rms_norm_eps", 1e-5)),
        rope_theta=float(theta),
        norm_topk_prob=bool(cfg.get("norm_topk_prob", False)),
        group_size=int(group_size),
        clip_qkv=None if cfg.get("clip_qkv") is None else float(cfg["clip_qkv"]),
    )


def read_hf_state(path: str) -> dict[str, Any]:
    """All tensors of the ``*.safetensors`` files in ``path`` (CPU)."""
    from safetensors.torch import load_file  # noqa: PLC0415

    files = sorted(f for f in os.listdir(path) if f.endswith(".safetensors"))
    if not files:
        raise FileNotFoundError("no .safetensors files in %s" % path)
    sd: dict[str, Any] = {}
    for f in files:
        sd.update(load_file(os.path.join(path, f), device="cpu"))
    return sd


def _device_rtn(w: Any, group: int) -> "tuple[Any, Any]":
    from lemoq.quant import rtn  # noqa: PLC0415

    q = rtn.quantize_rtn(w, bits=8, group_size=group)
    return q["codes_padded"], q["scale_f16"]


def _get(sd: Mapping[str, Any], name: str) -> Any:
    for key in (name, "model." + name):
        if key in sd:
            return sd[key]
    raise KeyError("checkpoint has no tensor %r" % name)


def quantize_state_dict(sd: Mapping[str, Any], shape: OlmoeShape, *, device: Any = "cuda",
                        quantizer: Quantizer | None = None, tie_word_embeddings: bool = False) -> OlmoeW8Weights:
    """Pack and RTN-w8-quantize an HF OLMoE state dict for the decode step."""
    s = shape
    dev = torch.device(device)
    q8 = quantizer if quantizer is not None else _device_rtn
    g = s.group_size
    HD = s.heads * s.head_dim

    def f32(t: Any) -> Any:
        return t.to(device=dev, dtype=torch.float32).contiguous()

    def f16(t: Any) -> Any:
        return t.to(device=dev, dtype=torch.float16).contiguous()

    def check(t: Any, want: tuple, what: str) -> Any:
        if tuple(t.shape) != want:
            raise ValueError("%s has shape %s, expected %s" % (what, tuple(t.shape), want))
        return t

    def quant(w: Any, rows: int, cols: int, what: str) -> "tuple[Any, Any]":
        check(w, (rows, cols), what)
        c, sc = q8(f32(w), g)
        return c.to(dev), sc.to(dev)

    layers = []
    for i in range(s.layers):
        p = "layers.%d." % i
        qkv = torch.cat([_get(sd, p + "self_attn.%s_proj.weight" % n) for n in ("q", "k", "v")], 0)
        qkv_c, qkv_s = quant(qkv, 3 * HD, s.hidden, p + "qkv")
        o_c, o_s = quant(_get(sd, p + "self_attn.o_proj.weight"), s.hidden, HD, p + "o_proj")
        try:
            gu = _get(sd, p + "mlp.experts.gate_up_proj")
            dn = _get(sd, p + "mlp.experts.down_proj")
        except KeyError:
            e_w = lambda e, n: _get(sd, p + "mlp.experts.%d.%s_proj.weight" % (e, n))  # noqa: E731
            gu = torch.stack([torch.cat([e_w(e, "gate"), e_w(e, "up")], 0) for e in range(s.num_experts)])
            dn = torch.stack([e_w(e, "down") for e in range(s.num_experts)])
        check(gu, (s.num_experts, 2 * s.ffn, s.hidden), p + "experts.gate_up")
        check(dn, (s.num_experts, s.hidden, s.ffn), p + "experts.down")
        gu_c, gu_s = quant(gu.reshape(s.num_experts * 2 * s.ffn, s.hidden), s.num_experts * 2 * s.ffn, s.hidden,
                           p + "experts.gate_up")
        dn_c, dn_s = quant(dn.reshape(s.num_experts * s.hidden, s.ffn), s.num_experts * s.hidden, s.ffn,
                           p + "experts.down")
        layers.append(LayerW8(
            ln_in=f16(check(_get(sd, p + "input_layernorm.weight"), (s.hidden,), "input_layernorm")),
            ln_post=f16(check(_get(sd, p + "post_attention_layernorm.weight"), (s.hidden,), "post_attention_layernorm")),
            q_norm=f16(check(_get(sd, p + "self_attn.q_norm.weight"), (HD,), "q_norm")),
            k_norm=f16(check(_get(sd, p + "self_attn.k_norm.weight"), (HD,), "k_norm")),
            qkv_codes=qkv_c, qkv_scale=qkv_s, o_codes=o_c, o_scale=o_s,
            router=f16(check(_get(sd, p + "mlp.gate.weight"), (s.num_experts, s.hidden), "router")),
            gu_codes=gu_c.reshape(s.num_experts, 2 * s.ffn, s.hidden),
            gu_scale=gu_s.reshape(s.num_experts, 2 * s.ffn, s.hidden // g),
            dn_codes=dn_c.reshape(s.num_experts, s.hidden, s.ffn),
            dn_scale=dn_s.reshape(s.num_experts, s.hidden, s.ffn // g),
        ))
    embed = check(_get(sd, "embed_tokens.weight"), (s.vocab, s.hidden), "embed_tokens")
    if tie_word_embeddings:
        lm = embed
    elif "lm_head.weight" in sd:
        lm = check(sd["lm_head.weight"], (s.vocab, s.hidden), "lm_head")
    else:
        # an untied checkpoint without its lm_head would silently decode with the
        # embedding as the output projection: refuse it instead
        raise KeyError("lm_head.weight is missing and tie_word_embeddings is False")
    lm_c, lm_s = quant(lm, s.vocab, s.hidden, "lm_head")
    return OlmoeW8Weights(shape=s, embed=f16(embed), final_norm=f16(check(_get(sd, "norm.weight"), (s.hidden,), "norm")),
                          lm_codes=lm_c, lm_scale=lm_s, layers=layers)


def load_hf_olmoe(path: str, device: Any = "cuda", *, group_size: int = 128,
                  quantizer: Quantizer | None = None) -> OlmoeW8Weights:
    """A local HF OLMoE checkpoint directory (``config.json`` + safetensors) ->
    packed W8 weights for ``DecodeSession``."""
    with open(os.path.join(path, "config.json")) as f:
        cfg = json.load(f)
    shape = shape_from_hf_config(cfg, group_size=group_size)
    return quantize_state_dict(read_hf_state(path), shape, device=device, quantizer=quantizer,
                               tie_word_embeddings=bool(cfg.get("tie_word_embeddings", False)))


def save_packed(w: OlmoeW8Weights, path: str) -> None:
    """Write the packed weights (safetensors) and their shape, code width and
    lm_head kind (JSON) to ``path``."""
    from safetensors.torch import save_file  # noqa: PLC0415

    os.makedirs(path, exist_ok=True)
    tensors = {"embed": w.embed, "final_norm": w.final_norm}
    if w.lm_f16 is not None:
        tensors["lm_f16"] = w.lm_f16
    else:
        tensors.update(lm_codes=w.lm_codes, lm_scale=w.lm_scale)
    for i, L in enumerate(w.layers):
        for f in fields(LayerW8):
            tensors["layers.%d.%s" % (i, f.name)] = getattr(L, f.name)
    save_file({k: v.detach().to("cpu").contiguous() for k, v in tensors.items()}, os.path.join(path, PACKED_TENSORS))
    with open(os.path.join(path, PACKED_META), "w") as f:
        json.dump({"format": _FORMAT, "shape": asdict(w.shape), "bits": int(w.bits),
                   "lm_head": "fp16" if w.lm_f16 is not None else "w8"}, f, indent=1, sort_keys=True)


def load_packed(path: str, device: Any = "cuda") -> OlmoeW8Weights:
    """Read weights written by ``save_packed`` (bit for bit) onto ``device``."""
    from safetensors.torch import load_file  # noqa: PLC0415

    with open(os.path.join(path, PACKED_META)) as f:
        meta = json.load(f)
    if meta.get("format") != _FORMAT:
        raise ValueError("unknown packed format %r" % meta.get("format"))
    shape = OlmoeShape(**meta["shape"])
    t = load_file(os.path.join(path, PACKED_TENSORS), device="cpu")
    dev = torch.device(device)
    on = lambda x: x.to(dev).contiguous()  # noqa: E731
    layers = [LayerW8(**{f.name: on(t["layers.%d.%s" % (i, f.name)]) for f in fields(LayerW8)})
              for i in range(shape.layers)]
    bits, lm_head = int(meta.get("bits", 8)), meta.get("lm_head", "w8")  # files without them: the w8a16 cell
    if bits not in (4, 8) or lm_head not in ("w8", "fp16"):
        raise ValueError("unknown packed weights: bits %r, lm_head %r" % (bits, lm_head))
    if lm_head == "fp16":
        return OlmoeW8Weights(shape=shape, embed=on(t["embed"]), final_norm=on(t["final_norm"]), lm_codes=None,
                              lm_scale=None, layers=layers, bits=bits, lm_f16=on(t["lm_f16"]))
    return OlmoeW8Weights(shape=shape, embed=on(t["embed"]), final_norm=on(t["final_norm"]), lm_codes=on(t["lm_codes"]),
                          lm_scale=on(t["lm_scale"]), layers=layers, bits=bits)
