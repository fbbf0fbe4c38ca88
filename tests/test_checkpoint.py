"""OLMoE checkpoint loading (lemoq.model.checkpoint) on the CPU.

A tiny HF ``OlmoeForCausalLM`` is written with ``save_pretrained`` (safetensors,
the per-expert hub layout), loaded by ``load_hf_olmoe`` with the oracle's RTN
as the quantizer (the device RTN kernel is bit-exact to it; the GPU test of
the same load lives in test_gpu_checkpoint.py), and decoded by the CPU oracle.
Against the HF model in fp64 on the unquantized weights, RTN-w8 costs median
KL ~1e-4 and median relative logit error ~0.015 (measured over three seeds).
The gate is median KL < 1e-3 and median relative error < 0.05 over 12
teacher-forced positions.  Each planted mapping mistake in the loader's output
(q/k rows swapped, gate/up swapped, experts permuted, layers swapped) fails
it.  The packed format round-trips bit for bit, and the fused (transformers 5
``gate_up_proj``) and per-expert layouts pack identically.
"""

from __future__ import annotations

import json
import os
from dataclasses import fields

import pytest
import torch

from lemoq.model import checkpoint as ck
from lemoq.model.olmoe import LayerW8
from oracle import quant as oq
from oracle.olmoe import OracleDecoder

transformers = pytest.importorskip("transformers")

N_POS = 12
MED_KL = 1e-3
MED_REL = 0.05


def _rtn(w, g):
    q = oq.rtn_quantize_w8(w.detach().cpu().numpy(), g)
    return torch.from_numpy(q["codes_padded"]), torch.from_numpy(q["scale_f16"])


def _hf_model(seed, *, tie=False):
    from transformers import OlmoeConfig, OlmoeForCausalLM
    from transformers.utils import logging as hf_logging

    hf_logging.set_verbosity_error()
    torch.manual_seed(seed)
    cfg = OlmoeConfig(vocab_size=512, hidden_size=256, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=2, num_key_value_heads=2, num_experts=8, num_experts_per_tok=2,
                      norm_topk_prob=False, rms_norm_eps=1e-5, rope_theta=10000.0, max_position_embeddings=64,
                      tie_word_embeddings=tie, eos_token_id=None, pad_token_id=None, bos_token_id=None,
                      initializer_range=0.05, experts_implementation="eager", attn_implementation="eager")
    m = OlmoeForCausalLM(cfg).eval()
    with torch.no_grad():
        for n, p in m.named_parameters():
            if "norm" in n:
                p.copy_(torch.rand_like(p) + 0.5)
    return m


@pytest.fixture(scope="module")
def saved(tmp_path_factory):
    m = _hf_model(1)
    d = str(tmp_path_factory.mktemp("olmoe_ckpt"))
    m.save_pretrained(d, safe_serialization=True)
    toks = torch.randint(0, 512, (N_POS,), generator=torch.Generator().manual_seed(51))
    with torch.no_grad():
        ref = m.double()(toks[None]).logits[0]
    return d, toks, ref


def _stats(ref, w, toks):
    o = OracleDecoder(w, max_seq=N_POS + 4)
    out = torch.stack([o.step(int(t), p).double() for p, t in enumerate(toks)])
    p, q = torch.log_softmax(ref, -1), torch.log_softmax(out, -1)
    kl = (p.exp() * (p - q)).sum(-1)
    rel = (out - ref).abs().max(-1).values / ref.abs().max()
    return float(kl.median()), float(rel.median())


def test_shape_from_config(saved):
    d, _, _ = saved
    with open(os.path.join(d, "config.json")) as f:
        cfg = json.load(f)
    s = ck.shape_from_hf_config(cfg)
    assert (s.hidden, s.heads, s.head_dim, s.layers, s.num_experts, s.top_k, s.ffn, s.vocab) == (
        256, 2, 128, 2, 8, 2, 128, 512)
    assert s.rope_theta == 10000.0 and s.eps == 1e-5 and s.norm_topk_prob is False
    with pytest.raises(NotImplementedError):
        ck.shape_from_hf_config({**cfg, "num_key_value_heads": 1})
    assert ck.shape_from_hf_config({**cfg, "clip_qkv": 8.0}).clip_qkv == 8.0
    assert ck.shape_from_hf_config({**cfg, "clip_qkv": None}).clip_qkv is None


def test_loaded_checkpoint_decodes_like_hf(saved):
    d, toks, ref = saved
    w = ck.load_hf_olmoe(d, device="cpu", quantizer=_rtn)
    kl, rel = _stats(ref, w, toks)
    assert kl < MED_KL and rel < MED_REL, (kl, rel)


def _swap_qk(w):
    L = w.layers[0]
    hd = w.shape.heads * w.shape.head_dim
    for name in ("qkv_codes", "qkv_scale"):
        t = getattr(L, name).clone()
        t[:hd], t[hd:2 * hd] = getattr(L, name)[hd:2 * hd].clone(), getattr(L, name)[:hd].clone()
        setattr(L, name, t)


def _swap_gate_up(w):
    F = w.shape.ffn
    for L in w.layers:
        for name in ("gu_codes", "gu_scale"):
            t = getattr(L, name)
            setattr(L, name, torch.cat([t[:, F:], t[:, :F]], 1))


def _permute_experts(w):
    perm = torch.roll(torch.arange(w.shape.num_experts), 1)
    for L in w.layers:
        for name in ("gu_codes", "gu_scale", "dn_codes", "dn_scale"):
            setattr(L, name, getattr(L, name)[perm])


def _swap_layers(w):
    w.layers = [w.layers[1], w.layers[0]]


@pytest.mark.parametrize("plant", [_swap_qk, _swap_gate_up, _permute_experts, _swap_layers],
                         ids=["qk_swapped", "gate_up_swapped", "experts_permuted", "layers_swapped"])
def test_planted_loader_mistake_fails_the_gate(saved, plant):
    d, toks, ref = saved
    w = ck.load_hf_olmoe(d, device="cpu", quantizer=_rtn)
    plant(w)
    kl, rel = _stats(ref, w, toks)
    assert not (kl < MED_KL and rel < MED_REL), (plant.__name__, kl, rel)


def _equal(a, b):
    tensors = [("embed", a.embed, b.embed), ("final_norm", a.final_norm, b.final_norm),
               ("lm_codes", a.lm_codes, b.lm_codes), ("lm_scale", a.lm_scale, b.lm_scale)]
    for i, (la, lb) in enumerate(zip(a.layers, b.layers)):
        tensors += [("%d.%s" % (i, f.name), getattr(la, f.name), getattr(lb, f.name)) for f in fields(LayerW8)]
    for name, x, y in tensors:
        assert x.dtype == y.dtype and x.shape == y.shape, name
        assert torch.equal(x.view(torch.uint8) if x.dtype != torch.uint8 else x,
                           y.view(torch.uint8) if y.dtype != torch.uint8 else y), name


def test_packed_round_trip_is_bitwise(saved, tmp_path):
    d, _, _ = saved
    w = ck.load_hf_olmoe(d, device="cpu", quantizer=_rtn)
    ck.save_packed(w, str(tmp_path))
    w2 = ck.load_packed(str(tmp_path), device="cpu")
    assert w2.shape == w.shape
    _equal(w, w2)
    with open(os.path.join(str(tmp_path), ck.PACKED_META)) as f:
        meta = json.load(f)
    meta["format"] = "something-else"
    with open(os.path.join(str(tmp_path), ck.PACKED_META), "w") as f:
        json.dump(meta, f)
    with pytest.raises(ValueError):
        ck.load_packed(str(tmp_path), device="cpu")


def test_fused_and_per_expert_layouts_pack_identically(saved):
    d, _, _ = saved
    sd = ck.read_hf_state(d)
    with open(os.path.join(d, "config.json")) as f:
        shape = ck.shape_from_hf_config(json.load(f))
    a = ck.quantize_state_dict(sd, shape, device="cpu", quantizer=_rtn)
    fused = {k: v for k, v in sd.items() if ".mlp.experts." not in k}
    for i in range(shape.layers):
        p = "model.layers.%d.mlp.experts." % i
        fused[p + "gate_up_proj"] = torch.stack([torch.cat([sd[p + "%d.gate_proj.weight" % e],
                                                            sd[p + "%d.up_proj.weight" % e]], 0)
                                                 for e in range(shape.num_experts)])
        fused[p + "down_proj"] = torch.stack([sd[p + "%d.down_proj.weight" % e] for e in range(shape.num_experts)])
    b = ck.quantize_state_dict(fused, shape, device="cpu", quantizer=_rtn)
    _equal(a, b)


def test_tied_embeddings_and_shape_errors(tmp_path):
    m = _hf_model(2, tie=True)
    m.save_pretrained(str(tmp_path), safe_serialization=True)
    w = ck.load_hf_olmoe(str(tmp_path), device="cpu", quantizer=_rtn)
    c, s = _rtn(m.model.embed_tokens.weight.float(), 128)
    assert torch.equal(w.lm_codes, c) and torch.equal(w.lm_scale.view(torch.int16), s.view(torch.int16))
    sd = ck.read_hf_state(str(tmp_path))
    with open(os.path.join(str(tmp_path), "config.json")) as f:
        shape = ck.shape_from_hf_config(json.load(f))
    bad = dict(sd)
    bad["model.layers.0.mlp.gate.weight"] = bad["model.layers.0.mlp.gate.weight"][:, :128]
    with pytest.raises(ValueError):
        ck.quantize_state_dict(bad, shape, device="cpu", quantizer=_rtn)
    missing = {k: v for k, v in sd.items() if "layers.1.self_attn.o_proj" not in k}
    with pytest.raises(KeyError):
        ck.quantize_state_dict(missing, shape, device="cpu", quantizer=_rtn)


def test_untied_checkpoint_without_lm_head_is_refused(saved):
    """An untied checkpoint whose lm_head is missing must not fall back to the embedding."""
    d, _, _ = saved
    sd = ck.read_hf_state(d)
    with open(os.path.join(d, "config.json")) as f:
        shape = ck.shape_from_hf_config(json.load(f))
    assert "lm_head.weight" in sd
    no_lm = {k: v for k, v in sd.items() if k != "lm_head.weight"}
    with pytest.raises(KeyError):
        ck.quantize_state_dict(no_lm, shape, device="cpu", quantizer=_rtn, tie_word_embeddings=False)
    tied = ck.quantize_state_dict(no_lm, shape, device="cpu", quantizer=_rtn, tie_word_embeddings=True)
    c, _ = _rtn(sd["model.embed_tokens.weight"].float(), 128)
    assert torch.equal(tied.lm_codes, c)


def test_packed_round_trip_of_4bit_weights_with_fp16_lm_head(tmp_path):
    """The w4a16 cell's weights (4-bit attention and experts packed two per byte,
    fp16 lm_head) keep their code width and lm_head kind through save/load, bit
    for bit; a file without the two keys reads as the w8a16 cell."""
    from dataclasses import asdict

    from lemoq.model.olmoe import OlmoeShape, OlmoeW8Weights
    from oracle.olmoe import Shape, random_host_weights

    small = Shape(hidden=256, heads=2, head_dim=128, layers=2, num_experts=4, top_k=2, ffn=128, vocab=64)
    hw = random_host_weights(small, seed=3, bits=4, lm_head="fp16")
    w = OlmoeW8Weights(shape=OlmoeShape(**asdict(small)), embed=hw.embed, final_norm=hw.final_norm, lm_codes=None,
                       lm_scale=None, layers=[LayerW8(**{f.name: getattr(L, f.name) for f in fields(LayerW8)})
                                              for L in hw.layers], bits=4, lm_f16=hw.lm_f16)
    ck.save_packed(w, str(tmp_path))
    w2 = ck.load_packed(str(tmp_path), device="cpu")
    assert (w2.bits, w2.lm_codes, w2.lm_scale) == (4, None, None)
    assert torch.equal(w2.lm_f16, w.lm_f16) and w2.layers[0].gu_codes.shape == (4, 256, 128)
    for i, (la, lb) in enumerate(zip(w.layers, w2.layers)):
        for f in fields(LayerW8):
            assert torch.equal(getattr(la, f.name), getattr(lb, f.name)), (i, f.name)
    with open(os.path.join(str(tmp_path), ck.PACKED_META)) as f:
        meta = json.load(f)
    assert (meta["bits"], meta["lm_head"]) == (4, "fp16")
    meta["bits"] = 3
    with open(os.path.join(str(tmp_path), ck.PACKED_META), "w") as f:
        json.dump(meta, f)
    with pytest.raises(ValueError):
        ck.load_packed(str(tmp_path), device="cpu")
