"""GPU side of checkpoint loading: a tiny HF OLMoE checkpoint quantized by the
device RTN kernel (``load_hf_olmoe(..., device="cuda")``) gives bit-exactly
the codes and scales of the CPU oracle's RTN, decodes greedily in a captured
graph in step with the CPU oracle (per-step KL < 0.01, identical tokens
except at near-ties), also with HF OLMoE's clip_qkv set in the config, and
reloaded from the packed format decodes bitwise identically."""

from __future__ import annotations

import os
from dataclasses import fields

import pytest
import torch

from lemoq.model import checkpoint as ck
from lemoq.model.olmoe import DecodeSession, LayerW8
from oracle import quant as oq
from oracle.olmoe import OracleDecoder

pytestmark = pytest.mark.gpu
transformers = pytest.importorskip("transformers")


def _rtn(w, g):
    q = oq.rtn_quantize_w8(w.detach().cpu().numpy(), g)
    return torch.from_numpy(q["codes_padded"]), torch.from_numpy(q["scale_f16"])


def _write_ckpt(tmp_path_factory, clip_qkv=None):
    from transformers import OlmoeConfig, OlmoeForCausalLM
    from transformers.utils import logging as hf_logging

    hf_logging.set_verbosity_error()
    torch.manual_seed(4)
    cfg = OlmoeConfig(vocab_size=512, hidden_size=256, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=2, num_key_value_heads=2, num_experts=8, num_experts_per_tok=2,
                      norm_topk_prob=False, rms_norm_eps=1e-5, rope_theta=10000.0, max_position_embeddings=64,
                      tie_word_embeddings=False, eos_token_id=None, pad_token_id=None, bos_token_id=None,
                      initializer_range=0.05, clip_qkv=clip_qkv)
    m = OlmoeForCausalLM(cfg)
    with torch.no_grad():
        for n, p in m.named_parameters():
            if "norm" in n:
                p.copy_(torch.rand_like(p) + 0.5)
    d = str(tmp_path_factory.mktemp("olmoe_gpu_ckpt"))
    m.save_pretrained(d, safe_serialization=True)
    return d


@pytest.fixture(scope="module")
def ckpt_dir(tmp_path_factory):
    return _write_ckpt(tmp_path_factory)


@pytest.fixture(scope="module")
def ckpt_dir_clip(tmp_path_factory):
    """The same model with HF OLMoE's clip_qkv set (0.4 clamps a good share of q/k/v)."""
    return _write_ckpt(tmp_path_factory, clip_qkv=0.4)


def test_device_rtn_load_is_bit_exact_to_the_oracle(ckpt_dir, dev):
    print("case: device RTN load vs oracle RTN", flush=True)
    wg = ck.load_hf_olmoe(ckpt_dir, device=dev)
    wc = ck.load_hf_olmoe(ckpt_dir, device="cpu", quantizer=_rtn)
    pairs = [("lm_codes", wg.lm_codes, wc.lm_codes), ("lm_scale", wg.lm_scale, wc.lm_scale),
             ("embed", wg.embed, wc.embed)]
    for i, (a, b) in enumerate(zip(wg.layers, wc.layers)):
        pairs += [("%d.%s" % (i, f.name), getattr(a, f.name), getattr(b, f.name)) for f in fields(LayerW8)]
    for name, a, b in pairs:
        a = a.cpu()
        assert a.dtype == b.dtype and a.shape == b.shape, name
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), name


@pytest.mark.parametrize("clip", [False, True], ids=["plain", "clip_qkv"])
def test_loaded_checkpoint_decodes_with_the_oracle(clip, ckpt_dir, ckpt_dir_clip, dev, tmp_path):
    print("case: loaded checkpoint decode (clip_qkv %s)" % clip, flush=True)
    w = ck.load_hf_olmoe(ckpt_dir_clip if clip else ckpt_dir, device=dev)
    assert w.shape.clip_qkv == (0.4 if clip else None)
    prompt, steps = [5, 77, 300, 12], 12
    sess = DecodeSession(w, prompt, max_new_tokens=steps, num_splits=None)
    sess.prefill()
    kv = sess.kv_cpu()
    logits = []
    for _ in range(steps):
        sess.replay(1)
        logits.append(sess.logits_cpu())
    toks = [int(t) for t in sess.history[len(prompt) - 1: len(prompt) + steps].tolist()]
    oracle = OracleDecoder(w.to_host(), sess.max_seq, kv=kv)
    flips = 0
    for i in range(steps):
        ref = oracle.step(toks[i + 1], len(prompt) + i).double()
        got = logits[i].double()
        p, q = torch.log_softmax(ref, -1), torch.log_softmax(got, -1)
        kl = float((p.exp() * (p - q)).sum())
        diff = float((ref - got).abs().max())
        assert kl < 1e-2 and diff <= 2e-2 * float(ref.abs().max()), (i, kl, diff)
        if int(torch.argmax(ref)) != int(torch.argmax(got)):
            top = torch.topk(ref, 2).values
            assert float(top[0] - top[1]) <= 2 * diff, i
            flips += 1
    assert flips <= 1

    # packed format: saved, reloaded onto the device, the same graph step bit for bit
    ck.save_packed(w, str(tmp_path))
    w2 = ck.load_packed(str(tmp_path), device=dev)
    assert w2.shape == w.shape  # clip_qkv travels with the shape
    s2 = DecodeSession(w2, prompt, max_new_tokens=steps, num_splits=None)
    s2.prefill()
    s2.replay(steps)
    assert s2.generated() == sess.generated()
    assert torch.equal(s2.logits_cpu(), logits[-1])
    assert os.path.exists(os.path.join(str(tmp_path), ck.PACKED_META))
