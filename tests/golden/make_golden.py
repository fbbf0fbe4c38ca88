"""Writes tests/golden/*.npz: small seeded input/output vectors of the decode path.

The reference ships no golden vectors (its results/ directory is empty), so
these are produced by this repository's CPU oracle (oracle/), whose functions
are pinned independently (tests/test_oracle_*.py).  The fixtures freeze those
outputs so a later change to the oracle or to the HIP kernels that alters a
bit-exact result (RTN codes/scales, KV-INT8 bytes, routing ids) or the tiny
model's decode fails loudly.  Run from the repo root:

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from oracle import ops  # noqa: E402
from oracle import quant as oq  # noqa: E402
from oracle.olmoe import OracleDecoder, Shape, oracle_prefill, random_host_weights  # noqa: E402

TINY = Shape(hidden=256, heads=2, head_dim=128, layers=2, num_experts=4, top_k=2, ffn=128, vocab=512)
TINY_SEED = 20261201
TINY_PROMPT = [1, 7, 300, 42, 5, 5, 99, 1]
TINY_STEPS = 8
PREFILL_PROMPT_LEN = 24
PREFILL_STEPS = 6


def rtn_fixture() -> dict:
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((8, 256)) * 0.02).astype(np.float32)
    w[0, :16] = [127, -63.5, 0.5, 1.5, 2.5, -0.5, -1.5, 3.49, 3.5, -127, 100.5, 0, 64.5, -64.5, 126.5, -126.5]
    w[1, :128] = 0.0  # an all-zero group
    w2 = (rng.standard_normal((3, 130)) * 0.02).astype(np.float32)  # padded to 256
    q = oq.rtn_quantize_w8(w, 128)
    q2 = oq.rtn_quantize_w8(w2, 128)
    return {"w": w, "codes": q["codes_padded"], "scale32": q["scale"], "scale16": q["scale_f16"],
            "w_pad": w2, "codes_pad": q2["codes_padded"], "scale16_pad": q2["scale_f16"]}


def kv_fixture() -> dict:
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((16, 128)) * 2).astype(np.float16)
    x[3] = 0
    x[5, :8] = [2.0, 1.0, 0.5, -1.0, -2.0, 0.25, 0.0078125, -0.0078125]
    x[5, 8:] = 0
    codes, scales = oq.kv_quantize_rows(x)
    return {"x": x, "codes": codes, "scales": scales}


def route_fixture() -> dict:
    rng = np.random.default_rng(3)
    z = (rng.standard_normal((64, 64)) * 1.5).astype(np.float16)
    z[0, :] = 0  # all tied
    z[1, :10] = 3  # tie across the k-th boundary
    out = {"logits": z}
    for norm in (False, True):
        w, i = oq.route_order(z.astype(np.float32), 8, norm)
        out["ids_norm%d" % norm] = i
        out["w_norm%d" % norm] = w
    return out


def tiny_decode_fixture() -> dict:
    hw = random_host_weights(TINY, seed=TINY_SEED)
    od = OracleDecoder(hw, len(TINY_PROMPT) + TINY_STEPS)
    tokens, logits = od.run(TINY_PROMPT, TINY_STEPS)
    return {"prompt": np.array(TINY_PROMPT, dtype=np.int64), "tokens": np.array(tokens, dtype=np.int64),
            "logits": torch.stack(logits).numpy(), "seed": np.array(TINY_SEED, dtype=np.int64)}


def tiny_prefill_fixture() -> dict:
    """The batched prefill of a 24-token prompt (``oracle_prefill``: last-position logits and every
    layer's KV-INT8 rows), then greedy decode steps from that cache."""
    hw = random_host_weights(TINY, seed=TINY_SEED)
    prompt = np.random.default_rng(4).integers(0, TINY.vocab, PREFILL_PROMPT_LEN).astype(np.int64)
    S = PREFILL_PROMPT_LEN + PREFILL_STEPS
    logits, kv = oracle_prefill(hw, prompt, S)
    od = OracleDecoder(hw, S, kv=kv)
    seed = od.greedy(logits)
    tokens, step_logits = od.run([], PREFILL_STEPS, start_pos=PREFILL_PROMPT_LEN, seed_token=seed)
    T = PREFILL_PROMPT_LEN
    return {"prompt": prompt, "logits": logits.numpy(), "seed": np.array(TINY_SEED, dtype=np.int64),
            "kc": np.stack([c["kc"][:, :T].numpy() for c in kv]), "ks": np.stack([c["ks"][:, :T].numpy() for c in kv]),
            "vc": np.stack([c["vc"][:, :T].numpy() for c in kv]), "vs": np.stack([c["vs"][:, :T].numpy() for c in kv]),
            "tokens": np.array(tokens, dtype=np.int64), "step_logits": torch.stack(step_logits).numpy()}


def main() -> None:
    fixtures = {"rtn_w8": rtn_fixture(), "kv_int8": kv_fixture(), "routing": route_fixture(),
                "tiny_decode": tiny_decode_fixture(), "tiny_prefill": tiny_prefill_fixture()}
    for name, arrays in fixtures.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **arrays)
        print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
