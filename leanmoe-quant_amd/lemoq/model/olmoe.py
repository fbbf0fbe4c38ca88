"""OLMoE decode-step module on the HIP kernels: weights, KV cache, session.

This replaces the reference's HF-patched model + ``StaticCacheDecodeSession``
(``benchmarks/cudagraph.py:511-820``) for the canonical cell
``--moe grouped --dequant fused --attn kernel --execution cudagraph
--bit-width w8a16`` with W8 lm_head and KV-INT8 (``runner.py:2447-2521``,
``fusion_switches.py:49-57``):

* ``OlmoeShape`` — the model shape (OLMoE-1B-7B by default: H 2048, 16 layers,
  16 heads x 128, 64 experts top-8, F 1024, vocab 50304).
* ``OlmoeW8Weights.random(shape, seed)`` — seeded random init generated and
  RTN-w8-quantized on the device (attention q|k|v packed row-wise, o_proj,
  experts, lm_head); router, embedding and norm weights stay fp16.
  ``random(..., bits=4, lm_head="fp16")`` gives the reference's w4a16 cell
  (``--bit-width w4a16``, ``benchmarks/runner.py:451-482``): attention and
  experts as 4-bit symmetric codes packed two per byte, the lm_head in fp16
  (``runner.py:393-412``).
* ``DecodeSession`` — fixed-address KV cache (KV-INT8, or fp16 rows with
  ``kv_cache="fp16"``: the same cell with KV-INT8 off, ``attn_decode.py:930-948,
  999-1008``) and step buffers, the step
  enqueued by one native call (``lemoq_olmoe_decode_step``), captured once
  into a hipGraph (``torch.cuda.CUDAGraph``) and replayed.  Greedy selection
  and the position advance run on the device, so consecutive replays need no
  host round trip.  ``prefill()`` runs the prompt as one batch on the matrix
  cores (``lemoq.model.prefill``), as the reference's session does; the
  prompt can also be fed through the step itself (one replay per position).

Layout in HBM (per layer): ``qkv_codes`` (3*heads*D, H) int8 with fp16 scales
(3*heads*D, H/g); ``o_codes`` (H, heads*D); ``gu_codes`` (E, 2F, H) and
``dn_codes`` (E, H, F) int8 with per-group fp16 scales; ``kc``/``vc`` (heads, S, D)
int8 and ``ks``/``vs`` (heads, S) fp16 for S = max_seq cache slots (the fp16
cache: ``k``/``v`` (heads, S, D) fp16).
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field, fields
from typing import Any

import torch

from lemoq import _hip

__all__ = ["OlmoeShape", "OLMOE_1B_7B", "OlmoeW8Weights", "LayerW8", "DecodeSession", "KV_CACHE_KINDS"]

LOG2E = 1.4426950408889634
# The decode cache kinds: "int8" (KV-INT8 codes + fp16 per-token scales, the
# canonical cell) and "fp16" (the rows as they are: the cell with KV-INT8 off).
KV_CACHE_KINDS = ("int8", "fp16")
# Split-KV blocks per head of the step's attention: one block per 64 cache
# slots, at least 2, and at most one wave of blocks over the chip
# (heads * splits <= compute units; 16 splits per head for OLMoE's 16 heads on
# a 256-CU MI355X).  A grid larger than one block per CU runs a second round
# of blocks, which costs more than the longer splits save; the LSE merge grows
# with the split count (2.5 us at 8 splits, 2.9 at 16, 3.6 at 32).
STEP_SLOTS_PER_SPLIT = 64
STEP_MAX_SPLITS = 64


def step_num_splits(max_seq: int, heads: int, compute_units: int = 256) -> int:
    ns = -(-int(max_seq) // STEP_SLOTS_PER_SPLIT)
    cap = max(1, min(STEP_MAX_SPLITS, int(compute_units) // max(1, int(heads))))
    return max(1, min(max(2, ns), cap))


@dataclass(frozen=True)
class OlmoeShape:
    hidden: int = 2048
    heads: int = 16
    head_dim: int = 128
    layers: int = 16
    num_experts: int = 64
    top_k: int = 8
    ffn: int = 1024
    vocab: int = 50304
    eps: float = 1e-5
    rope_theta: float = 10000.0
    norm_topk_prob: bool = False
    group_size: int = 128
    init_std: float = 0.02
    # HF OLMoE's clip_qkv: the normed q, the normed k and v are clamped to
    # +-clip_qkv before RoPE (None: no clamp)
    clip_qkv: float | None = None

    @property
    def qkv_rows(self) -> int:
        return 3 * self.heads * self.head_dim

    def weight_bytes_per_token(self) -> int:
        """Bytes of weights one decode step streams (w8 codes + fp16 scales, fp16 rest)."""
        H, HD, F, g = self.hidden, self.heads * self.head_dim, self.ffn, self.group_size
        w8 = lambda rows, cols: rows * cols + rows * (cols // g) * 2  # noqa: E731
        per_layer = (
            w8(3 * HD, H)
            + w8(H, HD)
            + self.top_k * (w8(2 * F, H) + w8(H, F))
            + self.num_experts * H * 2  # fp16 router
            + 4 * H * 2  # ln_in, ln_post (H) and q_norm, k_norm (HD == H for OLMoE)
        )
        return self.layers * per_layer + w8(self.vocab, H) + H * 2 + H * 2


OLMOE_1B_7B = OlmoeShape()


@dataclass
class LayerW8:
    ln_in: Any
    ln_post: Any
    q_norm: Any
    k_norm: Any
    qkv_codes: Any
    qkv_scale: Any
    o_codes: Any
    o_scale: Any
    router: Any
    gu_codes: Any
    gu_scale: Any
    dn_codes: Any
    dn_scale: Any


@dataclass
class OlmoeW8Weights:
    """The decode step's weights.  ``bits`` is the code width of attention and
    experts: 8 (int8 codes, the canonical w8a16 cell) or 4 (4-bit symmetric
    codes packed two per byte, the even column in the low nibble: the w4a16
    cell).  ``lm_f16`` is an fp16 lm_head (vocab, H) in place of ``lm_codes`` /
    ``lm_scale`` (which are then None)."""

    shape: OlmoeShape
    embed: Any
    final_norm: Any
    lm_codes: Any
    lm_scale: Any
    layers: list[LayerW8] = field(default_factory=list)
    bits: int = 8
    lm_f16: Any = None

    @property
    def device(self) -> Any:
        return self.embed.device

    def to_host(self) -> "OlmoeW8Weights":
        """Copy every tensor to the CPU (the form the CPU oracle consumes)."""
        cpu = lambda t: None if t is None else t.detach().to("cpu")  # noqa: E731
        return OlmoeW8Weights(
            shape=self.shape,
            embed=cpu(self.embed),
            final_norm=cpu(self.final_norm),
            lm_codes=cpu(self.lm_codes),
            lm_scale=cpu(self.lm_scale),
            layers=[LayerW8(**{f.name: cpu(getattr(L, f.name)) for f in fields(LayerW8)}) for L in self.layers],
            bits=self.bits,
            lm_f16=cpu(self.lm_f16),
        )

    def int8_codes(self) -> "OlmoeW8Weights":
        """The same weights with attention and expert codes as int8 (the batched
        prefill's operand type): 8-bit weights as they are; 4-bit codes unpacked,
        an exact re-encoding (code * scale is the same value), so the prefill's
        fp16(code * scale) weights are the w4a16 cell's separate-arm weights.
        Scales, norms, router, embedding and lm_head are shared, not copied."""
        if self.bits == 8:
            return self
        from lemoq.quant.pack import unpack_4bit  # noqa: PLC0415

        def layer(L: LayerW8) -> LayerW8:
            codes = {n: unpack_4bit(getattr(L, n), signed=True).contiguous()
                     for n in ("qkv_codes", "o_codes", "gu_codes", "dn_codes")}
            return LayerW8(**{f.name: codes.get(f.name, getattr(L, f.name)) for f in fields(LayerW8)})

        return OlmoeW8Weights(shape=self.shape, embed=self.embed, final_norm=self.final_norm, lm_codes=self.lm_codes,
                              lm_scale=self.lm_scale, layers=[layer(L) for L in self.layers], bits=8,
                              lm_f16=self.lm_f16)

    def weight_bits(self) -> Any:
        """The byte model's storage of each weight family (``lemoq.bytes.WeightBits``)."""
        from lemoq.bytes import WeightBits  # noqa: PLC0415

        return WeightBits(attention=self.bits, experts=self.bits, lm_head=16 if self.lm_f16 is not None else 8,
                          group_size=self.shape.group_size)

    @classmethod
    def random(cls, shape: OlmoeShape = OLMOE_1B_7B, *, seed: int = 0, device: Any = "cuda", bits: int = 8,
               lm_head: str = "w8") -> "OlmoeW8Weights":
        """Seeded random init on the device, RTN-quantized by the HIP kernel.

        Linear, expert, router and embedding weights ~ N(0, init_std) (the HF
        ``_init_weights`` distribution); norm weights ~ U(0.5, 1.5) so that a
        mixed-up norm weight changes the answer.  Generation order is fixed:
        embedding, then per layer (ln_in, ln_post, q_norm, k_norm, q|k|v, o,
        router, gate_up, down), then final norm, lm_head.  ``bits`` 8 or 4
        (attention and experts; RTN symmetric, groups of ``group_size``);
        ``lm_head`` "w8" (RTN w8) or "fp16".
        """
        from lemoq.quant import rtn  # noqa: PLC0415

        if bits not in (4, 8):
            raise ValueError("bits must be 4 or 8, got %r" % (bits,))
        if lm_head not in ("w8", "fp16"):
            raise ValueError("lm_head must be 'w8' or 'fp16', got %r" % (lm_head,))
        if bits == 4 and shape.group_size % 32 != 0:
            raise ValueError("4-bit weights need group_size % 32 == 0, got %d" % shape.group_size)
        dev = torch.device(device)
        _hip.require_rocm(torch.empty(0, device=dev), what="OlmoeW8Weights.random")
        gen = torch.Generator(device=dev)
        gen.manual_seed(int(seed))
        s = shape
        g = s.group_size
        HD = s.heads * s.head_dim

        def normal(*size: int) -> Any:
            return torch.randn(size, generator=gen, device=dev, dtype=torch.float32) * s.init_std

        def gamma(n: int) -> Any:
            return (torch.rand((n,), generator=gen, device=dev, dtype=torch.float32) + 0.5).to(torch.float16)

        def q8_lm(w: Any) -> tuple[Any, Any]:
            q = rtn.quantize_rtn(w, bits=8, group_size=g)
            return q["codes_padded"], q["scale_f16"]

        def q8(w: Any) -> tuple[Any, Any]:  # attention and experts at `bits`
            if bits == 8:
                return q8_lm(w)
            q = rtn.quantize_rtn(w, bits=4, group_size=g)
            return q["packed"], q["scale_f16"]

        per = 8 // bits  # codes per byte

        embed = normal(s.vocab, s.hidden).to(torch.float16)
        layers = []
        for _ in range(s.layers):
            ln_in, ln_post, qn, kn = gamma(s.hidden), gamma(s.hidden), gamma(HD), gamma(HD)
            qkv_c, qkv_s = q8(normal(3 * HD, s.hidden))
            o_c, o_s = q8(normal(s.hidden, HD))
            router = normal(s.num_experts, s.hidden).to(torch.float16)
            gu = normal(s.num_experts * 2 * s.ffn, s.hidden)
            gu_c, gu_s = q8(gu)
            del gu
            dn = normal(s.num_experts * s.hidden, s.ffn)
            dn_c, dn_s = q8(dn)
            del dn
            layers.append(
                LayerW8(
                    ln_in=ln_in, ln_post=ln_post, q_norm=qn, k_norm=kn,
                    qkv_codes=qkv_c, qkv_scale=qkv_s, o_codes=o_c, o_scale=o_s, router=router,
                    gu_codes=gu_c.reshape(s.num_experts, 2 * s.ffn, s.hidden // per),
                    gu_scale=gu_s.reshape(s.num_experts, 2 * s.ffn, s.hidden // g),
                    dn_codes=dn_c.reshape(s.num_experts, s.hidden, s.ffn // per),
                    dn_scale=dn_s.reshape(s.num_experts, s.hidden, s.ffn // g),
                )
            )
        final_norm = gamma(s.hidden)
        lm = normal(s.vocab, s.hidden)
        if lm_head == "fp16":
            return cls(shape=s, embed=embed, final_norm=final_norm, lm_codes=None, lm_scale=None, layers=layers,
                       bits=bits, lm_f16=lm.to(torch.float16))
        lm_c, lm_s = q8_lm(lm)
        return cls(shape=s, embed=embed, final_norm=final_norm, lm_codes=lm_c, lm_scale=lm_s, layers=layers,
                   bits=bits)


class DecodeSession:
    """Static-shape decode session over a KV cache, captured as one hipGraph step.

    Mirrors ``StaticCacheDecodeSession`` (``benchmarks/cudagraph.py:511-820``):
    ``prefill()``, ``capture()``, ``replay()``, ``decode_eager()``,
    ``set_position()``, ``logits_cpu()``, ``reset()``.  ``prompt_ids`` is a 1-D
    sequence of token ids (the canonical prompt is ``ctx`` ones); the cache has
    ``ctx + max_new_tokens`` slots.  ``kv_cache``: ``"int8"`` (KV-INT8, the
    canonical cell) or ``"fp16"`` (KV-INT8 off: the attention reads the fp16
    rows the step writes, as the reference does without its int8 mirror);
    None follows the reference's ``kv_int8`` switch (``LEMOQ_KV_INT8``, on by
    default; ``lemoq.kernels.fusion_switches``).  The step follows the weights:
    4-bit attention and experts (``weights.bits == 4``, the w4a16 cell) and an
    fp16 lm_head (``weights.lm_f16``) run the step's 4-bit layer and fp16
    lm_head.
    """

    def __init__(
        self,
        weights: OlmoeW8Weights,
        prompt_ids: Any,
        *,
        max_new_tokens: int,
        num_splits: int | None = None,
        kv_cache: str | None = None,
    ) -> None:
        from lemoq.kernels.attn_decode import resolve_num_splits  # noqa: PLC0415
        from lemoq.kernels.rope import rotary_cos_sin  # noqa: PLC0415

        s = weights.shape
        dev = weights.device
        _hip.require_rocm(weights.embed, what="DecodeSession")
        prompt = torch.as_tensor(prompt_ids, dtype=torch.int64).reshape(-1)
        if prompt.numel() < 1:
            raise ValueError("prompt must hold at least one token")
        if int(prompt.min()) < 0 or int(prompt.max()) >= s.vocab:
            raise ValueError("prompt token ids must lie in [0, vocab)")
        if max_new_tokens < 1:
            raise ValueError("max_new_tokens must be >= 1")
        from lemoq.kernels.fusion_switches import require_built  # noqa: PLC0415

        switches = require_built()  # refuses a switch set to an arm this build does not have
        if kv_cache is None:  # the reference's kv_int8 switch (LEMOQ_KV_INT8, default on)
            kv_cache = "int8" if switches["kv_int8"] else "fp16"
        if kv_cache not in KV_CACHE_KINDS:
            raise ValueError("kv_cache must be one of %s, got %r" % (KV_CACHE_KINDS, kv_cache))
        self.kv_cache = kv_cache
        self.weights = weights
        self.shape = s
        self.device = dev
        self.ctx = int(prompt.numel())
        self.max_new_tokens = int(max_new_tokens)
        self.max_seq = self.ctx + self.max_new_tokens
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        self.num_splits = (step_num_splits(self.max_seq, s.heads, cus) if num_splits is None
                           else resolve_num_splits(num_splits, heads=s.heads, device=dev))
        S, D, HD = self.max_seq, s.head_dim, s.heads * s.head_dim

        i8 = dict(dtype=torch.int8, device=dev)
        f16 = dict(dtype=torch.float16, device=dev)
        self.kv = []
        for _ in range(s.layers):
            if kv_cache == "fp16":
                self.kv.append({"k": torch.zeros((s.heads, S, D), **f16),
                                "v": torch.zeros((s.heads, S, D), **f16)})
                continue
            self.kv.append(
                {
                    "kc": torch.zeros((s.heads, S, D), **i8),
                    "ks": torch.ones((s.heads, S), **f16),
                    "vc": torch.zeros((s.heads, S, D), **i8),
                    "vs": torch.ones((s.heads, S), **f16),
                }
            )
        cos, sin = rotary_cos_sin(torch.arange(S), D, s.rope_theta)
        self.cos_tab = cos.to(dev).contiguous()
        self.sin_tab = sin.to(dev).contiguous()
        self.prompt = prompt.to(dev)
        self.token = torch.zeros((1,), dtype=torch.int64, device=dev)
        self.pos = torch.zeros((1,), dtype=torch.int64, device=dev)
        self.filled = torch.zeros((1,), dtype=torch.int32, device=dev)
        self.history = torch.zeros((S + 1,), dtype=torch.int64, device=dev)
        self.h = torch.zeros((s.hidden,), **f16)
        self.xn = torch.zeros((s.hidden,), **f16)
        self.qkv = torch.zeros((3 * HD,), **f16)
        self.q_rot = torch.zeros((HD,), **f16)
        self.attn = torch.zeros((HD,), **f16)
        self.part_m = torch.zeros((s.heads * self.num_splits,), dtype=torch.float32, device=dev)
        self.part_l = torch.zeros_like(self.part_m)
        self.part_acc = torch.zeros((s.heads * self.num_splits * D,), dtype=torch.float32, device=dev)
        self.router_logits = torch.zeros((s.num_experts,), **f16)
        self.top_w = torch.zeros((s.top_k,), **f16)
        self.top_i = torch.zeros((s.top_k,), dtype=torch.int64, device=dev)
        self.act = torch.zeros((s.top_k, s.ffn), **f16)
        self.logits = torch.zeros((s.vocab,), **f16)
        n_parts = int(_hip.load().lemoq_lm_head_argmax_parts(s.vocab))
        self.am_val = torch.zeros((n_parts,), dtype=torch.float32, device=dev)
        self.am_idx = torch.zeros((n_parts,), dtype=torch.int32, device=dev)
        # o_proj partial sums per group of 4 heads and the residual after
        # attention (the step's fused merge + o_proj path; unused by shapes it
        # does not cover, which run merge, o_proj and router as three launches)
        self.o_part = torch.zeros((max(1, HD // 512), s.hidden), dtype=torch.float32, device=dev)
        self.h_mid = torch.zeros((s.hidden,), **f16)

        P = _hip.ptr
        self._layer_structs = (_hip.LemoqOlmoeLayer * s.layers)()
        for i, (L, kv) in enumerate(zip(weights.layers, self.kv)):
            ls = self._layer_structs[i]
            for name in (
                "ln_in", "ln_post", "q_norm", "k_norm", "qkv_codes", "qkv_scale", "o_codes",
                "o_scale", "router", "gu_codes", "gu_scale", "dn_codes", "dn_scale",
            ):
                t = getattr(L, name)
                if not t.is_contiguous() or t.device != dev:
                    raise ValueError("layer %d weight %s must be contiguous on %s" % (i, name, dev))
                setattr(ls, name, P(t))
            if kv_cache == "fp16":  # fp16 rows behind kc / vc, no scales
                ls.kc, ls.vc, ls.ks, ls.vs = P(kv["k"]), P(kv["v"]), None, None
            else:
                for name in ("kc", "ks", "vc", "vs"):
                    setattr(ls, name, P(kv[name]))
        st = _hip.LemoqOlmoeStep()
        st.hidden, st.heads, st.head_dim = s.hidden, s.heads, s.head_dim
        st.ffn, st.num_experts, st.top_k = s.ffn, s.num_experts, s.top_k
        st.vocab, st.group, st.num_layers = s.vocab, s.group_size, s.layers
        st.max_seq, st.num_splits, st.norm_topk_prob = S, self.num_splits, int(bool(s.norm_topk_prob))
        st.eps = float(s.eps)
        st.clip_qkv = math.inf if s.clip_qkv is None else float(s.clip_qkv)
        st.qk_scale = float((1.0 / math.sqrt(D)) * LOG2E)
        st.layers = ctypes.cast(self._layer_structs, ctypes.POINTER(_hip.LemoqOlmoeLayer))
        st.embed, st.final_norm = P(weights.embed), P(weights.final_norm)
        if weights.lm_f16 is not None:
            if not weights.lm_f16.is_contiguous() or weights.lm_f16.device != dev:
                raise ValueError("lm_f16 must be contiguous on %s" % dev)
            st.lm_f16, st.lm_codes, st.lm_scale = P(weights.lm_f16), None, None
        else:
            st.lm_codes, st.lm_scale, st.lm_f16 = P(weights.lm_codes), P(weights.lm_scale), None
        if weights.bits not in (4, 8):
            raise ValueError("weights.bits must be 4 or 8, got %r" % (weights.bits,))
        st.weight_bits = int(weights.bits)
        st.cos_tab, st.sin_tab = P(self.cos_tab), P(self.sin_tab)
        st.token, st.pos, st.filled = P(self.token), P(self.pos), P(self.filled)
        st.prompt, st.prompt_len = P(self.prompt), self.ctx
        st.history, st.history_len = P(self.history), int(self.history.numel())
        for name in ("h", "xn", "qkv", "q_rot", "attn", "part_m", "part_l", "part_acc",
                     "router_logits", "top_w", "top_i", "act", "logits", "am_val", "am_idx", "o_part",
                     "h_mid"):
            setattr(st, name, P(getattr(self, name)))
        st.am_len = n_parts
        st.kv_fp16 = int(kv_cache == "fp16")
        self._step = st
        self.graph: Any = None
        self.graph_multi: Any = None  # steps_per_graph decode steps in one graph (capture(steps_per_graph=K))
        self.steps_per_graph = 1
        self.stream: Any = None
        self._host_pos = 0
        self._seed_token: int | None = None
        self._prefill_weights: Any = None
        self.reset()

    # ------------------------------------------------------------------ state
    def reset(self) -> None:
        """Back to position 0 with the first prompt token (cache slots are overwritten as it runs)."""
        self._reset_device_state()
        torch.cuda.synchronize(self.device)

    def _reset_device_state(self) -> None:
        """The device side of ``reset``, enqueued on the current stream (no synchronisation)."""
        self.token.copy_(self.prompt[:1])
        self.pos.zero_()
        self.filled.fill_(1)
        self.history.zero_()
        self.history[:1].copy_(self.prompt[:1])
        self._host_pos = 0

    def set_position(self, position: int, token: int | None = None) -> None:
        """Move the decode position (graph-safe: only device scalars change)."""
        if position < 0 or position >= self.max_seq:
            raise RuntimeError("position %d outside the cache capacity %d" % (position, self.max_seq))
        self.pos.fill_(int(position))
        self.filled.fill_(int(position) + 1)
        if token is not None:
            self.token.fill_(int(token))
        self._host_pos = int(position)

    @property
    def position(self) -> int:
        """The device's decode position (synchronises); equals the host-side count
        the capacity check uses, which every step enqueued through this session
        advances."""
        return int(self.pos.item())

    # ------------------------------------------------------------------ steps
    def _enqueue_step(self) -> None:
        _hip.call("lemoq_olmoe_decode_step", ctypes.byref(self._step), _hip.stream_of(self.device))

    def _check_room(self, n: int) -> None:
        """Refuse, before anything is enqueued, a step that would run past the last
        cache slot (the device would attend over nothing and keep advancing).  Uses
        the host-side position, so it needs no device synchronisation."""
        if n < 0 or self._host_pos + n > self.max_seq:
            raise RuntimeError("decode position %d + %d steps would exceed the cache capacity %d"
                               % (self._host_pos, n, self.max_seq))

    def decode_eager(self) -> Any:
        """One step without the graph; returns the step's fp16 logits (device)."""
        self._check_room(1)
        self._enqueue_step()
        self._host_pos += 1
        return self.logits

    @property
    def attn_output_fused(self) -> bool:
        """Whether the step runs merge + o_proj as one launch and the residual add
        in the router launch (the shape rule of csrc/step.hip)."""
        s = self.shape
        HD = s.heads * s.head_dim
        return (bool(self._step.o_part) and bool(self._step.h_mid)
                and s.head_dim == 128 and s.heads % 4 == 0
                and self.num_splits <= 64 and s.hidden in (2048, 4096) and HD // 512 in (1, 2, 4, 8)
                and s.group_size % 16 == 0 and HD % s.group_size == 0)

    @property
    def launches_per_step(self) -> int:
        """Kernel launches in one captured step (see csrc/step.hip): 6 per layer
        on the fused attention-output path, 7 otherwise, the lm_head and greedy
        selection, and for a 4-bit step whose q|k|v GEMV cannot gather the
        embedding row itself (hidden not 2048 / 4096 / 8192) one gather."""
        per_layer = 6 if self.attn_output_fused else 7
        gather = self.weights.bits == 4 and self.shape.hidden not in (2048, 4096, 8192)
        return per_layer * self.shape.layers + 2 + int(gather)

    def capture(self, steps_per_graph: int = 1) -> dict[str, Any]:
        """Capture one decode step into a hipGraph (state is untouched by the capture).

        ``steps_per_graph`` K > 1 also captures K steps back to back into a second
        graph, which ``replay`` then uses for whole groups of K steps.  Each step
        reads and advances the device's position and token, so a K-step replay
        computes exactly what K one-step replays do, with one graph launch instead
        of K (the reference replays one step per graph and synchronises after
        each, ``benchmarks/cudagraph.py:751-766``).
        """
        k = int(steps_per_graph)
        if k < 1:
            raise ValueError("steps_per_graph must be >= 1, got %d" % k)
        if self.graph is None:
            self.stream = torch.cuda.Stream(device=self.device)
            self.stream.wait_stream(torch.cuda.current_stream(self.device))
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=self.stream):
                self._enqueue_step()
            torch.cuda.synchronize(self.device)
            self.graph = graph
        if k > 1 and (self.graph_multi is None or self.steps_per_graph != k):
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=self.stream):
                for _ in range(k):
                    self._enqueue_step()
            torch.cuda.synchronize(self.device)
            self.graph_multi = graph
            self.steps_per_graph = k
        return {"capture_success": True, "launches_per_step": self.launches_per_step,
                "steps_per_graph": self.steps_per_graph if self.graph_multi is not None else 1}

    def replay(self, n: int = 1, *, synchronize: bool = True) -> Any:
        """Replay the captured step ``n`` times back to back; returns the last logits.

        With a multi-step graph (``capture(steps_per_graph=K)``), ``n // K``
        replays of it run first, then ``n % K`` one-step replays."""
        if self.graph is None:
            raise RuntimeError("capture() must succeed before replay()")
        n = int(n)
        self._check_room(n)
        k = self.steps_per_graph if self.graph_multi is not None else 1
        for _ in range(n // k if k > 1 else 0):
            self.graph_multi.replay()
        for _ in range(n % k if k > 1 else n):
            self.graph.replay()
        self._host_pos += n
        if synchronize:
            torch.cuda.synchronize(self.device)
        return self.logits

    def prefill(self, mode: str = "batched", *, kv_f16: list | None = None) -> int:
        """Fill the KV cache with the prompt and seed the first decode token; returns it.

        ``mode="batched"`` (default) is the reference's prefill: one multi-token
        forward (``lemoq.model.prefill.prefill_prompt``, the path of
        ``StaticCacheDecodeSession.prefill``, ``benchmarks/cudagraph.py:578-599``),
        then the greedy pick of the last position's logits (``lemoq_argmax_advance``).
        ``mode="stepped"`` feeds the prompt through the captured decode step, one
        replay per position (decode numerics for every prompt token).
        ``kv_f16`` (batched only): a list that receives per layer the fp16 k and v
        rows the cache bytes were quantised from (see ``prefill_prompt``).  4-bit
        weights run the batched prefill on an int8 re-encoding of their codes
        (``OlmoeW8Weights.int8_codes``, made once per session and kept: for the
        OLMoE shape 6.7 GB beside the 4-bit weights), the separate arm's
        arithmetic; an fp16 lm_head ends it with the fp16 GEMV of the last row.
        """
        if mode not in ("batched", "stepped"):
            raise ValueError("prefill mode must be 'batched' or 'stepped', got %r" % (mode,))
        if self.graph is None:
            self.capture()
        # stream order keeps the reset ahead of the prefill's launches; the
        # seed token's read below synchronises once at the end
        self._reset_device_state()
        if mode == "stepped":
            self.replay(self.ctx)  # advances the host-side position to ctx
        elif mode == "batched":
            from lemoq.model.prefill import prefill_prompt  # noqa: PLC0415

            if self._prefill_weights is None:  # 4-bit codes as int8 for the prefill GEMMs, once
                self._prefill_weights = self.weights.int8_codes()
            self.history[: self.ctx].copy_(self.prompt)
            self.pos.fill_(self.ctx - 1)
            prefill_prompt(self._prefill_weights, self.prompt, self.kv, self.cos_tab, self.sin_tab, self.max_seq,
                           self.logits, step={"token": self.token, "pos": self.pos, "filled": self.filled,
                                              "history": self.history}, kv_f16=kv_f16)
            self._host_pos = self.ctx
        self._seed_token = int(self.token.item())
        return self._seed_token

    @property
    def seed_token_id(self) -> int:
        """The first decode token, chosen by ``prefill()`` (synchronises)."""
        if self._seed_token is None:
            raise RuntimeError("prefill must run before reading the seed token")
        return self._seed_token

    def next_token_cpu(self) -> int:
        """The token the next step consumes: the greedy pick of the last step (synchronises)."""
        return int(self.token.item())

    def replay_at_position(self, position: int, *, synchronize: bool = True) -> Any:
        """Replay the captured step at ``position`` (with the token already in
        place), as the reference's ``replay_at_position``; returns the logits."""
        p = int(position)
        if p < 0 or p >= self.max_seq:
            raise RuntimeError("position %d outside the cache capacity %d" % (p, self.max_seq))
        self.pos.fill_(p)
        self.filled.fill_(p + 1)
        self._host_pos = p
        return self.replay(1, synchronize=synchronize)

    def buffer_addresses(self) -> tuple[int, ...]:
        """Device addresses of the fixed step inputs and outputs (token, position,
        filled length, logits, history): they never move after construction, which
        is what lets one captured graph serve every step."""
        return tuple(int(t.data_ptr()) for t in (self.token, self.pos, self.filled, self.logits, self.history))

    def generated(self) -> list[int]:
        """Tokens chosen after the prompt so far (device history -> host)."""
        p = self.position
        return [int(t) for t in self.history[self.ctx : p + 1].tolist()]

    def logits_cpu(self) -> Any:
        torch.cuda.synchronize(self.device)
        return self.logits.detach().to("cpu").clone()

    def kv_cpu(self) -> list[dict[str, Any]]:
        """Host copy of every layer's KV cache (for the CPU oracle): kc/ks/vc/vs for
        KV-INT8, k/v for the fp16 cache."""
        torch.cuda.synchronize(self.device)
        return [{k: v.detach().to("cpu").clone() for k, v in kv.items()} for kv in self.kv]
