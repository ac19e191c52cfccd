"""CPU oracle for Qwen3 greedy decode -- TEST INFRASTRUCTURE, not the product.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker (or as
the timed CPU baseline); the engine in ``starter_amd`` never does.

What it restates.  The reference engine's eager path (reference
``engine/engine.py``) and the "native Qwen" it is judged against
(transformers ``models/qwen3/modeling_qwen3.py``, pinned 4.51.3 in reference
``requirements.txt:11``; 5.15.0 is what is installed here) are the same
arithmetic: every op is a PyTorch op on BF16 tensors, so FP32 compute with a
round to BF16 after each op, and the cast boundaries below are the ones those
files write.  The forward here follows HF's op sequence (separate q/k/v and
gate/up projections, SDPA with ``enable_gqa``, a cache that holds exactly the
live keys), which is what the contest's judge replays
(reference ``QWEN_ENGINE_CONTRACT.md`` "The quality rule").

How it is pinned (tests/test_oracle.py):
  * against HF fixtures written by ``tests/golden/make_golden.py`` (token
    streams and logits for a tiny config in fp32 and bf16, and for the full
    Qwen3-4B config 1 in bf16);
  * per function against what the mathematics fixes: float64 closed forms
    with the cast placement applied by hand (RMSNorm, RoPE, SwiGLU, linear),
    brute-force softmax attention, identities (RoPE at position 0, a single
    key), and first-index argmax ties.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

#: Finite masked score, reference ``engine/engine.py:27-30``.
NEG = torch.finfo(torch.bfloat16).min


def bf16_from_bits(bits: np.ndarray) -> torch.Tensor:
    """BF16 tensor from raw uint16 bits (copies, so memmaps stay read-only)."""
    return torch.from_numpy(np.array(bits, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


def rope_tables(theta: float, head_dim: int, length: int, dtype=torch.bfloat16):
    """cos/sin for absolute positions [0, length).

    Reference ``engine/engine.py:240-259`` (``_grow_rope``) and HF
    ``Qwen3RotaryEmbedding`` (``modeling_qwen3.py:121,126-137``): FP32
    inverse frequencies ``1/theta^(2i/D)``, FP32 angle ``pos*inv``, the
    angles duplicated over both halves, cos/sin in FP32, one cast to BF16.
    """
    exponent = torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim
    inv_freq = 1.0 / (theta ** exponent)
    pos = torch.arange(length, dtype=torch.int64).float()
    freqs = torch.outer(pos, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype).contiguous(), emb.sin().to(dtype).contiguous()


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``Qwen3RMSNorm.forward``: reference ``engine/engine.py:75-88``, HF ``:59-64``.

    FP32 mean of squares, ``x * rsqrt(var + eps)`` in FP32, round to the input
    dtype, then the gain multiply as a BF16 op (a second rounding).
    """
    dtype = x.dtype
    xf = x.float()
    variance = xf.pow(2).mean(-1, keepdim=True)
    xf = xf * torch.rsqrt(variance + eps)
    return weight * xf.to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """Reference ``engine/engine.py:91-93``; HF ``modeling_qwen3.py:140-145``."""
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """``x*cos + rotate_half(x)*sin`` as three BF16 ops (each product rounds).

    Reference ``engine/engine.py:96-109``; HF ``apply_rotary_pos_emb``
    ``modeling_qwen3.py:148-170``.  ``cos``/``sin`` must broadcast against x.
    """
    return (x * cos) + (rotate_half(x) * sin)


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``silu(gate) * up``: reference ``engine/engine.py:464-468``, HF ``:81-83``.

    ``F.silu`` rounds to BF16, then the multiply rounds again.
    """
    return F.silu(gate) * up


def linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """``x @ W.T`` with FP32 accumulation and one BF16 rounding (``F.linear``)."""
    return F.linear(x, weight)


def argmax_first(logits: torch.Tensor) -> torch.Tensor:
    """Greedy choice: first maximal index over the BF16 logits (``torch.argmax``).

    Reference ``engine/engine.py:833,1077``; ``OPTIMIZATION_GUIDE.md`` LM-head row.
    """
    return logits.argmax(dim=-1)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
              start: int) -> torch.Tensor:
    """GQA attention of T queries at absolute positions start.. over keys 0..start+T-1.

    q ``[B,Hq,T,D]``, k/v ``[B,Hkv,start+T,D]`` (exactly the live keys).
    HF's SDPA glue (``integrations/sdpa_attention.py:97-163``): no mask and
    ``enable_gqa`` when the whole prompt is one forward (``is_causal`` for T>1);
    a later chunk spells the causal rule out as an additive mask with
    ``NEG`` (reference ``engine/engine.py:777-787``; ``j <= start + i``),
    which sends SDPA through ``repeat_kv``.
    """
    T = q.shape[2]
    if start == 0 or T == 1:
        return F.scaled_dot_product_attention(
            q, k, v, scale=scale, is_causal=T > 1, enable_gqa=True)
    groups = q.shape[1] // k.shape[1]
    keys = torch.arange(start + T)
    queries = torch.arange(start, start + T).unsqueeze(1)
    mask = torch.where(keys <= queries, 0.0, NEG).to(q.dtype).view(1, 1, T, start + T)
    k = k.repeat_interleave(groups, dim=1)
    v = v.repeat_interleave(groups, dim=1)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=scale)


class Qwen3Oracle:
    """Eager Qwen3 forward with a fixed-capacity cache, on the CPU.

    ``tensors`` maps HF names to raw BF16 bits (``np.uint16``), as returned by
    ``starter_amd.checkpoint.load_checkpoint``.  ``dtype`` is the compute
    dtype (BF16 for parity; FP32 reproduces the reference's fp32 CPU test,
    reference ``tests/test_equivalence.py:25-27``).
    """

    def __init__(self, cfg, tensors: dict, dtype=torch.bfloat16, threads: int | None = None,
                 device: str = "cpu"):
        if threads:
            torch.set_num_threads(threads)
        self.cfg = cfg
        self.dtype = dtype
        #: The oracle runs on the CPU.  ``device`` exists for the test harness's
        #: native comparator (``oracle/native_server.py``), which replays this
        #: op sequence eagerly on a GPU to time it; parity never uses it.
        self.device = torch.device(device)
        self.D = cfg.head_dim
        self.Hq = cfg.num_attention_heads
        self.Hkv = cfg.num_key_value_heads
        self.eps = cfg.rms_norm_eps
        self.scale = cfg.head_dim ** -0.5

        def t(name):
            return bf16_from_bits(tensors[name]).to(dtype).to(self.device)

        self.embed = t("model.embed_tokens.weight")
        self.lm_head = (self.embed if cfg.tie_word_embeddings
                        else t("lm_head.weight"))
        self.final_norm = t("model.norm.weight")
        self.layers = []
        for i in range(cfg.num_hidden_layers):
            p = f"model.layers.{i}."
            self.layers.append({
                "in_ln": t(p + "input_layernorm.weight"),
                "post_ln": t(p + "post_attention_layernorm.weight"),
                "q": t(p + "self_attn.q_proj.weight"),
                "k": t(p + "self_attn.k_proj.weight"),
                "v": t(p + "self_attn.v_proj.weight"),
                "o": t(p + "self_attn.o_proj.weight"),
                "q_norm": t(p + "self_attn.q_norm.weight"),
                "k_norm": t(p + "self_attn.k_norm.weight"),
                "gate": t(p + "mlp.gate_proj.weight"),
                "up": t(p + "mlp.up_proj.weight"),
                "down": t(p + "mlp.down_proj.weight"),
            })
        self.cos = self.sin = None
        self.cache_k = self.cache_v = None
        #: The projection; tests swap in another summation order (see
        #: ``f32_linear``) to measure what reordering alone moves.
        self.linear = linear
        #: The attention (``attention`` above); the GPU comparator swaps in its own.
        self.attend = attention

    def reset(self, batch: int, capacity: int) -> None:
        """Fresh cache of ``capacity`` slots (reference ``engine/engine.py:843-862``)."""
        cos, sin = rope_tables(self.cfg.rope_theta, self.D, max(capacity + 1, 4096), self.dtype)
        self.cos, self.sin = cos.to(self.device), sin.to(self.device)
        shape = (batch, self.Hkv, capacity, self.D)
        self.cache_k = self.cache_v = None
        self.cache_k = [torch.zeros(shape, dtype=self.dtype, device=self.device) for _ in self.layers]
        self.cache_v = [torch.zeros(shape, dtype=self.dtype, device=self.device) for _ in self.layers]

    def block(self, x: torch.Tensor, i: int, start: int) -> torch.Tensor:
        """One ``Qwen3DecoderLayer`` (HF ``modeling_qwen3.py:294-323``, attention ``:241-280``)."""
        L = self.layers[i]
        B, T, _ = x.shape
        cos = self.cos[start:start + T].view(1, 1, T, self.D)
        sin = self.sin[start:start + T].view(1, 1, T, self.D)

        residual = x
        h = rms_norm(x, L["in_ln"], self.eps)
        lin = self.linear
        q = rms_norm(lin(h, L["q"]).view(B, T, self.Hq, self.D), L["q_norm"], self.eps)
        k = rms_norm(lin(h, L["k"]).view(B, T, self.Hkv, self.D), L["k_norm"], self.eps)
        v = lin(h, L["v"]).view(B, T, self.Hkv, self.D)
        q = apply_rope(q.transpose(1, 2), cos, sin)
        k = apply_rope(k.transpose(1, 2), cos, sin)
        self.cache_k[i][:, :, start:start + T] = k
        self.cache_v[i][:, :, start:start + T] = v.transpose(1, 2)
        a = self.attend(q, self.cache_k[i][:, :, :start + T], self.cache_v[i][:, :, :start + T],
                        self.scale, start)
        a = a.transpose(1, 2).reshape(B, T, self.Hq * self.D)
        x = residual + lin(a, L["o"])

        residual = x
        h = rms_norm(x, L["post_ln"], self.eps)
        mlp = lin(swiglu(lin(h, L["gate"]), lin(h, L["up"])), L["down"])
        return residual + mlp

    @torch.inference_mode()
    def forward(self, ids: torch.Tensor, start: int) -> torch.Tensor:
        """Consume ``ids [B,T]`` at positions start..start+T-1; logits ``[B,V]`` of the last."""
        x = F.embedding(ids.to(self.device), self.embed)
        for i in range(len(self.layers)):
            x = self.block(x, i, start)
        x = rms_norm(x, self.final_norm, self.eps)
        return self.linear(x[:, -1, :], self.lm_head)

    @torch.inference_mode()
    def prefill(self, ids: torch.Tensor, chunk: int | None = None) -> torch.Tensor:
        """Prompt pass, optionally in chunks of ``chunk`` tokens per row
        (reference ``engine/engine.py:738-803``)."""
        P = ids.shape[1]
        chunk = chunk or P
        logits = None
        for s in range(0, P, chunk):
            logits = self.forward(ids[:, s:s + chunk], s)
        return logits

    @torch.inference_mode()
    def generate(self, input_ids: list[list[int]], max_new_tokens: int,
                 keep_logits: bool = False, chunk: int | None = None):
        """The baseline greedy loop (reference ``tests/test_equivalence.py:72-86``).

        Returns ``(steps, logits)``: ``steps`` is a list of ``max_new_tokens``
        lists of B ids; ``logits[i]`` (when kept) is the ``[B,V]`` tensor step
        i's ids were chosen from.
        """
        ids = torch.tensor(input_ids, dtype=torch.int64)
        B, P = ids.shape
        self.reset(B, P + max_new_tokens)
        steps, kept = [], []
        logits = self.prefill(ids, chunk)
        for step in range(max_new_tokens):
            token = argmax_first(logits)
            steps.append(token.tolist())
            if keep_logits:
                kept.append(logits.clone())
            if step + 1 < max_new_tokens:
                logits = self.forward(token.view(B, 1), P + step)
        return steps, kept


class f32_linear:
    """``x @ W.T`` summed by torch's FP32 GEMM (weights kept as FP32 copies),
    rounded once to BF16: the same products and one rounding as ``linear``, in
    another summation order -- a reordering the reference accepts
    (``AGENTS.md`` "reorder freely, never reformulate").  Used only to
    measure the logit noise that reordering alone produces."""

    def __init__(self):
        self.w32 = {}

    def __call__(self, x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
        w = self.w32.get(id(weight))
        if w is None:
            w = self.w32[id(weight)] = weight.float()
        return (x.float() @ w.T).to(x.dtype)


def top2_gap(logits: torch.Tensor) -> torch.Tensor:
    """Per-row gap between the largest and second-largest logit (FP32)."""
    top = logits.float().topk(2, dim=-1).values
    return top[..., 0] - top[..., 1]


def reference_tables_f64(theta: float, head_dim: int, length: int):
    """float64 closed form of the RoPE angles (for pinning ``rope_tables``)."""
    i = np.arange(0, head_dim, 2, dtype=np.float64)
    inv = 1.0 / np.power(theta, i / head_dim)
    ang = np.outer(np.arange(length, dtype=np.float64), inv)
    ang = np.concatenate([ang, ang], axis=1)
    return np.cos(ang), np.sin(ang)


def softmax_attention_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    """Brute-force float64 attention of one query row over keys (for pinning)."""
    s = (k.astype(np.float64) @ q.astype(np.float64)) * scale
    p = np.exp(s - s.max())
    return (p[:, None] * v.astype(np.float64)).sum(0) / p.sum()


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even to BF16, returned as float64 (for pinning)."""
    f = np.asarray(x, dtype=np.float64).astype(np.float32).view(np.uint32).astype(np.uint64)
    r = ((f + 0x7FFF + ((f >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).astype(np.float64)


def ulp_bf16(x: float) -> float:
    """Spacing of BF16 values at |x| (for tolerances written in tests)."""
    if x == 0:
        return 2.0 ** -133
    return 2.0 ** (math.floor(math.log2(abs(x))) - 7)
