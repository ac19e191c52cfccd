"""The reference engine's eager decode step on the CPU -- TEST INFRASTRUCTURE.

Used only as ``bench.py``'s ``cpu_baseline`` leg: the CPU figure beside the
GPU numbers is this path timed on the host's cores.  It is not the parity
oracle (that is ``qwen3_cpu.Qwen3Oracle``, which follows HF's op sequence);
it restates the op sequence reference ``engine/engine.py`` runs when it has
no GPU (``self.cuda`` False: no Triton kernels, no graph, ``self.gqa`` False):

  * one fused q|k|v GEMM and one fused gate|up GEMM per layer
    (reference ``engine/engine.py:158-181``; F.linear ``:450``);
  * eager RMSNorm, per-head q/k RMSNorm + RoPE (``:75-109,458-462``);
  * the new key and value written with ``index_copy_`` at the device position
    (``:709-718``);
  * ``repeat_interleave`` of the whole K/V cache to the 32 query heads and SDPA
    over the full capacity with an additive ``NEG`` mask on the slots past the
    position (``:263-280,816-822``);
  * the residual add then the next norm (``_add_norm``, ``:452-456``);
    SwiGLU by ``chunk`` (``:464-468``); LM head + argmax (``:833``).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .qwen3_cpu import NEG, apply_rope, bf16_from_bits, rms_norm, rope_tables


class RefCpuDecode:
    """One self-feeding BF16 decode step of the reference engine's CPU path."""

    def __init__(self, cfg, tensors: dict):
        self.cfg = cfg
        self.Hq, self.Hkv, self.D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        self.eps = cfg.rms_norm_eps
        self.scale = cfg.head_dim ** -0.5

        def t(name):
            return bf16_from_bits(tensors[name])

        self.embed = t("model.embed_tokens.weight")
        self.lm_head = self.embed if cfg.tie_word_embeddings else t("lm_head.weight")
        self.final_norm = t("model.norm.weight")
        self.layers = []
        for i in range(cfg.num_hidden_layers):
            p = f"model.layers.{i}."
            self.layers.append({
                "in_ln": t(p + "input_layernorm.weight"),
                "post_ln": t(p + "post_attention_layernorm.weight"),
                "qkv": torch.cat([t(p + "self_attn.q_proj.weight"), t(p + "self_attn.k_proj.weight"),
                                  t(p + "self_attn.v_proj.weight")]).contiguous(),
                "q_norm": t(p + "self_attn.q_norm.weight"),
                "k_norm": t(p + "self_attn.k_norm.weight"),
                "o": t(p + "self_attn.o_proj.weight"),
                "gate_up": torch.cat([t(p + "mlp.gate_proj.weight"), t(p + "mlp.up_proj.weight")]).contiguous(),
                "down": t(p + "mlp.down_proj.weight"),
            })
        self.cache_k = self.cache_v = None

    def reset(self, batch: int, capacity: int) -> None:
        self.batch, self.capacity = batch, capacity
        self.cos, self.sin = rope_tables(self.cfg.rope_theta, self.D, max(capacity + 1, 4096))
        shape = (batch, self.Hkv, capacity, self.D)
        self.cache_k = [torch.zeros(shape, dtype=torch.bfloat16) for _ in self.layers]
        self.cache_v = [torch.zeros(shape, dtype=torch.bfloat16) for _ in self.layers]
        self.arange = torch.arange(capacity)

    @torch.inference_mode()
    def step(self, token: torch.Tensor, pos: int) -> torch.Tensor:
        """token [B, 1] at position ``pos`` -> the greedy next token [B, 1]."""
        B, Hq, Hkv, D, C = self.batch, self.Hq, self.Hkv, self.D, self.capacity
        q_size, kv_size = Hq * D, Hkv * D
        position = torch.tensor([pos])
        cos = self.cos.index_select(0, position).view(1, 1, 1, D)
        sin = self.sin.index_select(0, position).view(1, 1, 1, D)
        mask = torch.where(self.arange <= pos, 0.0, NEG).to(torch.bfloat16).view(1, 1, 1, C)
        residual = F.embedding(token, self.embed)
        n = rms_norm(residual, self.layers[0]["in_ln"], self.eps)
        for i, L in enumerate(self.layers):
            qkv = F.linear(n, L["qkv"])
            q, k, v = qkv.split([q_size, kv_size, kv_size], dim=-1)
            q = apply_rope(rms_norm(q.view(B, 1, Hq, D), L["q_norm"], self.eps), cos, sin)
            k = apply_rope(rms_norm(k.view(B, 1, Hkv, D), L["k_norm"], self.eps), cos, sin)
            self.cache_k[i].index_copy_(2, position, k.transpose(1, 2))
            self.cache_v[i].index_copy_(2, position, v.view(B, 1, Hkv, D).transpose(1, 2))
            keys = self.cache_k[i].repeat_interleave(Hq // Hkv, dim=1)
            values = self.cache_v[i].repeat_interleave(Hq // Hkv, dim=1)
            a = F.scaled_dot_product_attention(q.transpose(1, 2), keys, values, attn_mask=mask, scale=self.scale)
            a = a.transpose(1, 2).reshape(B, 1, q_size)
            residual = residual + F.linear(a, L["o"])
            m = rms_norm(residual, L["post_ln"], self.eps)
            gate, up = F.linear(m, L["gate_up"]).chunk(2, dim=-1)
            residual = residual + F.linear(F.silu(gate) * up, L["down"])
            nxt = self.layers[i + 1]["in_ln"] if i + 1 < len(self.layers) else self.final_norm
            n = rms_norm(residual, nxt, self.eps)
        return F.linear(n, self.lm_head)[:, -1, :].argmax(dim=-1, keepdim=True)
