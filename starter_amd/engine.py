"""Qwen3-4B greedy decode on MI355X: the drop-in ``Engine`` of reference ``engine/engine.py``.

API (identical to reference ``engine/engine.py:112-118,1069-1105``;
``QWEN_ENGINE_CONTRACT.md`` "What you submit"):

    eng = Engine(model_path)                 # local HF checkpoint directory
    for step in eng.generate(input_ids, max_new_tokens):
        ...                                  # list[int], one id per sequence

``generate`` yields exactly ``max_new_tokens`` lists, greedy (first index on
exact ties), every call starting from a clean state.  The private
``_ensure_shape(batch, prompt, new)`` and ``_forward_prefill(ids, prompt)``
keep the reference's names (its tests call them, reference
``tests/test_equivalence.py:161-163``).

Everything below the API is new: PyTorch-ROCm owns device memory and the
stream; every operation of the forward is a gfx950 HIP kernel in
``csrc/`` called through the C ABI of ``include/q3.h`` (``_lib``).  There is
no eager or PyTorch fallback: if ``libq3.so`` is missing, construction fails.

Device layout (bytes sized for one 288 GB HBM3E device):
  * weights, BF16, [N, K] row-major: per layer ``qkv`` [6144, 2560]
    (q | k | v rows), ``o`` [2560, 4096], ``gate_up`` [19456, 2560] with gate
    and up rows interleaved (row 2j = gate_j, 2j+1 = up_j) so one wave or
    tile owns both halves of its SwiGLU outputs, ``down`` [2560, 9728];
    the tied embedding [151936, 2560] doubles as the LM head;
  * KV cache: K and V each one allocation [layers, B, 8, capacity, 128] BF16,
    capacity = prompt + new tokens (reference ``engine/engine.py:844-862``);
  * RoPE tables [max(4096, capacity + 1), 128] BF16, computed on the host in
    FP32 exactly as the reference does and uploaded once per shape.

Decode step (one hipGraph, self-feeding like reference ``:805-839``), B <= 8:
  gemv(embed+norm -> qkv) | attn(norm/rope/append + split-K GQA) | merge |
  gemv(o, +residual) | gemv(norm -> gate_up -> SwiGLU) | gemv(down, +residual) |
  gemv(norm -> qkv of the next layer) ... | gemv(norm -> lm_head -> argmax
  partials) | argmax finish (token -> input buffer, pos += 1).
For B > GEMV_BATCH_MAX the projections stream 16-row tiled weight copies into
MFMA (B <= 64), their split-K partials summed by the consuming kernel (the
attention prologue, the residual add + RMSNorm); above 64 rows, or for shapes
that do not tile, the LDS-tiled MFMA GEMM with separate norm kernels.
"""

from __future__ import annotations

import ctypes
import os
import sys
import time

import numpy as np
import torch

from . import _lib
from ._lib import call
from .checkpoint import Qwen3Config, load_checkpoint

DEVICE = "cuda:0"

#: The weights' dtype (reference ``engine/engine.py`` ``LOAD_DTYPE``, which its
#: CPU test sets to float32).  The kernels compute in BF16 only, so any other
#: value is refused at construction rather than silently ignored.
LOAD_DTYPE = torch.bfloat16

#: Prompt tokens (batch x prompt) per prefill chunk.  The reference caps a
#: chunk at 16384 tokens for an 80 GB H100 (``engine/engine.py:34``); with
#: 288 GB the full 131072-token prompts of the benchmark fit in one pass
#: (~8 GB of activations).
PREFILL_CHUNK_TOKENS = 131072

#: Headroom kept free when sizing the KV cache.
MEMORY_MARGIN_BYTES = 2 << 30

#: Largest decode batch on the dot2 GEMVs (fused norm prologue and argmax
#: epilogue).  Above it, up to SKINNY_BATCH_MAX, projections stream 16-row
#: tiled weight copies into MFMA (``q3_skinny_tiled``), which at 5+ rows beats
#: the GEMV's VALU-bound dot products; above that the LDS-tiled GEMM.
GEMV_BATCH_MAX = 4
SKINNY_BATCH_MAX = 64

#: Decode attention and its split merge in one launch where the grid allows it
#: (``q3_attn_decode_fused``); False keeps two launches (tests compare them).
FUSED_ATTENTION = os.environ.get("Q3_FUSED_ATTENTION", "1") != "0"
FUSED_ATTENTION_MAX_LAYERS = 64

#: At 1-2 rows, also the q|k|v projection in that launch (``q3_qkv_attn``):
#: attention starts streaming its keys while the projection runs and waits
#: only for its own KV head's rows; at one row the o projection and its
#: residual join too (their weights stream while the attention runs).  False
#: keeps the projections separate.
QKV_ATTENTION = os.environ.get("Q3_QKV_ATTENTION", "1") != "0"

#: At one row, also the previous layer's down projection and residual join in
#: that launch (``q3_down_qkv_attn``): its weights stream beside the q|k|v
#: rows', which wait for its residual as flagged words, one kernel boundary
#: fewer per layer.  False keeps the down projection a launch of its own.
DOWN_ATTENTION = os.environ.get("Q3_DOWN_ATTENTION", "1") != "0"

#: The contest judge's tie margin (reference QWEN_ENGINE_CONTRACT.md
#: "tieMarginLogits", currently 2.0): an emitted token must be the replayed
#: argmax or within this many logits of it.
TIE_MARGIN_LOGITS = 2.0


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _log(msg: str) -> None:
    # stderr: stdout belongs to the caller (bench.py prints one JSON line there).
    print(f"[engine] {msg}", file=sys.stderr, flush=True)


def rope_tables(theta: float, head_dim: int, length: int) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin [length, head_dim] in BF16, built in FP32 on the host.

    Same formula and cast point as reference ``engine/engine.py:240-259``:
    ``inv = 1/theta**(arange(0, D, 2)/D)`` (FP32), ``freqs = outer(pos, inv)``,
    ``emb = cat(freqs, freqs)``, cos/sin in FP32, one cast to BF16.
    """
    exponent = torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim
    inv_freq = 1.0 / (theta ** exponent)
    pos = torch.arange(length, dtype=torch.int64).float()
    emb = torch.cat((torch.outer(pos, inv_freq),) * 2, dim=-1)
    return emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)


def _check_ids(input_ids, vocab: int) -> torch.Tensor:
    """Prompt ids as an int64 [B, P] tensor; ids index the embedding table on the
    device, so anything outside [0, vocab) is rejected here."""
    ids = torch.tensor(input_ids, dtype=torch.int64)
    if ids.dim() != 2 or ids.shape[0] == 0 or ids.shape[1] == 0:
        raise ValueError("input_ids must be a non-empty list of equal-length, non-empty lists")
    if int(ids.min()) < 0 or int(ids.max()) >= vocab:
        raise ValueError(f"token ids must lie in [0, {vocab})")
    return ids


def _bf16(arr: np.ndarray, device: str) -> torch.Tensor:
    a = np.ascontiguousarray(arr)
    if not a.flags.writeable:  # read-only memory map: torch wants a writable buffer
        a = a.copy()
    host = torch.from_numpy(a.view(np.int16))
    return host.to(device, non_blocking=False).view(torch.bfloat16)


class Engine:
    """Greedy Qwen3 decode engine; dimensions come from the checkpoint's config."""

    def __init__(self, model_path: str) -> None:
        if LOAD_DTYPE != torch.bfloat16:
            raise ValueError(f"LOAD_DTYPE {LOAD_DTYPE}: the gfx950 kernels compute in BF16 only")
        if not torch.cuda.is_available() or not str(DEVICE).startswith("cuda"):
            raise RuntimeError(f"Engine needs a ROCm GPU (gfx950) as DEVICE, got {DEVICE!r} "
                               f"(visible: {torch.cuda.is_available()}); there is no CPU path")
        _lib.lib()  # fail now, not mid-generation, if the kernels are not built
        self.device = torch.device(DEVICE)
        torch.cuda.set_device(self.device)
        self.started = time.monotonic()
        cfg, tensors = load_checkpoint(model_path)
        self.cfg: Qwen3Config = cfg
        self.LAYERS = cfg.num_hidden_layers
        self.HIDDEN = cfg.hidden_size
        self.INTER = cfg.intermediate_size
        self.HEADS = cfg.num_attention_heads
        self.KV_HEADS = cfg.num_key_value_heads
        self.HEAD_DIM = cfg.head_dim
        self.VOCAB = cfg.vocab_size
        self.EPS = float(cfg.rms_norm_eps)
        self.THETA = float(cfg.rope_theta)
        self.SCALE = self.HEAD_DIM ** -0.5
        if self.HEAD_DIM != 128 or self.HEADS != 4 * self.KV_HEADS:
            raise ValueError("kernels are built for head_dim 128 and 4 query heads per KV head")
        if self.HIDDEN % 64 or self.INTER % 64 or self.HIDDEN > _lib.GEMV_MAX_NORM_K:
            raise ValueError("hidden and intermediate sizes must be multiples of 64; hidden <= 4096")
        self.q_size = self.HEADS * self.HEAD_DIM
        self.kv_size = self.KV_HEADS * self.HEAD_DIM
        self.qkv_size = self.q_size + 2 * self.kv_size
        self.stream = torch.cuda.Stream(device=self.device)

        dev = DEVICE
        self.embed = _bf16(tensors["model.embed_tokens.weight"], dev)
        self.lm_head = (self.embed if cfg.tie_word_embeddings
                        else _bf16(tensors["lm_head.weight"], dev))
        self.final_norm = _bf16(tensors["model.norm.weight"], dev)
        self.layers = []
        for i in range(self.LAYERS):
            p = f"model.layers.{i}."
            qkv = np.concatenate([tensors[p + "self_attn.q_proj.weight"],
                                  tensors[p + "self_attn.k_proj.weight"],
                                  tensors[p + "self_attn.v_proj.weight"]], axis=0)
            gate, up = tensors[p + "mlp.gate_proj.weight"], tensors[p + "mlp.up_proj.weight"]
            gate_up = np.stack([gate, up], axis=1).reshape(2 * self.INTER, self.HIDDEN)
            self.layers.append({
                "in_ln": _bf16(tensors[p + "input_layernorm.weight"], dev),
                "post_ln": _bf16(tensors[p + "post_attention_layernorm.weight"], dev),
                "q_norm": _bf16(tensors[p + "self_attn.q_norm.weight"], dev),
                "k_norm": _bf16(tensors[p + "self_attn.k_norm.weight"], dev),
                "qkv": _bf16(qkv, dev),
                "o": _bf16(tensors[p + "self_attn.o_proj.weight"], dev),
                "gate_up": _bf16(gate_up, dev),
                "down": _bf16(tensors[p + "mlp.down_proj.weight"], dev),
            })
        del tensors
        torch.cuda.synchronize()

        self.rope_len = 0
        self.cos_table = self.sin_table = None
        self._grow_rope(4096)

        self.tiled = None  # 16-row tiled weight copies, made on first use
        self.batch = 0
        self.capacity = 0
        self.cache_k = self.cache_v = None
        self.graph = None
        self.keep_logits = False
        self._prefill_bufs = {}
        self._prefill_part = None
        _log(f"loaded {self.LAYERS} layers in {time.monotonic() - self.started:.1f}s; "
             f"qkv and gate_up packed")

    # ------------------------------------------------------------------ rope

    def _grow_rope(self, length: int) -> None:
        if length <= self.rope_len:
            return
        length = max(length, 4096)
        cos, sin = rope_tables(self.THETA, self.HEAD_DIM, length)
        self.cos_table = cos.to(self.device)
        self.sin_table = sin.to(self.device)
        self.rope_len = length

    # --------------------------------------------------------------- helpers

    @property
    def _s(self) -> int:
        return self.stream.cuda_stream

    def _empty(self, *shape, dtype=torch.bfloat16):
        return torch.empty(*shape, dtype=dtype, device=self.device)

    # ------------------------------------------------------------ shape prep

    def _ensure_shape(self, batch: int, seq_len: int, max_new_tokens: int) -> None:
        """(Re)build caches, decode buffers and the decode graph for (batch, capacity).

        Keyed on (batch, prompt + new) like reference ``engine/engine.py:843-880``,
        so a different prompt/new split with the same capacity reuses the graph:
        nothing in it depends on the prompt length (positions are device data).
        """
        capacity = seq_len + max_new_tokens
        if self.batch == batch and self.capacity == capacity and self.graph is not None:
            return
        _log(f"building for batch={batch} capacity={capacity}")
        self._release_graph()
        self.cache_k = self.cache_v = None
        self._prefill_bufs = {}
        self._prefill_part = None
        torch.cuda.synchronize()
        torch.cuda.empty_cache()

        self._grow_rope(capacity + 1)
        L, Hkv, D = self.LAYERS, self.KV_HEADS, self.HEAD_DIM
        cache_bytes = 2 * L * batch * Hkv * capacity * D * 2
        free, _ = torch.cuda.mem_get_info(self.device)
        if cache_bytes + MEMORY_MARGIN_BYTES > free:
            raise MemoryError(f"KV cache needs {cache_bytes / 2**30:.1f} GiB; "
                              f"{free / 2**30:.1f} GiB free")
        self.cache_k = torch.zeros(L, batch, Hkv, capacity, D, dtype=torch.bfloat16, device=self.device)
        self.cache_v = torch.zeros_like(self.cache_k)
        self.batch, self.capacity = batch, capacity

        B, H, V = batch, self.HIDDEN, self.VOCAB
        self.splits = call("q3_attn_splits", B, Hkv, capacity)
        # Where one split would leave half the CUs idle (128 sequence x KV head
        # pairs), two splits whose second hands its partial to the first; the
        # two-launch path then also takes two splits (and a merge launch), so
        # both compute the same bits.  Decided before anything is sized by the
        # split count.
        pair_ok = (self.LAYERS <= FUSED_ATTENTION_MAX_LAYERS and
                   call("q3_attn_pair_grid", B, self.HEADS, Hkv, capacity) > 0)
        if pair_ok:
            self.splits = 2
        self.g_token = torch.zeros(B, dtype=torch.int64, device=self.device)
        self.g_pos = torch.zeros(1, dtype=torch.int64, device=self.device)
        self.g_counter = torch.zeros(1, dtype=torch.int32, device=self.device)
        # Step records (q3.h): the token fed at each position (-1: the greedy
        # choice) and, per position, {argmax, max logit, fed token's logit,
        # fed token}; read by replay(), never by the host inside the graph.
        self.g_feed = torch.full((capacity + 1, B), -1, dtype=torch.int64, device=self.device)
        self.g_rec = torch.zeros(capacity + 1, B, 4, dtype=torch.int32, device=self.device)
        self.resid = self._empty(B, H)
        self.nbuf = self._empty(B, H)
        self.qkv_buf = self._empty(B, self.qkv_size)
        self.attn_out = self._empty(B, self.q_size)
        self.act = self._empty(B, self.INTER)
        self.part_acc = self._empty(B, self.HEADS, self.splits, D, dtype=torch.float32)
        self.part_ml = self._empty(B, self.HEADS, self.splits, 2, dtype=torch.float32)
        # Attention and its split merge in one launch when the grid is small
        # enough (batch 1-4 at moderate context): flagged exchange words, zeroed
        # at the start of every call, and a timeout word checked every step.
        # The exchange words' flag encodes (position, layer) with layer < 64
        # (q3_attn_decode_fused), so deeper models keep the two launches.
        self.attn_pair = FUSED_ATTENTION and pair_ok
        self.attn_fused = self.attn_pair or (FUSED_ATTENTION and self.splits > 1 and
                                             self.LAYERS <= FUSED_ATTENTION_MAX_LAYERS and
                                             call("q3_attn_fused_grid", B, self.HEADS, Hkv, capacity,
                                                  self.splits) > 0)
        words = (call("q3_attn_xbuf_words", B, self.HEADS, 2 if self.attn_pair else self.splits)
                 if self.attn_fused else 4)
        self.attn_x = torch.zeros(words, dtype=torch.int32, device=self.device)
        self.attn_err = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.small = B <= GEMV_BATCH_MAX
        # The q|k|v projection in the same launch, its outputs passed as
        # flagged words (cleared with the attention's).
        self.qkv_attn = (QKV_ATTENTION and self.small and self.attn_fused and
                         call("q3_qkv_attn_grid", B, self.HEADS, Hkv, capacity, self.splits, H, 0) > 0)
        self.qkv_attn_o = (self.qkv_attn and
                           call("q3_qkv_attn_grid", B, self.HEADS, Hkv, capacity, self.splits, H, 1) > 0)
        self.down_attn = (DOWN_ATTENTION and self.qkv_attn_o and
                          call("q3_down_qkv_attn_grid", self.HEADS, Hkv, capacity, self.splits, H, self.INTER) > 0)
        self.rx = torch.zeros(call("q3_down_rx_words", H) if self.down_attn else 4, dtype=torch.int32,
                              device=self.device)
        self.qkv_x = torch.zeros(B * self.qkv_size if self.qkv_attn else 4, dtype=torch.int32, device=self.device)
        self.o_x = torch.zeros(B * self.q_size if self.qkv_attn_o else 4, dtype=torch.int32, device=self.device)
        # Rows per workgroup of the gate/up GEMV, whose weights that launch
        # brings into L2 ahead of it.
        self.gate_up_group = 2 * self.INTER // call("q3_gemv_partials", B, 2 * self.INTER, _lib.EPI_SWIGLU)
        self.skinny = not self.small and B <= SKINNY_BATCH_MAX and self._skinny_shapes_ok(B)
        # Split-K workspace of the MFMA decode projections: every projection's
        # partials, [splits, B, N] FP32, one consumer at a time.
        ws = 0
        if self.skinny:
            self._make_tiled()
            for N, K in self._projections():
                ws = max(ws, call("q3_skinny_splits", B, N, K) * B * N)
        self.skinny_ws = self._empty(max(ws, 1), dtype=torch.float32)
        if self.small:
            self.lm_parts = call("q3_gemv_partials", B, V, _lib.EPI_ARGMAX)
        elif self.skinny:
            self.lm_parts = V // 64
        if self.small or self.skinny:
            self.part_val = self._empty(self.lm_parts, B, dtype=torch.float32)
            self.part_idx = self._empty(self.lm_parts, B, dtype=torch.int32)
        self.logits = self._empty(B, V)
        self._capture()

    def _records(self) -> tuple:
        """(feed, rec, npos) of the step records, as the LM-head and argmax-finish launchers take them."""
        return _ptr(self.g_feed), _ptr(self.g_rec), self.capacity + 1

    def _projections(self) -> list[tuple[int, int]]:
        """(N, K) of qkv, o, gate_up, down and the LM head."""
        H = self.HIDDEN
        return [(self.qkv_size, H), (H, self.q_size), (2 * self.INTER, H), (H, self.INTER), (self.VOCAB, H)]

    def _skinny_shapes_ok(self, B: int) -> bool:
        """The fused MFMA decode path needs every projection to tile (N % 64,
        K % 256, at most 16 splits), the LM head unsplit, hidden <= 4096."""
        if self.HIDDEN > 4096:
            return False
        for N, K in self._projections():
            if N % 64 or K % 256 or call("q3_skinny_splits", B, N, K) > 16:
                return False
        return call("q3_skinny_splits", B, self.VOCAB, self.HIDDEN) == 1

    def _make_tiled(self) -> None:
        """16-row tiled copies of every decode weight (``q3_tile16``), kept for the
        engine's lifetime: 8 GB next to the row-major set, which the GEMVs and the
        prefill GEMM read."""
        if self.tiled is not None:
            return
        t0 = time.monotonic()
        tiled = {}
        with torch.cuda.stream(self.stream):
            for w in [self.lm_head] + [L[k] for L in self.layers for k in ("qkv", "o", "gate_up", "down")]:
                if id(w) in tiled or w.shape[0] % 16 or w.shape[1] % 32:
                    continue
                t = torch.empty_like(w)
                call("q3_tile16", _ptr(w), w.shape[0], w.shape[1], _ptr(t), self._s)
                tiled[id(w)] = t
        self.stream.synchronize()
        self.tiled = tiled
        _log(f"tiled weight copies made in {time.monotonic() - t0:.2f}s")

    def _release_graph(self) -> None:
        if self.graph is not None:
            torch.cuda.synchronize()
            call("q3_graph_destroy", self.graph)
            self.graph = None

    def __del__(self):
        try:
            self._release_graph()
        except Exception:  # noqa: BLE001 - interpreter shutdown
            pass

    # --------------------------------------------------------------- decode

    def _enqueue_decode(self) -> None:
        """One self-feeding decode step on ``self.stream`` (reference ``_forward_decode``)."""
        if self.skinny:
            self._enqueue_decode_skinny()
            return
        s = self._s
        B, H, I, V = self.batch, self.HIDDEN, self.INTER, self.VOCAB
        D, Hq, Hkv, C = self.HEAD_DIM, self.HEADS, self.KV_HEADS, self.capacity
        layer_stride = self.cache_k[0].numel() * 2
        kc0, vc0 = self.cache_k.data_ptr(), self.cache_v.data_ptr()
        tok, pos = _ptr(self.g_token), _ptr(self.g_pos)
        resid, qkv, attn, act, nbuf = (_ptr(self.resid), _ptr(self.qkv_buf), _ptr(self.attn_out),
                                       _ptr(self.act), _ptr(self.nbuf))
        for i, L in enumerate(self.layers):
            if self.qkv_attn:
                self._qkv_attn_layer(i, L)
            elif self.small:
                if i == 0:
                    call("q3_gemv", _lib.X_EMBED_NORM, _ptr(self.embed), H, tok, _ptr(L["in_ln"]), self.EPS,
                         resid, _ptr(L["qkv"]), B, self.qkv_size, H, _lib.EPI_STORE, qkv, self.qkv_size,
                         None, None, None, None, None, 0, s)
                else:
                    call("q3_gemv", _lib.X_NORM, resid, H, None, _ptr(L["in_ln"]), self.EPS, None,
                         _ptr(L["qkv"]), B, self.qkv_size, H, _lib.EPI_STORE, qkv, self.qkv_size,
                         None, None, None, None, None, 0, s)
            else:
                if i == 0:
                    call("q3_embed_rmsnorm", tok, _ptr(self.embed), resid, nbuf, _ptr(L["in_ln"]), B, H,
                         self.EPS, s)
                else:
                    call("q3_rmsnorm", resid, H, _ptr(L["in_ln"]), nbuf, H, B, H, self.EPS, s)
                self._proj(nbuf, H, L["qkv"], self.qkv_size, H, _lib.EPI_STORE, qkv, self.qkv_size)
            if not self.qkv_attn:
                self._attention(i, L, (qkv, self.qkv_size, None, 0), kc0 + i * layer_stride,
                                vc0 + i * layer_stride)
            if self.small:
                if not self.qkv_attn_o:
                    call("q3_gemv", _lib.X_PLAIN, attn, self.q_size, None, None, 0.0, None, _ptr(L["o"]),
                         B, H, self.q_size, _lib.EPI_RESID, resid, H, None, None, None, None, None, 0, s)
                call("q3_gemv", _lib.X_NORM, resid, H, None, _ptr(L["post_ln"]), self.EPS, None,
                     _ptr(L["gate_up"]), B, 2 * I, H, _lib.EPI_SWIGLU, act, I, None, None, None, None, None, 0, s)
                if not (self.down_attn and i + 1 < self.LAYERS):  # else in the next layer's launch
                    call("q3_gemv", _lib.X_PLAIN, act, I, None, None, 0.0, None, _ptr(L["down"]),
                         B, H, I, _lib.EPI_RESID, resid, H, None, None, None, None, None, 0, s)
            else:
                self._proj(attn, self.q_size, L["o"], H, self.q_size, _lib.EPI_RESID, resid, H)
                call("q3_rmsnorm", resid, H, _ptr(L["post_ln"]), nbuf, H, B, H, self.EPS, s)
                self._proj(nbuf, H, L["gate_up"], 2 * I, H, _lib.EPI_SWIGLU, act, I)
                self._proj(act, I, L["down"], H, I, _lib.EPI_RESID, resid, H)
        if self.small:
            epi = _lib.EPI_STORE_ARGMAX if self.keep_logits else _lib.EPI_ARGMAX
            call("q3_gemv", _lib.X_NORM, resid, H, None, _ptr(self.final_norm), self.EPS, None,
                 _ptr(self.lm_head), B, V, H, epi, _ptr(self.logits), V, _ptr(self.part_val),
                 _ptr(self.part_idx), pos, *self._records(), s)
            call("q3_argmax_finish", _ptr(self.part_val), _ptr(self.part_idx), self.lm_parts, B, tok, pos,
                 _ptr(self.g_counter), *self._records(), s)
        else:
            call("q3_rmsnorm", resid, H, _ptr(self.final_norm), nbuf, H, B, H, self.EPS, s)
            self._proj(nbuf, H, self.lm_head, V, H, _lib.EPI_STORE, _ptr(self.logits), V)
            call("q3_argmax_rows", _ptr(self.logits), V, B, V, tok, pos, _ptr(self.g_counter), *self._records(), s)

    def _enqueue_decode_skinny(self) -> None:
        """Decode step for 5..64 rows: tiled-weight MFMA projections whose split-K
        partials go straight to their consumers -- qkv into the attention
        prologue, o and down into the residual add + next RMSNorm -- so a layer is
        seven or eight kernels (reference ``engine/engine.py:805-839`` runs the
        same math as separate ops)."""
        s = self._s
        B, H, I, V = self.batch, self.HIDDEN, self.INTER, self.VOCAB
        Hq, Hkv, C = self.HEADS, self.KV_HEADS, self.capacity
        layer_stride = self.cache_k[0].numel() * 2
        kc0, vc0 = self.cache_k.data_ptr(), self.cache_v.data_ptr()
        tok, pos = _ptr(self.g_token), _ptr(self.g_pos)
        resid, attn, act, nbuf, ws = (_ptr(self.resid), _ptr(self.attn_out), _ptr(self.act), _ptr(self.nbuf),
                                      _ptr(self.skinny_ws))
        T = lambda w: _ptr(self.tiled[id(w)])  # noqa: E731
        s_qkv = call("q3_skinny_splits", B, self.qkv_size, H)
        s_o = call("q3_skinny_splits", B, H, self.q_size)
        s_down = call("q3_skinny_splits", B, H, I)
        call("q3_embed_rmsnorm", tok, _ptr(self.embed), resid, nbuf, _ptr(self.layers[0]["in_ln"]), B, H,
             self.EPS, s)
        for i, L in enumerate(self.layers):
            call("q3_skinny_partials", nbuf, H, T(L["qkv"]), B, self.qkv_size, H, ws, s)
            self._attention(i, L, (None, self.qkv_size, ws, s_qkv), kc0 + i * layer_stride, vc0 + i * layer_stride)
            call("q3_skinny_partials", attn, self.q_size, T(L["o"]), B, H, self.q_size, ws, s)
            call("q3_add_rmsnorm_partials", ws, s_o, resid, _ptr(L["post_ln"]), nbuf, B, H, self.EPS, s)
            call("q3_skinny_tiled", nbuf, H, T(L["gate_up"]), B, 2 * I, H, _lib.EPI_SWIGLU, act, I, ws, s)
            call("q3_skinny_partials", act, I, T(L["down"]), B, H, I, ws, s)
            nxt = self.layers[i + 1]["in_ln"] if i + 1 < self.LAYERS else self.final_norm
            call("q3_add_rmsnorm_partials", ws, s_down, resid, _ptr(nxt), nbuf, B, H, self.EPS, s)
        call("q3_skinny_argmax", nbuf, H, T(self.lm_head), B, V, H, _ptr(self.logits) if self.keep_logits else None,
             V, _ptr(self.part_val), _ptr(self.part_idx), pos, *self._records(), s)
        call("q3_argmax_finish", _ptr(self.part_val), _ptr(self.part_idx), self.lm_parts, B, tok, pos,
             _ptr(self.g_counter), *self._records(), s)

    def _qkv_attn_layer(self, i: int, L: dict) -> None:
        """Layer i's q|k|v projection, attention and split merge as one launch
        (``q3_qkv_attn``), with the o projection and its residual join at one
        row (``qkv_attn_o``); layer 0 takes its input from the embedding.  With
        ``down_attn``, layers past the first also run layer i - 1's down
        projection and its residual join first (``q3_down_qkv_attn``)."""
        B, H, I, Hq, Hkv, C, s = (self.batch, self.HIDDEN, self.INTER, self.HEADS, self.KV_HEADS, self.capacity,
                                  self._s)
        layer_stride = self.cache_k[0].numel() * 2
        first, with_o = i == 0, self.qkv_attn_o
        resid = _ptr(self.resid)
        if self.down_attn and not first:
            call("q3_down_qkv_attn", _ptr(self.act), _ptr(self.layers[i - 1]["down"]), I, _ptr(self.rx), resid,
                 _ptr(L["in_ln"]), self.EPS, _ptr(L["qkv"]), H, _ptr(self.qkv_x), _ptr(L["q_norm"]),
                 _ptr(L["k_norm"]), _ptr(self.cos_table), _ptr(self.sin_table), _ptr(self.g_pos),
                 self.cache_k.data_ptr() + i * layer_stride, self.cache_v.data_ptr() + i * layer_stride,
                 _ptr(self.attn_x), _ptr(L["o"]), _ptr(self.o_x), _ptr(L["gate_up"]), 2 * I, self.gate_up_group,
                 Hq, Hkv, C, self.splits, i, self.SCALE, _ptr(self.attn_err), s)
            return
        call("q3_qkv_attn", _lib.X_EMBED_NORM if first else _lib.X_NORM, _ptr(self.embed) if first else resid,
             H, _ptr(self.g_token) if first else None, _ptr(L["in_ln"]), self.EPS,
             resid if first or with_o else None, _ptr(L["qkv"]), H, _ptr(self.qkv_x), _ptr(L["q_norm"]),
             _ptr(L["k_norm"]), _ptr(self.cos_table), _ptr(self.sin_table), _ptr(self.g_pos),
             self.cache_k.data_ptr() + i * layer_stride, self.cache_v.data_ptr() + i * layer_stride,
             _ptr(self.attn_x), None if with_o else _ptr(self.attn_out), _ptr(L["o"]) if with_o else None,
             _ptr(self.o_x) if with_o else None, _ptr(L["gate_up"]) if with_o else None, 2 * I,
             self.gate_up_group, B, Hq, Hkv, C, self.splits, i, self.SCALE, _ptr(self.attn_err), s)

    def _attention(self, i: int, L: dict, src: tuple, kc: int, vc: int) -> None:
        """Layer i's decode attention into attn_out: q/k norm + RoPE + KV append,
        split-K GQA and the split merge (one launch when ``attn_fused``: merging
        workgroups, or two splits of which the first merges, ``attn_pair``).
        ``src`` is (qkv, ld, qkv partials, partial count)."""
        B, Hq, Hkv, C, s = self.batch, self.HEADS, self.KV_HEADS, self.capacity, self._s
        pos, attn = _ptr(self.g_pos), _ptr(self.attn_out)
        common = (_ptr(L["q_norm"]), _ptr(L["k_norm"]), _ptr(self.cos_table), _ptr(self.sin_table), pos, kc, vc)
        if self.attn_pair:
            call("q3_attn_decode_pair", *src, *common, _ptr(self.attn_x), attn, B, Hq, Hkv, C, i, self.EPS,
                 self.SCALE, _ptr(self.attn_err), s)
            return
        if self.attn_fused:
            call("q3_attn_decode_fused", *src, *common, _ptr(self.attn_x), attn, B, Hq, Hkv, C, self.splits, i,
                 self.EPS, self.SCALE, _ptr(self.attn_err), s)
            return
        # The partial buffers hold [B, Hq, splits] records; the launcher cannot see their size.
        records = B * Hq * self.splits
        if self.part_acc.numel() < records * self.HEAD_DIM or self.part_ml.numel() < records * 2:
            raise RuntimeError("attention partial buffers are smaller than the split count needs")
        call("q3_attn_decode", *src, *common, _ptr(self.part_acc), _ptr(self.part_ml),
             attn if self.splits == 1 else None, B, Hq, Hkv, C, self.splits, self.EPS, self.SCALE, s)
        if self.splits > 1:
            call("q3_attn_merge", _ptr(self.part_acc), _ptr(self.part_ml), attn, B, Hq, self.splits, s)

    def _proj(self, x: int, ldx: int, w: torch.Tensor, N: int, K: int, epi: int, y: int, ldy: int) -> None:
        """Decode projection for batches outside the GEMV and fused MFMA paths (more
        than 64 rows, or shapes that do not tile): the LDS-tiled MFMA GEMM."""
        call("q3_gemm", x, ldx, _ptr(w), self.batch, N, K, epi, y, ldy, self._s)

    def _capture(self) -> None:
        """Warm every kernel eagerly, then record one decode step as a hipGraph.

        Reference ``engine/engine.py:1029-1059``.  A failed capture raises: the
        engine has no eager decode mode to fall back to.
        """
        with torch.cuda.stream(self.stream):
            for _ in range(2):
                self.g_pos.fill_(max(0, self.capacity - 2))
                self.g_token.zero_()
                self._clear_exchange()
                self._enqueue_decode()
            self.g_pos.zero_()
            self.g_token.zero_()
        self.stream.synchronize()
        self._check_step()
        call("q3_graph_begin", self._s)
        try:
            self._enqueue_decode()
        except Exception:
            exec_ptr = ctypes.c_void_p()
            _lib.lib().q3_graph_end(self._s, ctypes.byref(exec_ptr))
            if exec_ptr.value:
                call("q3_graph_destroy", exec_ptr.value)
            raise
        exec_ptr = ctypes.c_void_p()
        call("q3_graph_end", self._s, ctypes.byref(exec_ptr))
        self.graph = exec_ptr.value
        _log(f"decode graph captured (batch={self.batch}, splits={self.splits})")

    def _clear_exchange(self) -> None:
        """Zero the fused launches' exchange words (attention partials, q|k|v
        rows, attention output) and timeout word on the decode stream.  Their flags are derived
        from (position, layer), so words left by an earlier call at the same
        positions would read as fresh."""
        self.attn_x.zero_()
        self.qkv_x.zero_()
        self.o_x.zero_()
        self.rx.zero_()
        self.attn_err.zero_()

    def _begin_decode(self, logits: torch.Tensor, seq_len: int) -> None:
        """First token = argmax of the prefill's last logits; positions restart
        at the prompt length (reference ``engine/engine.py:1077-1079``)."""
        with torch.cuda.stream(self.stream):
            call("q3_argmax_rows", _ptr(logits), self.VOCAB, self.batch, self.VOCAB, _ptr(self.g_token), None,
                 None, None, None, 0, self._s)
            self.g_pos.fill_(seq_len)
            self.g_feed.fill_(-1)  # self-feeding (a replay that raised may have left a stream)
            self._clear_exchange()

    def _decode_step(self) -> torch.Tensor:
        """Replay the captured step: g_token <- next token, g_pos += 1."""
        call("q3_graph_launch", self.graph, self._s)
        return self.g_token

    def _check_step(self) -> None:
        """Raise if the fused attention launch reported a merge wait past its
        time bound (``attn_err``), and drop the step's state so the next call
        rebuilds it."""
        if self.attn_fused and int(self.attn_err.cpu()[0]):
            self.graph_key_reset()
            raise RuntimeError("the fused attention launch did not complete: a workgroup waited for "
                               "another's words past its time bound")

    # -------------------------------------------------------------- prefill

    def _prefill_buffers(self, rows: int) -> dict:
        bufs = self._prefill_bufs.get(rows)
        if bufs is None:
            self._prefill_bufs = {}
            bufs = {
                "resid": self._empty(rows, self.HIDDEN),
                "n": self._empty(rows, self.HIDDEN),
                "qkv": self._empty(rows, self.qkv_size),
                "q": self._empty(rows, self.q_size),
                "a": self._empty(rows, self.q_size),
                "act": self._empty(rows, self.INTER),
            }
            self._prefill_bufs[rows] = bufs
        return bufs

    def _prefill_partials(self, floats: int) -> torch.Tensor:
        """FP32 split-K partials of the prompt pass's projections (the residual
        projections of 256-4095-token chunks, or the split tail tiles of
        q3_gemm_ws: at most 126 MB), grown on demand."""
        if self._prefill_part is None or self._prefill_part.numel() < floats:
            self._prefill_part = None
            self._prefill_part = self._empty(floats, dtype=torch.float32)
        return self._prefill_part

    def _forward_prefill(self, ids: torch.Tensor, seq_len: int) -> torch.Tensor:
        """Consume the prompt ``ids [B, P]``; return the last position's logits [B, 1, V].

        Reference ``engine/engine.py:738-803``: chunks of ``PREFILL_CHUNK_TOKENS
        // B`` tokens per sequence, causal within the chunk and over every
        earlier key; the cache is written for every prompt position.
        """
        B = ids.shape[0]
        if B != self.batch or seq_len > self.capacity or ids.shape[1] != seq_len:
            raise ValueError(f"prefill of {tuple(ids.shape)} does not fit the cache "
                             f"(batch {self.batch}, capacity {self.capacity})")
        if int(ids.min()) < 0 or int(ids.max()) >= self.VOCAB:
            raise ValueError(f"token ids must lie in [0, {self.VOCAB})")
        if ids.is_cuda:
            # Made on the caller's stream, read on ours: keep the block alive until
            # our stream is done with it.
            self.stream.wait_stream(torch.cuda.current_stream())
            ids.record_stream(self.stream)
        chunk = seq_len
        if B * seq_len > PREFILL_CHUNK_TOKENS:
            chunk = max(1, PREFILL_CHUNK_TOKENS // B)
        H, I, D, Hq, Hkv, C = self.HIDDEN, self.INTER, self.HEAD_DIM, self.HEADS, self.KV_HEADS, self.capacity
        layer_stride = self.cache_k[0].numel() * 2
        kc0, vc0 = self.cache_k.data_ptr(), self.cache_v.data_ptr()
        s = self._s
        with torch.cuda.stream(self.stream):
            ids = ids.to(self.device, torch.int64)
            for start in range(0, seq_len, chunk):
                stop = min(start + chunk, seq_len)
                T = stop - start
                M = B * T
                bufs = self._prefill_buffers(B * min(chunk, seq_len))
                chunk_ids = ids[:, start:stop].contiguous()
                resid, n, qkv, q, a, act = (_ptr(bufs[k]) for k in ("resid", "n", "qkv", "q", "a", "act"))
                # Prompts too short to fill the CUs with whole 256 x 256 tiles split the
                # residual projections along K; their partials are summed (in split
                # order), joined to the residual and normalised by one row kernel,
                # which replaces the RMSNorm that follows each of them.
                s_o = call("q3_gemm_splits", M, H, self.q_size)
                s_d = call("q3_gemm_splits", M, H, I)
                # Longer prompts whose last round of tiles is at most half full split
                # those tiles along K (q3_gemm_ws); the same buffer holds either.
                floats = max(s_o, s_d) * M * H
                for n_, k_ in ((self.qkv_size, H), (2 * I, H), (H, self.q_size), (H, I)):
                    floats = max(floats, call("q3_gemm_ws_floats", M, n_, k_))
                part = _ptr(self._prefill_partials(floats)) if floats else None
                for i, L in enumerate(self.layers):
                    if i == 0:
                        call("q3_embed_rmsnorm", _ptr(chunk_ids), _ptr(self.embed), resid, n,
                             _ptr(L["in_ln"]), M, H, self.EPS, s)
                    elif not s_d:  # else the previous layer's down reduction normalised it
                        call("q3_rmsnorm", resid, H, _ptr(L["in_ln"]), n, H, M, H, self.EPS, s)
                    call("q3_gemm_ws", n, H, _ptr(L["qkv"]), M, self.qkv_size, H, _lib.EPI_STORE, qkv,
                         self.qkv_size, part, s)
                    call("q3_qk_norm_rope_kv", qkv, self.qkv_size, _ptr(L["q_norm"]), _ptr(L["k_norm"]),
                         _ptr(self.cos_table), _ptr(self.sin_table), None, start, q,
                         kc0 + i * layer_stride, vc0 + i * layer_stride, B, T, Hq, Hkv, D, C, self.EPS, s)
                    call("q3_attn_prefill", q, kc0 + i * layer_stride, vc0 + i * layer_stride, a, B, T,
                         start, Hq, Hkv, C, self.SCALE, s)
                    # Residual join and SwiGLU in the GEMM epilogues, at the reference's
                    # rounding points: resid = bf16(resid + bf16(acc)); act = bf16(bf16(silu(g)) * u).
                    if s_o:
                        call("q3_gemm_partials", a, self.q_size, _ptr(L["o"]), M, H, self.q_size, part, s_o, s)
                        call("q3_add_rmsnorm_partials", part, s_o, resid, _ptr(L["post_ln"]), n, M, H,
                             self.EPS, s)
                    else:
                        call("q3_gemm_ws", a, self.q_size, _ptr(L["o"]), M, H, self.q_size, _lib.EPI_RESID,
                             resid, H, part, s)
                        call("q3_rmsnorm", resid, H, _ptr(L["post_ln"]), n, H, M, H, self.EPS, s)
                    call("q3_gemm_ws", n, H, _ptr(L["gate_up"]), M, 2 * I, H, _lib.EPI_SWIGLU, act, I, part, s)
                    if s_d:
                        # The last layer's norm output is not used: the LM head
                        # normalises the last positions of resid itself.
                        nxt = self.layers[i + 1]["in_ln"] if i + 1 < len(self.layers) else self.final_norm
                        call("q3_gemm_partials", act, I, _ptr(L["down"]), M, H, I, part, s_d, s)
                        call("q3_add_rmsnorm_partials", part, s_d, resid, _ptr(nxt), n, M, H, self.EPS, s)
                    else:
                        call("q3_gemm_ws", act, I, _ptr(L["down"]), M, H, I, _lib.EPI_RESID, resid, H, part, s)
                last = bufs["resid"][(T - 1):]  # row T-1 of sequence 0; sequences are T rows apart
            # The final norm is applied on the last position only, then the tied LM head
            # (reference :800-803: the last layer's closing norm uses final_norm_w).
            logits = self._empty(B, self.VOCAB)
            if B <= _lib.GEMV_MAX_M:
                call("q3_gemv", _lib.X_NORM, _ptr(last), T * H, None, _ptr(self.final_norm), self.EPS, None,
                     _ptr(self.lm_head), B, self.VOCAB, H, _lib.EPI_STORE, _ptr(logits), self.VOCAB,
                     None, None, None, None, None, 0, s)
            else:
                n_last = self._empty(B, H)
                call("q3_rmsnorm", _ptr(last), T * H, _ptr(self.final_norm), _ptr(n_last), H, B, H,
                     self.EPS, s)
                call("q3_gemm", _ptr(n_last), H, _ptr(self.lm_head), B, self.VOCAB, H, _lib.EPI_STORE,
                     _ptr(logits), self.VOCAB, s)
        # The caller reads the logits on its own stream (reference
        # tests/test_equivalence.py:161-166 uses them at once): order its stream
        # after ours, and keep the block alive until the caller's stream is done.
        caller = torch.cuda.current_stream(self.device)
        caller.wait_stream(self.stream)
        logits.record_stream(caller)
        return logits.view(B, 1, self.VOCAB)

    # ------------------------------------------------------------- generate

    @torch.inference_mode()
    def generate(self, input_ids: list[list[int]], max_new_tokens: int):
        """Greedy continuation; yields ``max_new_tokens`` lists of one id per sequence.

        Reference ``engine/engine.py:1069-1105``: prefill, argmax, then one graph
        replay per further token with one step of device-to-host lookahead.
        """
        if max_new_tokens <= 0:
            return
        ids = _check_ids(input_ids, self.VOCAB)
        batch, seq_len = ids.shape
        self._ensure_shape(batch, seq_len, max_new_tokens)

        # No state carries between calls: positions restart at the prompt length,
        # and only slots below the running position are ever read.
        logits = self._forward_prefill(ids, seq_len)
        self._begin_decode(logits, seq_len)
        host = torch.empty(batch, dtype=torch.int64, pin_memory=True)
        host_err = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        done = torch.cuda.Event()
        pending = False
        for step in range(max_new_tokens):
            if not pending:
                self.stream.synchronize()
                out = self.g_token.cpu()
            else:
                done.synchronize()
                out = host.clone()
                if self.attn_fused and int(host_err[0]):
                    self._check_step()  # raises
            toks = out.tolist()
            if step + 1 < max_new_tokens:
                self._decode_step()
                with torch.cuda.stream(self.stream):
                    host.copy_(self.g_token, non_blocking=True)
                    host_err.copy_(self.attn_err, non_blocking=True)
                    done.record(self.stream)
                pending = True
            else:
                pending = False
            yield toks

    # ------------------------------------------------------ replay judge

    def _stream_tensor(self, rows, batch: int, name: str) -> torch.Tensor:
        t = torch.tensor(rows, dtype=torch.int64)
        if t.dim() != 2 or t.shape[1] != batch:
            raise ValueError(f"{name} must be a list of lists of {batch} ids")
        if t.numel() and (int(t.min()) < 0 or int(t.max()) >= self.VOCAB):
            raise ValueError(f"{name} ids must lie in [0, {self.VOCAB})")
        return t

    def _feed_stream(self, seq_len: int, tokens: torch.Tensor) -> None:
        """Feed ``tokens[k]`` at position ``seq_len + k`` (k >= 1) through the step
        records' feed table; ``tokens[0]`` is written as the first input."""
        with torch.cuda.stream(self.stream):
            self.g_feed.fill_(-1)
            if len(tokens) > 1:
                self.g_feed[seq_len + 1:seq_len + len(tokens)].copy_(tokens[1:])
            self.g_token.copy_(tokens[0])
            self.g_rec.zero_()

    def _records_of(self, seq_len: int, n: int) -> np.ndarray:
        """Step records [n, B, 4] of positions seq_len+1 .. seq_len+n (int32 words)."""
        self.stream.synchronize()
        return self.g_rec[seq_len + 1:seq_len + 1 + n].cpu().numpy()

    @torch.inference_mode()
    def replay(self, input_ids: list[list[int]], emitted: list[list[int]]) -> dict:
        """Teacher-forced replay of an emitted token stream through the captured decode step.

        Not part of the reference API.  The contest judge replays a stream this
        way (reference ``QWEN_ENGINE_CONTRACT.md`` "The quality rule"):
        ``emitted[k]`` (B ids) is checked against the logits computed from the
        prompt plus ``emitted[:k]``.  Step 0 is judged on the prompt pass's
        logits; every later step runs the production decode graph, fed from the
        step records' feed table, with no host copy or sync per step.  Returns
        numpy arrays [N, B]: ``argmax``, ``top`` (its BF16 logit) and ``logit``
        (the emitted token's BF16 logit).
        """
        ids = _check_ids(input_ids, self.VOCAB)
        batch, seq_len = ids.shape
        em = self._stream_tensor(emitted, batch, "emitted")
        n = em.shape[0]
        if n == 0:
            empty = np.zeros((0, batch))
            return {"argmax": empty.astype(np.int64), "top": empty, "logit": empty}
        self._ensure_shape(batch, seq_len, n)
        logits = self._forward_prefill(ids, seq_len).view(batch, self.VOCAB).float().cpu()
        top, arg = logits.max(dim=-1)
        first = {"argmax": logits.argmax(dim=-1).numpy(), "top": top.numpy(),
                 "logit": logits.gather(1, em[0].view(batch, 1))[:, 0].numpy()}
        self._feed_stream(seq_len, em.to(self.device))
        with torch.cuda.stream(self.stream):
            self.g_pos.fill_(seq_len)
            self._clear_exchange()
        for _ in range(n - 1):
            self._decode_step()
        rec = self._records_of(seq_len, n - 1)
        self._check_step()
        with torch.cuda.stream(self.stream):
            self.g_feed.fill_(-1)
        out = {
            "argmax": np.concatenate([first["argmax"][None], rec[..., 0].astype(np.int64)]),
            "top": np.concatenate([first["top"][None], rec[..., 1].view(np.float32)]),
            "logit": np.concatenate([first["logit"][None], rec[..., 2].view(np.float32)]),
        }
        if not np.array_equal(rec[..., 3], em[1:].numpy()):
            raise RuntimeError("replay fed a different stream than the one given")
        return out

    def replay_check(self, input_ids: list[list[int]], emitted: list[list[int]],
                     margin: float = TIE_MARGIN_LOGITS) -> list[tuple[int, int, float]]:
        """The contest's quality rule on this engine's own replay: every emitted
        token is the argmax of the replayed logits or within ``margin`` of the
        maximum (reference ``QWEN_ENGINE_CONTRACT.md`` "The quality rule",
        ``tieMarginLogits`` 2.0).  Returns the failing (step, row, shortfall)."""
        r = self.replay(input_ids, emitted)
        em = np.asarray(emitted, dtype=np.int64).reshape(r["argmax"].shape)
        short = r["top"] - r["logit"]
        bad = np.nonzero((em != r["argmax"]) & (short > margin))
        return [(int(k), int(b), float(short[k, b])) for k, b in zip(*bad)]

    # -------------------------------------------------------- diagnostics

    def prepare_trace(self, batch: int, seq_len: int, new_tokens: int) -> None:
        """Build the (batch, seq_len + new_tokens) step with the logits stored
        every step (the LM head's EPI_STORE_ARGMAX epilogue; every other kernel
        is the production one).  A diagnostic: ``trace_decode`` then reads the
        logits step by step; ``end_trace`` returns to the production graph."""
        self.keep_logits = True
        self.graph_key_reset()
        self._ensure_shape(batch, seq_len, new_tokens)

    def end_trace(self) -> None:
        self.keep_logits = False
        self.graph_key_reset()

    @torch.inference_mode()
    def trace_decode(self, first: list[int], seq_len: int, steps: int,
                     forced: list[list[int]] | None = None):
        """``steps`` decode steps from the cache as it stands (positions below
        ``seq_len`` already written, e.g. by the caller), the first fed
        ``first`` (B ids) at ``seq_len``.  With ``forced``, the step at
        ``seq_len + k`` (k >= 1) is fed ``forced[k - 1]`` through the feed table
        instead of the engine's choice.  Returns (the engine's choices
        [steps][B], logits [steps, B, V] on the CPU)."""
        if not self.keep_logits:
            raise RuntimeError("trace_decode needs prepare_trace first")
        B = self.batch
        feed = [first] + (list(forced[:steps - 1]) if forced is not None else [])
        self._feed_stream(seq_len, self._stream_tensor(feed, B, "forced").to(self.device))
        with torch.cuda.stream(self.stream):
            self.g_pos.fill_(seq_len)
            self._clear_exchange()
        kept = []
        for _ in range(steps):
            self._decode_step()
            self.stream.synchronize()
            kept.append(self.logits.cpu())
        rec = self._records_of(seq_len, steps)
        self._check_step()
        with torch.cuda.stream(self.stream):
            self.g_feed.fill_(-1)
        return rec[..., 0].astype(np.int64).tolist(), torch.stack(kept)

    @torch.inference_mode()
    def trace_logits(self, input_ids: list[list[int]], max_new_tokens: int,
                     forced: list[list[int]] | None = None):
        """Tokens plus the BF16 logits each step's ids were chosen from.

        Not part of the reference API: parity tests use it to compare per-step
        logits with the CPU oracle.  With ``forced`` (one list of B ids per
        step), step i+1 is fed ``forced[i]`` instead of the engine's own choice
        (teacher forcing, as the contest's judge replays a stream).  Returns
        (the engine's choices [N][B], logits [N, B, V] on the CPU).
        """
        ids = _check_ids(input_ids, self.VOCAB)
        batch, seq_len = ids.shape
        self.prepare_trace(batch, seq_len, max_new_tokens)
        try:
            logits = self._forward_prefill(ids, seq_len)
            first = logits.view(batch, -1).cpu()
            steps = [first.float().argmax(dim=-1).tolist()]
            if max_new_tokens > 1:
                feed = forced[0] if forced is not None else steps[0]
                more, kept = self.trace_decode(feed, seq_len, max_new_tokens - 1,
                                               forced[1:] if forced is not None else None)
                steps += more
                return steps, torch.cat([first[None], kept])
            return steps, first[None]
        finally:
            self.end_trace()

    def graph_key_reset(self) -> None:
        """Force the next ``_ensure_shape`` to rebuild (e.g. after toggling keep_logits)."""
        self._release_graph()
        self.batch = self.capacity = 0

