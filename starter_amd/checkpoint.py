"""Hugging Face Qwen3 checkpoint directories: a reader, and a seeded writer.

The engine takes ``model_path``, a local HF checkpoint directory
(``config.json`` + ``model.safetensors``, or shards listed in
``model.safetensors.index.json``), exactly as the reference's ``Engine``
does (reference ``engine/engine.py:124-133``, ``QWEN_ENGINE_CONTRACT.md``
"model_path is a directory holding the checkpoint exactly as published").
The reference loads it through ``transformers.AutoModelForCausalLM``; this
module reads the safetensors container directly (8-byte little-endian header
length, JSON header, raw little-endian tensor bytes) so the engine carries no
dependency on transformers, and memory-maps it so an 8 GB checkpoint is never
copied on the host.

Tensor names follow HF's Qwen3 layout: ``model.embed_tokens.weight``,
``model.layers.{i}.{input_layernorm,post_attention_layernorm}.weight``,
``model.layers.{i}.self_attn.{q,k,v,o}_proj.weight``,
``model.layers.{i}.self_attn.{q,k}_norm.weight``,
``model.layers.{i}.mlp.{gate,up,down}_proj.weight``, ``model.norm.weight``;
``lm_head.weight`` is absent when the embedding is tied.

The writer produces the benchmark's seeded random-init model: every matrix
N(0, 0.02) in BF16 from a counter-based stream (the C routine in
``csrc/seeded_init.c`` defines it), every norm gain 1.0.
"""

from __future__ import annotations

import ctypes
import dataclasses
import hashlib
import json
import os
import pathlib
from concurrent.futures import ThreadPoolExecutor

import numpy as np

BF16_ONE = 0x3F80

_DTYPES = {
    "BF16": (np.uint16, 2),
    "F16": (np.float16, 2),
    "F32": (np.float32, 4),
    "I64": (np.int64, 8),
}


@dataclasses.dataclass(frozen=True)
class Qwen3Config:
    """The dimensions the engine reads from ``config.json``.

    Mirrors the fields the reference reads at ``engine/engine.py:139-147``.
    """

    num_hidden_layers: int = 36
    hidden_size: int = 2560
    intermediate_size: int = 9728
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    head_dim: int = 128
    vocab_size: int = 151936
    rms_norm_eps: float = 1e-6
    rope_theta: float = 5_000_000.0
    tie_word_embeddings: bool = True
    max_position_embeddings: int = 262144

    @classmethod
    def from_json(cls, path: str | os.PathLike) -> "Qwen3Config":
        raw = json.loads(pathlib.Path(path).read_text())
        theta = raw.get("rope_theta")
        if theta is None:
            theta = (raw.get("rope_parameters") or {}).get("rope_theta")
        if theta is None:
            raise ValueError(f"{path}: no rope_theta")
        heads = raw["num_attention_heads"]
        return cls(
            num_hidden_layers=raw["num_hidden_layers"],
            hidden_size=raw["hidden_size"],
            intermediate_size=raw["intermediate_size"],
            num_attention_heads=heads,
            num_key_value_heads=raw.get("num_key_value_heads", heads),
            head_dim=raw.get("head_dim") or raw["hidden_size"] // heads,
            vocab_size=raw["vocab_size"],
            rms_norm_eps=raw.get("rms_norm_eps", 1e-6),
            rope_theta=float(theta),
            tie_word_embeddings=raw.get("tie_word_embeddings", True),
            max_position_embeddings=raw.get("max_position_embeddings", 262144),
        )

    def to_hf_json(self) -> dict:
        return {
            "architectures": ["Qwen3ForCausalLM"],
            "model_type": "qwen3",
            "hidden_size": self.hidden_size,
            "intermediate_size": self.intermediate_size,
            "num_hidden_layers": self.num_hidden_layers,
            "num_attention_heads": self.num_attention_heads,
            "num_key_value_heads": self.num_key_value_heads,
            "head_dim": self.head_dim,
            "vocab_size": self.vocab_size,
            "max_position_embeddings": self.max_position_embeddings,
            "rms_norm_eps": self.rms_norm_eps,
            "rope_theta": self.rope_theta,
            "rope_scaling": None,
            "tie_word_embeddings": self.tie_word_embeddings,
            "hidden_act": "silu",
            "attention_bias": False,
            "attention_dropout": 0.0,
            "use_sliding_window": False,
            "sliding_window": None,
            "max_window_layers": self.num_hidden_layers,
            "torch_dtype": "bfloat16",
            "bos_token_id": 151643 if self.vocab_size > 151645 else None,
            "eos_token_id": 151645 if self.vocab_size > 151645 else None,
        }


QWEN3_4B = Qwen3Config()


def tensor_specs(cfg: Qwen3Config) -> list[tuple[str, tuple[int, ...], str]]:
    """(name, shape, kind) in HF ``state_dict`` order; kind is "normal" or "ones"."""
    H, I, D = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
    q, kv = cfg.num_attention_heads * D, cfg.num_key_value_heads * D
    specs = [("model.embed_tokens.weight", (cfg.vocab_size, H), "normal")]
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}."
        specs += [
            (p + "self_attn.q_proj.weight", (q, H), "normal"),
            (p + "self_attn.k_proj.weight", (kv, H), "normal"),
            (p + "self_attn.v_proj.weight", (kv, H), "normal"),
            (p + "self_attn.o_proj.weight", (H, q), "normal"),
            (p + "self_attn.q_norm.weight", (D,), "ones"),
            (p + "self_attn.k_norm.weight", (D,), "ones"),
            (p + "mlp.gate_proj.weight", (I, H), "normal"),
            (p + "mlp.up_proj.weight", (I, H), "normal"),
            (p + "mlp.down_proj.weight", (H, I), "normal"),
            (p + "input_layernorm.weight", (H,), "ones"),
            (p + "post_attention_layernorm.weight", (H,), "ones"),
        ]
    specs.append(("model.norm.weight", (H,), "ones"))
    if not cfg.tie_word_embeddings:
        specs.append(("lm_head.weight", (cfg.vocab_size, H), "normal"))
    return specs


# ----------------------------------------------------------------- C helper


_SEED_LIB = None


def _seed_lib() -> ctypes.CDLL:
    global _SEED_LIB
    if _SEED_LIB is None:
        path = pathlib.Path(__file__).resolve().parent / "_lib" / "libq3seed.so"
        if not path.exists():
            raise ImportError(
                f"{path} is missing: run `python -m starter_amd.build` (or "
                "__graft_entry__.build()) first"
            )
        lib = ctypes.CDLL(str(path))
        lib.q3seed_stream.restype = ctypes.c_uint64
        lib.q3seed_stream.argtypes = [ctypes.c_uint64, ctypes.c_char_p]
        lib.q3seed_fill_normal_bf16.restype = None
        lib.q3seed_fill_normal_bf16.argtypes = [
            ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_double, ctypes.c_double]
        lib.q3seed_fill_const_bf16.restype = None
        lib.q3seed_fill_const_bf16.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint16]
        lib.q3seed_prompt_ids.restype = None
        lib.q3seed_prompt_ids.argtypes = [
            ctypes.c_uint64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64]
        _SEED_LIB = lib
    return _SEED_LIB


def seeded_tensor(name: str, shape: tuple[int, ...], kind: str, seed: int = 0,
                  std: float = 0.02, gain_std: float = 0.0,
                  out: np.ndarray | None = None) -> np.ndarray:
    """One tensor of the seeded model as raw BF16 bits (``np.uint16``).

    Matrices are N(0, std).  Norm gains ("ones") are exactly 1.0, or
    1 + N(0, gain_std) when ``gain_std`` > 0 (test models use that so the
    gain multiply is exercised).
    """
    n = int(np.prod(shape))
    if out is None:
        out = np.empty(shape, dtype=np.uint16)
    assert out.dtype == np.uint16 and out.size == n and out.flags.c_contiguous
    lib = _seed_lib()
    stream = lib.q3seed_stream(seed, name.encode())
    if kind == "ones" and gain_std <= 0:
        lib.q3seed_fill_const_bf16(out.ctypes.data, n, BF16_ONE)
    elif kind == "ones":
        lib.q3seed_fill_normal_bf16(stream, out.ctypes.data, n, 1.0, gain_std)
    else:
        lib.q3seed_fill_normal_bf16(stream, out.ctypes.data, n, 0.0, std)
    return out


def seeded_prompt(seed: int, batch: int, length: int, vocab: int = 151643) -> list[list[int]]:
    """Uniform ids in [0, vocab), an independent stream per row."""
    lib = _seed_lib()
    rows = []
    for r in range(batch):
        buf = np.empty(length, dtype=np.int64)
        lib.q3seed_prompt_ids(seed, r, buf.ctypes.data, length, vocab)
        rows.append(buf.tolist())
    return rows


# ------------------------------------------------------------------ writer


def _header_bytes(entries: dict) -> bytes:
    header = json.dumps(entries, separators=(",", ":")).encode()
    header += b" " * ((-len(header)) % 8)
    return len(header).to_bytes(8, "little") + header


def write_seeded_checkpoint(path: str | os.PathLike, cfg: Qwen3Config = QWEN3_4B,
                            seed: int = 0, std: float = 0.02,
                            gain_std: float = 0.0) -> dict[str, str]:
    """Write ``config.json`` + ``model.safetensors`` for the seeded model.

    Returns the per-tensor SHA-256 manifest (also written as
    ``seeded_manifest.json``).  Tensors are generated and written one at a
    time, so host memory peaks at one tensor.
    """
    path = pathlib.Path(path)
    path.mkdir(parents=True, exist_ok=True)
    specs = tensor_specs(cfg)
    entries = {"__metadata__": {"format": "pt", "seed": str(seed), "std": repr(std),
                                "gain_std": repr(gain_std)}}
    offset = 0
    for name, shape, _ in specs:
        nbytes = int(np.prod(shape)) * 2
        entries[name] = {"dtype": "BF16", "shape": list(shape),
                         "data_offsets": [offset, offset + nbytes]}
        offset += nbytes
    manifest = {}
    tmp = path / "model.safetensors.partial"
    with open(tmp, "wb") as f:
        f.write(_header_bytes(entries))
        for name, shape, kind in specs:
            t = seeded_tensor(name, shape, kind, seed, std, gain_std)
            manifest[name] = hashlib.sha256(t.data).hexdigest()
            f.write(t.data)
            del t
    os.replace(tmp, path / "model.safetensors")
    (path / "config.json").write_text(json.dumps(cfg.to_hf_json(), indent=2))
    (path / "seeded_manifest.json").write_text(
        json.dumps({"seed": seed, "std": std, "gain_std": gain_std, "sha256": manifest},
                   indent=1))
    return manifest


def ensure_seeded_checkpoint(path: str | os.PathLike, cfg: Qwen3Config = QWEN3_4B,
                             seed: int = 0, std: float = 0.02,
                             gain_std: float = 0.0) -> pathlib.Path:
    """Write the seeded checkpoint unless an identical one is already there."""
    path = pathlib.Path(path)
    want = cfg.to_hf_json()
    try:
        have = json.loads((path / "config.json").read_text())
        meta = json.loads((path / "seeded_manifest.json").read_text())
        size = (path / "model.safetensors").stat().st_size
        expect = sum(int(np.prod(s)) * 2 for _, s, _ in tensor_specs(cfg))
        if (have == want and meta.get("seed") == seed and meta.get("std") == std
                and meta.get("gain_std") == gain_std and size > expect):
            return path
    except (OSError, ValueError):
        pass
    write_seeded_checkpoint(path, cfg, seed, std, gain_std)
    return path


def manifest_of(weights: dict[str, np.ndarray], threads: int = 8) -> dict[str, str]:
    """SHA-256 of each tensor's raw bytes (hashlib releases the GIL)."""
    names = sorted(weights)
    with ThreadPoolExecutor(threads) as pool:
        digests = pool.map(lambda n: hashlib.sha256(
            np.ascontiguousarray(weights[n]).data).hexdigest(), names)
        return dict(zip(names, digests))


# ------------------------------------------------------------------ reader


def _read_safetensors(file: pathlib.Path) -> dict[str, tuple[np.ndarray, str]]:
    with open(file, "rb") as f:
        n = int.from_bytes(f.read(8), "little")
        header = json.loads(f.read(n))
    base = 8 + n
    mm = np.memmap(file, dtype=np.uint8, mode="r")
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        dtype = meta["dtype"]
        if dtype not in _DTYPES:
            raise ValueError(f"{file}: tensor {name} has unsupported dtype {dtype}")
        np_dtype, size = _DTYPES[dtype]
        start, end = meta["data_offsets"]
        shape = tuple(meta["shape"])
        if end - start != int(np.prod(shape)) * size:
            raise ValueError(f"{file}: tensor {name} byte range does not match its shape")
        arr = mm[base + start: base + end].view(np_dtype).reshape(shape)
        out[name] = (arr, dtype)
    return out


def _to_bf16_bits(arr: np.ndarray, dtype: str) -> np.ndarray:
    """Raw BF16 bits; F32/F16 checkpoints are rounded to nearest even, and a
    NaN stays a NaN (0x7FC0; rounding its bits could carry into infinity)."""
    if dtype == "BF16":
        return arr
    f = np.ascontiguousarray(arr, dtype=np.float32).view(np.uint32)
    rounded = ((f.astype(np.uint64) + 0x7FFF + ((f >> 16) & 1)) >> 16).astype(np.uint16)
    rounded[(f & 0x7FFFFFFF) > 0x7F800000] = 0x7FC0
    return rounded


def load_checkpoint(path: str | os.PathLike) -> tuple[Qwen3Config, dict[str, np.ndarray]]:
    """Config plus every tensor as BF16 bits (memory-mapped where already BF16)."""
    path = pathlib.Path(path)
    if not path.is_dir():
        raise FileNotFoundError(f"model_path {path} is not a directory")
    cfg = Qwen3Config.from_json(path / "config.json")
    index = path / "model.safetensors.index.json"
    if index.exists():
        files = sorted(set(json.loads(index.read_text())["weight_map"].values()))
    else:
        files = ["model.safetensors"]
    tensors = {}
    for name in files:
        for key, (arr, dtype) in _read_safetensors(path / name).items():
            tensors[key] = _to_bf16_bits(arr, dtype)
    missing = [n for n, _, _ in tensor_specs(cfg) if n not in tensors]
    if missing:
        raise KeyError(f"{path}: checkpoint lacks {missing[:4]}{'...' if len(missing) > 4 else ''}")
    for name, shape, _ in tensor_specs(cfg):
        if tuple(tensors[name].shape) != shape:
            raise ValueError(f"{path}: {name} has shape {tensors[name].shape}, want {shape}")
    return cfg, tensors
