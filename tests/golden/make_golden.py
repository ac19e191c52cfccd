"""Write the golden fixtures under tests/golden/ from HF's Qwen3 (CPU).

The reference's correctness oracle is "native Qwen": transformers'
``Qwen3ForCausalLM`` driven by the baseline greedy loop of reference
``tests/test_equivalence.py:72-86`` (``model(input_ids, past_key_values,
use_cache=True, logits_to_keep=1)``, argmax, feed back).  transformers is a
third-party dependency, not part of the reference tree (pinned 4.51.3 in
reference ``requirements.txt:11``; the installed 5.15.0 is what runs here).
This script runs it on seeded checkpoints written by
``starter_amd.checkpoint`` and stores token streams and logits as small
``.npz`` files (no pickles), with the library versions in ``golden_meta.json``.

Fixtures:
  tiny_{fp32,bf16}.npz  -- a 3-layer model with the reference test's geometry
                           (hidden 320, 8 q-heads over 2 kv-heads, head_dim
                           128, vocab 512; reference ``tests/test_equivalence.py:33-61``)
                           on the reference test's cases (``:208-220``).
  config1_bf16.npz      -- the full seeded Qwen3-4B at BASELINE config 1
                           (B=1, P=32, 32 new tokens), BF16 on CPU.
  config2_bf16.npz      -- the same model at BASELINE config 2 (B=1, P=1024,
                           512 new tokens): per step the token, the top-16
                           (id, logit) pairs, the top-2 gap and the logits at
                           a fixed 512-id subset; full logits at the first and
                           last steps.

Run (in this container only; it needs transformers):
    python tests/golden/make_golden.py [--skip-tiny] [--skip-full] [--skip-config2]
"""

from __future__ import annotations

import argparse
import json
import pathlib
import sys
import tempfile
import time

import numpy as np
import torch

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from starter_amd.checkpoint import Qwen3Config, write_seeded_checkpoint  # noqa: E402
from starter_amd.workloads import MODEL, MODEL_SEED, WORKLOADS  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent

TINY = Qwen3Config(num_hidden_layers=3, hidden_size=320, intermediate_size=640,
                   num_attention_heads=8, num_key_value_heads=2, head_dim=128,
                   vocab_size=512, max_position_embeddings=2048)
TINY_SEED, TINY_STD, TINY_GAIN_STD = 7, 0.05, 0.1

#: (name, batch, prompt, new, chunk tokens or 0) -- reference tests/test_equivalence.py:208-220
TINY_CASES = [
    ("batch1", 1, 16, 6, 0),
    ("batch4_gqa", 4, 20, 5, 0),
    ("batch3_long", 3, 64, 8, 0),
    ("single_token", 2, 12, 1, 0),
    ("chunked", 2, 48, 6, 32),
    ("chunked_tail", 3, 50, 4, 36),
    ("drift", 2, 32, 24, 0),
]


def tiny_prompt(case_index: int, batch: int, length: int) -> np.ndarray:
    g = np.random.Generator(np.random.PCG64(1000 + case_index))
    return g.integers(0, TINY.vocab_size, size=(batch, length), dtype=np.int64)


@torch.inference_mode()
def baseline_loop(model, ids: np.ndarray, new: int):
    """reference tests/test_equivalence.py:72-86, keeping each step's logits."""
    current = torch.from_numpy(ids)
    cache = None
    tokens, logits = [], []
    for _ in range(new):
        out = model(input_ids=current, past_key_values=cache, use_cache=True,
                    logits_to_keep=1, return_dict=True)
        step_logits = out.logits[:, -1, :]
        current = step_logits.argmax(dim=-1, keepdim=True)
        cache = out.past_key_values
        tokens.append(current[:, 0].numpy().copy())
        logits.append(step_logits.float().numpy().copy())
    return np.stack(tokens), np.stack(logits)


def load_hf(path, dtype):
    from transformers import AutoModelForCausalLM
    return AutoModelForCausalLM.from_pretrained(
        str(path), dtype=dtype, attn_implementation="sdpa", local_files_only=True).eval()


def make_tiny(tmp: pathlib.Path) -> None:
    path = tmp / "tiny"
    write_seeded_checkpoint(path, TINY, TINY_SEED, TINY_STD, TINY_GAIN_STD)
    for tag, dtype in (("fp32", torch.float32), ("bf16", torch.bfloat16)):
        model = load_hf(path, dtype)
        arrays = {}
        for i, (name, b, p, n, _) in enumerate(TINY_CASES):
            ids = tiny_prompt(i, b, p)
            tok, lg = baseline_loop(model, ids, n)
            arrays[f"{name}/ids"] = ids
            arrays[f"{name}/tokens"] = tok
            arrays[f"{name}/logits"] = lg.astype(np.float32)
        # reference tests/test_equivalence.py:120-142 (reset) and :174-197 (shape reuse):
        # the second call's expected stream is just the baseline on the second prompt.
        g = np.random.Generator(np.random.PCG64(77))
        arrays["reset/first"] = g.integers(0, TINY.vocab_size, (2, 24), dtype=np.int64)
        arrays["reset/second"] = g.integers(0, TINY.vocab_size, (2, 24), dtype=np.int64)
        arrays["reset/tokens"], arrays["reset/logits"] = baseline_loop(model, arrays["reset/second"], 5)
        arrays["reuse/first"] = g.integers(0, TINY.vocab_size, (2, 30), dtype=np.int64)
        arrays["reuse/second"] = g.integers(0, TINY.vocab_size, (2, 26), dtype=np.int64)
        arrays["reuse/tokens"], arrays["reuse/logits"] = baseline_loop(model, arrays["reuse/second"], 10)
        # reference tests/test_equivalence.py:145-171: prefill logits of a 2x40 prompt.
        arrays["prefill/ids"] = g.integers(0, TINY.vocab_size, (2, 40), dtype=np.int64)
        with torch.inference_mode():
            out = model(input_ids=torch.from_numpy(arrays["prefill/ids"]), use_cache=True,
                        logits_to_keep=1, return_dict=True)
        arrays["prefill/logits"] = out.logits[:, -1, :].float().numpy()
        np.savez_compressed(OUT / f"tiny_{tag}.npz", **arrays)
        print(f"wrote tiny_{tag}.npz", flush=True)
        del model


def full_model(tmp: pathlib.Path):
    path = tmp / "qwen3_4b_seeded"
    if not (path / "model.safetensors").exists():
        t0 = time.time()
        write_seeded_checkpoint(path, MODEL, MODEL_SEED)
        print(f"seeded checkpoint written in {time.time() - t0:.1f}s", flush=True)
    return path, load_hf(path, torch.bfloat16)


def step_summary(lg: np.ndarray, subset_size: int, subset_seed: int) -> dict:
    """Per-step fixture arrays of a batch-1 stream's logits [steps, V]."""
    top = np.argsort(-lg, axis=-1, kind="stable")[:, :16]
    srt = np.sort(lg, axis=-1)
    g = np.random.Generator(np.random.PCG64(subset_seed))
    subset = np.sort(g.choice(MODEL.vocab_size, subset_size, replace=False))
    return {"top_ids": top, "top_logits": np.take_along_axis(lg, top, axis=-1),
            "top2_gap": srt[:, -1] - srt[:, -2], "subset": subset, "subset_logits": lg[:, subset],
            "logits_first": lg[0], "logits_last": lg[-1]}


def make_config2(tmp: pathlib.Path) -> None:
    wl = WORKLOADS[2]
    path, model = full_model(tmp)
    ids = np.array(wl.prompt_ids(), dtype=np.int64)
    t0 = time.time()
    tok, lg = baseline_loop(model, ids, wl.new_tokens)
    print(f"config 2 on HF CPU bf16 in {time.time() - t0:.1f}s", flush=True)
    np.savez_compressed(OUT / "config2_bf16.npz", ids=ids, tokens=tok[:, 0],
                        **step_summary(lg[:, 0, :], 512, 512))
    print("wrote config2_bf16.npz", flush=True)


def make_full(tmp: pathlib.Path) -> None:
    wl = WORKLOADS[1]
    path, model = full_model(tmp)
    ids = np.array(wl.prompt_ids(), dtype=np.int64)
    t0 = time.time()
    tok, lg = baseline_loop(model, ids, wl.new_tokens)
    print(f"config 1 on HF CPU bf16 in {time.time() - t0:.1f}s", flush=True)
    lg = lg[:, 0, :]  # [steps, V] (batch 1)
    top = np.argsort(-lg, axis=-1, kind="stable")[:, :16]
    srt = np.sort(lg, axis=-1)
    g = np.random.Generator(np.random.PCG64(4096))
    subset = np.sort(g.choice(MODEL.vocab_size, 4096, replace=False))
    np.savez_compressed(
        OUT / "config1_bf16.npz",
        ids=ids,
        tokens=tok[:, 0],
        top_ids=top,
        top_logits=np.take_along_axis(lg, top, axis=-1),
        top2_gap=srt[:, -1] - srt[:, -2],
        subset=subset,
        subset_logits=lg[:, subset],
        logits_first=lg[0],
        logits_last=lg[-1],
    )
    manifest = json.loads((path / "seeded_manifest.json").read_text())
    (OUT / "qwen3_4b_seed0_manifest.json").write_text(json.dumps(manifest, indent=1))
    print("wrote config1_bf16.npz", flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--skip-full", action="store_true")
    ap.add_argument("--skip-tiny", action="store_true")
    ap.add_argument("--skip-config2", action="store_true")
    ap.add_argument("--model-dir", help="an existing seeded Qwen3-4B checkpoint directory to reuse")
    args = ap.parse_args()
    torch.manual_seed(0)
    import transformers
    with tempfile.TemporaryDirectory() as tmp:
        tmp = pathlib.Path(tmp)
        if args.model_dir:
            (tmp / "qwen3_4b_seeded").symlink_to(pathlib.Path(args.model_dir).resolve())
        if not args.skip_tiny:
            make_tiny(tmp)
        if not args.skip_full:
            make_full(tmp)
        if not args.skip_config2:
            make_config2(tmp)
    meta_path = OUT / "golden_meta.json"
    old = json.loads(meta_path.read_text()) if meta_path.exists() else {}
    meta = {
        "transformers": transformers.__version__,
        "torch": torch.__version__,
        "attn_implementation": "sdpa",
        "device": "cpu",
        "threads": torch.get_num_threads(),
        "tiny": {"config": TINY.to_hf_json(), "seed": TINY_SEED, "std": TINY_STD,
                 "gain_std": TINY_GAIN_STD, "cases": TINY_CASES},
        "config1": {"batch": 1, "prompt": 32, "new_tokens": 32, "model_seed": MODEL_SEED,
                    "prompt_seed": 1},
        "config2": {"batch": 1, "prompt": 1024, "new_tokens": 512, "model_seed": MODEL_SEED,
                    "prompt_seed": 2, "subset": 512},
    }
    if args.skip_tiny and args.skip_full and old:  # keep what the fixtures that were not rewritten were made with
        meta = {**old, "config2": meta["config2"]}
    (OUT / "golden_meta.json").write_text(json.dumps(meta, indent=1))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
