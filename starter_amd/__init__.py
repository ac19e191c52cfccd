"""MI355X-native Qwen3-4B greedy-decode engine (gfx950 HIP kernels behind a C ABI).

``from starter_amd.engine import Engine`` is the drop-in for the reference's
``engine/engine.py`` ``Engine(model_path)`` / ``Engine.generate(input_ids,
max_new_tokens)``.
"""
