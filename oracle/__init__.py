"""Test infrastructure: CPU restatement of the reference's Qwen3 greedy decode.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker (or the timed CPU
baseline), never as the product path.  The engine in ``starter_amd`` never
imports it.
"""
