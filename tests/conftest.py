import os
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests" / "golden"))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: generates the full 8 GB seeded model on the CPU")


def pytest_collection_modifyitems(config, items):
    if os.environ.get("Q3_SKIP_SLOW"):
        skip = pytest.mark.skip(reason="Q3_SKIP_SLOW set")
        for item in items:
            if "slow" in item.keywords:
                item.add_marker(skip)


@pytest.fixture(scope="session")
def tiny_ckpt(tmp_path_factory):
    """The tiny seeded model the HF fixtures were generated from."""
    from make_golden import TINY, TINY_GAIN_STD, TINY_SEED, TINY_STD

    from starter_amd.checkpoint import write_seeded_checkpoint

    path = tmp_path_factory.mktemp("tiny")
    write_seeded_checkpoint(path, TINY, TINY_SEED, TINY_STD, TINY_GAIN_STD)
    return path


@pytest.fixture(scope="session")
def tile_ckpt(tmp_path_factory):
    """A small seeded model whose projections all tile for the fused MFMA decode
    path (N % 64, K % 256): hidden 512, intermediate 1024, 8/2 heads, vocab 1024."""
    from starter_amd.checkpoint import Qwen3Config, write_seeded_checkpoint

    cfg = Qwen3Config(num_hidden_layers=2, hidden_size=512, intermediate_size=1024,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=128,
                      vocab_size=1024, max_position_embeddings=2048)
    path = tmp_path_factory.mktemp("tile")
    write_seeded_checkpoint(path, cfg, 5, 0.05, 0.1)
    return path


@pytest.fixture(scope="session")
def full_ckpt():
    """The seeded Qwen3-4B checkpoint (8 GB), written once per machine."""
    from starter_amd.checkpoint import ensure_seeded_checkpoint
    from starter_amd.workloads import MODEL, MODEL_SEED

    base = pathlib.Path(os.environ.get("Q3_CKPT_DIR", "/tmp/q3_seeded_qwen3_4b"))
    return ensure_seeded_checkpoint(base, MODEL, MODEL_SEED)
