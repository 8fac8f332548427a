import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built library")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP device visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def seeded_torch():
    import torch

    devices = [torch.cuda.current_device()] if torch.cuda.is_available() else []
    with torch.random.fork_rng(devices=devices):
        torch.manual_seed(0)
        yield torch


@pytest.fixture
def sequence_cls(monkeypatch):
    """The engine's Sequence with 4-token blocks (restored after the test)."""
    from microinfer_amd.engine.sequence import Sequence

    monkeypatch.setattr(Sequence, "block_size", 4)
    return Sequence


@pytest.fixture
def scheduler_factory(sequence_cls):
    from microinfer_amd.engine.blockmanager import BlockManager
    from microinfer_amd.engine.config import EngineConfig
    from microinfer_amd.engine.scheduler import Scheduler

    def make(*, num_blocks=8, **limits):
        values = dict(max_num_seqs=4, max_num_batched_tokens=8, max_model_len=32,
                      eos_token_id=0)
        values.update(limits)
        manager = BlockManager(num_blocks, sequence_cls.block_size)
        return Scheduler(EngineConfig(**values), manager), manager

    return make
