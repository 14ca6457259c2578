"""Shared test configuration: markers, repo-root import path, golden fixtures."""

from __future__ import annotations

import json
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm) device and the built libsqx_hip.so")
    config.addinivalue_line("markers", "slow: long-running (full-size shapes)")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm device visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def known_answers() -> dict:
    return json.loads((GOLDEN / "known_answers.json").read_text())


def print_case(*parts) -> None:
    """Name the case before a GPU step so a run that dies still says which one it was."""
    print("[case]", *parts, flush=True)
    sys.stdout.flush()
