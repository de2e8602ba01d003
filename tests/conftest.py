"""Shared pytest configuration: markers, import path, seeding."""

import os
import random
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running (minutes)")


def seed_all(seed: int = 42):
    """Same global seeding as the reference's test utilities (tests/utils.py:92-97)."""
    random.seed(seed)
    torch.manual_seed(seed)


@pytest.fixture(autouse=True)
def _seed():
    seed_all(42)
