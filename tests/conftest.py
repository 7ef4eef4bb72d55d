"""Shared pytest configuration.

Markers: ``gpu`` -- needs an MI355X (run with ``-m gpu``); everything else
runs on the CPU.  GPU tests print the case they are about to launch (and
flush) so a failure names its kernel and shape.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (HIP path through the C ABI)")


def announce(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
