"""Shared pytest configuration: the `gpu` marker and package import helpers."""
from __future__ import annotations

import importlib
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

PACKAGE = "4d_ttt_merging_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible in this process")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def import_package(name: str = ""):
    """Import the product package (or one of its submodules) by its digit-led name."""
    return importlib.import_module(PACKAGE + ("." + name if name else ""))


@pytest.fixture(scope="session")
def vgo():
    return import_package()


@pytest.fixture(scope="session")
def device():
    return torch.device("cuda", 0)
