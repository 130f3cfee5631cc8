"""Test configuration: the ``gpu`` marker and shared helpers.

Tests marked ``gpu`` need an AMD GPU (``torch.cuda`` on ROCm) and are skipped
elsewhere.  The repository root is put on ``sys.path`` so ``oracle`` and the
package import without installation.
"""
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="needs a HIP GPU")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
