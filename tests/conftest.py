import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_collection_modifyitems(config, items):
    """GPU tests are skipped (not failed) where no HIP device is visible."""
    if not any("gpu" in it.keywords for it in items):
        return
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP GPU visible")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)
