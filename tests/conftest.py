import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an MI355X (gfx950) GPU and the built HIP library')


def pytest_collection_modifyitems(config, items):
    """GPU tests need a visible device; without one they are skipped (the
    round-end GPU run has one, this container does not)."""
    try:
        import torch
        have_gpu = torch.cuda.is_available()
    except Exception:                    # pragma: no cover
        have_gpu = False
    if have_gpu:
        return
    skip = pytest.mark.skip(reason='no GPU visible')
    for item in items:
        if 'gpu' in item.keywords:
            item.add_marker(skip)
