import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, 'two-level-attention_amd'),
             os.path.join(ROOT, 'tests')):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line(
        'markers', 'gpu: needs a HIP GPU (MI355X) and the built libnfa_hip.so')


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason='no HIP GPU in this environment')
    for item in items:
        if 'gpu' in item.keywords:
            item.add_marker(skip)
