import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(REPO, 'dynamic-kv-cache_amd')
for p in (REPO, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an MI355X (HIP device) and the built libdkv.so')


@pytest.fixture(scope='session')
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip('no HIP device')
    from dkv import _lib
    _lib.load()  # fails loudly if libdkv.so is missing: there is no fallback path
    return torch.device('cuda:0')


def announce(msg):
    """Names the GPU case before it runs, so a fault that ends the process still says which case."""
    print(f'[gpu-case] {msg}', flush=True)
