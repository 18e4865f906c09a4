import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, 'vesta-gpu_amd')
for p in (PKG, REPO):
    if p not in sys.path:
        sys.path.insert(0, p)

REFERENCE = '/root/reference'


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an MI355X (run with -m gpu on the GPU box)')
    config.addinivalue_line('markers', 'slow: long CPU test')


@pytest.fixture(scope='session')
def small_text():
    with open(os.path.join(PKG, 'vesta', 'programs', 'gpt2.vst')) as fh:
        return fh.read()
