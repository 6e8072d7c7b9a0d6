import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / 'oracle', ROOT / 'tests' / 'golden'):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an MI355X; drives the HIP library through its C ABI')
    config.addinivalue_line('markers', 'slow: long CPU-side oracle run')


@pytest.fixture(scope='session')
def device():
    from cpde_amd import hip
    d = hip.Device(int(os.environ.get('CPDE_TEST_DEVICE', '0')))
    name, cus = d.info()
    print(f'\n[device] {name} CUs={cus}', flush=True)
    yield d
    d.close()


@pytest.fixture(params=['network', 'partition', 'layer', 'table'])
def path(request, monkeypatch):
    """Which kernel family a plan uses (chosen at plan creation): the
    schema-specialised network-fused kernels on Taylor-scaled stacks (the
    default) or on unscaled stacks with partition-sum compositions, the
    layer-fused kernels, or the table-driven ones."""
    monkeypatch.setenv('CPDE_FUSED', {'network': '2', 'partition': '2', 'layer': '1', 'table': '0'}[request.param])
    monkeypatch.setenv('CPDE_SCALED', '0' if request.param == 'partition' else '1')
    return request.param
