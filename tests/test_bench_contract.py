"""The benchmark script's contract on the CPU: it parses, names every
configuration it times, refuses more than one GPU with a message before
touching a device, and computes the roofline of the epoch from shapes alone."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def run(*args):
    return subprocess.run([sys.executable, str(ROOT / 'bench.py'), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_help_lists_every_workload():
    r = run('--help')
    assert r.returncode == 0, r.stderr
    for name in ('fourier_fit_order6', 'fourier_fit_order2', 'poisson_disk_order2', 'fourier_3d_order4',
                 'fourier_large_order6'):
        assert name in r.stdout


def test_more_than_one_gpu_is_refused():
    r = run('--gpus', '2')
    assert r.returncode != 0
    assert 'one GPU' in r.stderr or '--gpus 1' in r.stderr


def test_workload_table_and_epoch_roofline():
    sys.path.insert(0, str(ROOT))
    import bench
    assert set(bench.WORKLOADS) >= {'fourier_fit_order6', 'fourier_fit_order2', 'poisson_disk_order2',
                                    'fourier_3d_order4', 'fourier_large_order6'}
    wl = bench.WORKLOADS['fourier_fit_order6'].make()
    t_roof = wl.flops_per_epoch() / bench.PEAK_FP32_MFMA + wl.bytes_per_epoch() / bench.PEAK_HBM
    assert abs(t_roof * 1e6 - 64.83) < 0.05   # T_roof of the 729-point order-6 fit
    assert bench.WORKLOADS['poisson_disk_order2'].server
