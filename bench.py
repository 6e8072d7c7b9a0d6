"""Benchmark of the cPDE training epoch on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu-baseline]

One step is one training epoch: forward propagation of every derivative row
through the network, the cost, the weight gradient (adjoint compositions,
transposed products, split-K weight contraction) and one RPROP update -- the
work of Server::pass + network::train (cuda/cpde_server.cu:223-257,
cuda/cpde_engine.cuh:993-1014), a superset of the reference's
"fwd+cost+wgrad" timing scope.  Inputs, targets and weights are resident in
HBM before the timed region starts.

Matching workloads drive the device library directly through its C ABI; the
Poisson workload (two expression costs combined by a cost graph) runs through
the protocol server's training command.

Prints one JSON line.  ``value`` is points x derivative rows per second for the
whole job; ``ms_per_step`` the wall-clock milliseconds per epoch.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time
from dataclasses import dataclass
from pathlib import Path
from typing import Callable

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from cpde_amd import hip, workloads  # noqa: E402

METRIC = 'ms/epoch (fwd+cost+wgrad) at order 6, 729 pts; points·derivs/s; % roofline'
# The reference's published order-6 figure for this workload shape: 5.65 ms/epoch
# on an RTX 3090, i.e. 729*28/5.65e-3 points*derivs/s (README.md:63).
PUBLISHED_POINTS_DERIVS_PER_S = 729 * 28 / 5.65e-3
# The reference's published ms/epoch of the same 729-point 2->128x4->1 epoch
# (forward, loss, weight gradient) per derivative order (README.md:57-63).
PUBLISHED_MS = {0: 0.41, 1: 0.68, 2: 1.10, 3: 1.72, 4: 2.40, 5: 3.59, 6: 5.65}
PEAK_FP32_MFMA = 157.3e12   # flop/s, dense
PEAK_HBM = 8.0e12           # bytes/s
MFMA_KINDS = {'gemm_forward', 'gemm_transposed', 'gemm_wgrad', 'fused_forward', 'fused_backward', 'network_forward',
              'network_backward', 'network_epoch'}
# CPU baseline sample: about this many multiply-adds of the linear steps
# (rows x points x sum of n_in*n_out), ~12 s of the reference CPU server on
# one core of the benchmark host.
CPU_SAMPLE_MACS = 3.0e9

# HBM bytes per launch from rocprofv3 counter passes over this benchmark
# (profiles/network_kernels_<workload>_traffic.md and _counters.md): mean FETCH_SIZE and
# WRITE_SIZE in KiB per dispatch, scaled by what the same counters read for a
# plain 256 MiB copy (``--copy-calibration``): 268,435,456 B / 131,084.475 KiB
# read, 268,435,456 B / 262,144 KiB written.
COPY_SCALE = (268435456 / (131084.475 * 1024), 268435456 / (262144 * 1024))
TRAFFIC_KIB = {
    'fourier_fit_order2': {'network_epoch': (5101.3, 30162.8), 'gemm_wgrad': (6878.0, 3898.0),
                           'split_reduce': (3952.1, 2713.1)},
    'fourier_fit_order6': {'network_epoch': (20859.94, 134919.15), 'gemm_wgrad': (31754.55, 4077.5),
                           'split_reduce': (4544.0, 2713.12)},
    'poisson_disk_order2': {'network_epoch': (6934.3, 54427.2), 'gemm_wgrad': (7005.0, 2946.7),
                            'split_reduce': (1940.5, 261.7)},
    'fourier_3d_order4': {'network_forward': (51367.6, 5739531.1), 'network_backward': (1753565.2, 3341379.0),
                          'gemm_wgrad': (2329450.2, 4388.1), 'split_reduce': (22647.6, 1113.0)},
    'fourier_large_order6': {'network_backward': (4986651.81, 8870448.64), 'network_forward': (423199.55, 14688002.1),
                             'gemm_wgrad': (6994723.69, 4064.13)},
}


@dataclass
class Spec:
    make: Callable
    steps: int          # timed epochs by default
    warmup: int
    trace_steps: int
    op90: tuple | None  # (warm-ups, epochs per batch, batches) of the server timing command
    server: bool = False


WORKLOADS = {
    **{f'fourier_fit_order{k}': Spec(lambda k=k: workloads.fourier_fit(k), 500, 50, 20, (20, 100, 7)) for k in range(7)},
    'poisson_disk_order2': Spec(lambda: workloads.PoissonWorkload(), 500, 50, 20, None, server=True),
    'fourier_3d_order4': Spec(lambda: workloads.fourier_3d(), 30, 3, 3, (3, 10, 3)),
    'fourier_large_order6': Spec(lambda: workloads.fourier_large(), 10, 2, 2, (2, 3, 3)),
}


def describe(wl, name):
    if isinstance(wl, workloads.PoissonWorkload):
        return {'workload': name, 'network': '→'.join(str(n) for n in wl.neurons) + ' sigmoid',
                'points': wl.size, 'leaves': [{'rows': r, 'points': p} for r, p in wl.leaves()],
                'step': 'graph pass (interior (u_xx+u_yy+f)^2 + boundary u^2, hipRTC) + weight gradient + RPROP'}
    return {
        'workload': name,
        'network': '→'.join(str(n) for n in wl.neurons) + ' sigmoid',
        'points': wl.size,
        'derivative_rows': wl.rows,
        'chunk': wl.chunk or wl.size,
        'step': 'forward + matching cost + weight gradient + RPROP',
    }


def point_rows(wl):
    return wl.point_rows() if isinstance(wl, workloads.PoissonWorkload) else wl.size * wl.rows


def linear_macs(wl):
    return point_rows(wl) * sum(a * b for a, b in zip(wl.neurons, wl.neurons[1:]))


def traffic(workload, kind):
    kib = TRAFFIC_KIB.get(workload, {}).get(kind)
    if kib is None:
        return None
    return round(kib[0] * 1024 * COPY_SCALE[0] + kib[1] * 1024 * COPY_SCALE[1])


def roofline(report, workload):
    """Dominant kernel class by device time; achieved = its algorithmic work
    per launch divided by its mean launch duration; traffic = its measured HBM
    bytes per launch where a counter pass exists for this workload."""
    kind = max(report, key=lambda k: report[k][1])
    launches, ms, work = report[kind]
    seconds = ms / 1e3
    if kind in MFMA_KINDS:
        achieved, peak, unit, bound = work / seconds / 1e12, PEAK_FP32_MFMA / 1e12, 'TFLOP/s', 'mfma'
    else:
        achieved, peak, unit, bound = work / seconds / 1e9, PEAK_HBM / 1e9, 'GB/s', 'hbm'
    return {'kernel': kind, 'bound': bound, 'achieved': round(achieved, 3), 'peak': peak, 'unit': unit,
            'frac': round(achieved / peak, 4), 'traffic': traffic(workload, kind),
            'launches': launches, 'mean_launch_us': round(ms * 1e3 / launches, 3),
            'work_per_launch': work / launches}


def published_ratio(wl, ms):
    """Published reference ms/epoch over ours for the 729-point Fourier fits."""
    for order, ref in PUBLISHED_MS.items():
        if wl.name == f'fourier_fit_order{order}' and wl.size == 729:
            return {'reference_ms': ref, 'speedup': round(ref / ms, 2)}
    return None


def server_op90(wl, warm, iterations, batches):
    """The reference's own timing scope through the protocol server (op 90:
    forward + cost + weight gradient, no optimizer; C++ host, no Python in the
    loop): median over batches of per-epoch wall and device milliseconds."""
    from cpde_amd import wire
    from cpde_amd.build import SERVER
    with wire.Session(SERVER) as s:
        ids = wl.upload(s)
        r = s.timing(ids['net'], ids['cost'], warm=warm, iterations=iterations, batches=batches,
                     layers=len(wl.neurons) - 1)
    wall, gpu = float(np.median(r['wall_ms'])), float(np.median(r['gpu_ms']))
    return {'ms_per_epoch_wall': round(wall, 5), 'ms_per_epoch_device': round(gpu, 5),
            'points_derivs_per_s': round(wl.size * wl.rows / (wall / 1e3), 1),
            'vs_published': published_ratio(wl, wall),
            'loss': r['loss'], 'scope': f'op 90: {batches} batches x {iterations} epochs after {warm} warm-ups'}


def cpu_sample(wl):
    """A bounded sample of the workload for the CPU baseline: all of it when it
    is small, else evenly spaced points; plus the number of epochs to run."""
    if isinstance(wl, workloads.PoissonWorkload):
        return wl, max(1, round(CPU_SAMPLE_MACS / linear_macs(wl)))
    per_point = linear_macs(wl) / wl.size
    points = min(wl.size, max(64, int(CPU_SAMPLE_MACS / per_point)))
    sample = wl if points == wl.size else wl.subset(points)
    return sample, max(1, round(CPU_SAMPLE_MACS / linear_macs(sample)))


def upload_all(session, wl):
    ids = wl.upload(session)
    if isinstance(wl, workloads.PoissonWorkload):
        return ids['net'], ids['costs'], wl.graph()
    return ids['net'], [ids['cost']], None


def port_epochs(sample, epochs):
    """Seconds for `epochs` matching epochs of the C restatement (oracle/), one
    thread: forward + cost + weight gradient, then one RPROP pass over the
    parameters, as in the timed step."""
    sys.path.insert(0, str(ROOT / 'oracle'))
    import oracle
    x = sample.inputs.transpose(0, 2, 1)
    t0 = time.perf_counter()
    for _ in range(epochs):
        oracle.matching_epoch(sample.neurons, sample.linear, sample.init, sample.cost_schema, x,
                              sample.target[:, :, None], sample.weight_block(), chunk=sample.chunk,
                              rows=sample.cost_rows, target_rows=sample.target_rows,
                              weight_samples=sample.weight_samples, outputs=False)
        for w in sample.init:
            w = np.array(w, np.float32)
            z = np.zeros_like(w)
            oracle.rprop(w, np.full_like(w, 0.002), z, z)
    return time.perf_counter() - t0


def cpu_baseline(wl):
    """The CPU side of the same epoch on one thread.  Preferred: the
    reference's own CPU server built from its sources (oracle/_ref), driven over
    the wire protocol with training epochs (op 8/15: forward + cost + weight
    gradient + statistics + RPROP).  The C restatement of the same matching
    epoch is timed on the same sample beside it (``port``), or alone when the
    reference build is absent."""
    sys.path.insert(0, str(ROOT / 'oracle'))
    import oracle
    sample, epochs = cpu_sample(wl)
    ref = oracle.reference_server()
    what = (f'{epochs} training epoch(s) of {sample.name} ({point_rows(sample)} point-rows'
            f'{")" if sample is wl else f", a {sample.size}-point even subsample of the {wl.size}-point workload)"}')
    port = None
    if not isinstance(wl, workloads.PoissonWorkload):
        seconds = port_epochs(sample, epochs)
        port = {'value': round(point_rows(sample) * epochs / seconds, 1), 'unit': 'points·derivs/s', 'cores': 1,
                'kind': 'port', 'seconds': round(seconds, 3),
                'sample': f'{what} of the C restatement: fwd+cost+wgrad+RPROP, single thread'}
    if ref is not None:
        from cpde_amd import wire
        with wire.Session(ref) as s:
            net, costs, graph = upload_all(s, sample)
            t0 = time.perf_counter()
            s.train(net, costs, epochs, method=0, fresh=1, log=0, graph=graph)
            seconds = time.perf_counter() - t0
        out = {'value': round(point_rows(sample) * epochs / seconds, 1), 'unit': 'points·derivs/s', 'cores': 1,
               'kind': 'reference', 'seconds': round(seconds, 3),
               'sample': f'{what} on the reference CPU server (serial BLAS): fwd+cost+wgrad+stats+RPROP, '
                         'single thread'}
        if port is not None:
            port['ratio_to_reference'] = round(port['value'] / out['value'], 3)
            out['port'] = port
        return out
    return port


def copy_calibration(mib=256, repeats=5):
    """A plain device-to-device copy of known size: what FETCH_SIZE and
    WRITE_SIZE read for it converts those counters into bytes for the kernels
    measured under the same profiler."""
    import torch
    x = torch.ones(mib << 18, dtype=torch.float32, device='cuda')
    y = torch.empty_like(x)
    for _ in range(repeats):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({'copy_bytes_read': x.numel() * 4, 'copy_bytes_written': y.numel() * 4,
                      'launches': repeats}), flush=True)
    return 0


def settle(step, sync, settle_ms):
    """Untimed epochs until ``settle_ms`` of wall time have passed: the GPU
    leaves its idle clocks over the first tens of milliseconds of load (the
    epoch's device time falls from ~135 to ~118 us over its first 100-200
    epochs after an idle gap), and the timed region measures the steady state,
    as the reference's own benchmark does (20 warm-ups, then 7 x 100 epochs)."""
    t0 = time.perf_counter()
    epochs = 0
    while (time.perf_counter() - t0) * 1e3 < settle_ms:
        for _ in range(8):
            step()
        epochs += 8
        sync()
    return {'epochs': epochs, 'ms': round((time.perf_counter() - t0) * 1e3, 1)}


def run_direct(wl, steps, warmup, trace_steps, settle_ms):
    """Matching epochs through the C ABI: returns (wall ms per step, device ms
    per step, loss, device description, trace report, settle record)."""
    device = hip.Device(0)
    name, cus = device.info()
    run = hip.MatchingRun(device, wl)

    def step():
        run.step(collect=True, update=True)

    settled = settle(step, device.synchronize, settle_ms)
    for _ in range(warmup):
        step()
    device.synchronize()
    device.mark(0)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    device.mark(1)
    device.synchronize()
    wall = time.perf_counter() - t0
    device_ms = device.elapsed(0, 1)
    loss = run.loss()
    device.trace(True)
    for _ in range(trace_steps):
        step()
    report = device.trace_report()
    device.trace(False)
    run.close()
    device.close()
    return wall * 1e3 / steps, device_ms / steps, loss, f'{name}, {cus} CUs', report, settled


def run_server(wl, steps, warmup, trace_steps, settle_ms):
    """Graph training epochs through the protocol server (op 15): the server's
    own loop, with the per-epoch scalar download and validation the protocol
    requires.  A second session with CPDE_TRACE_FILE set gives the kernel report."""
    from cpde_amd import wire
    from cpde_amd.build import SERVER
    with wire.Session(SERVER) as s:
        net, costs, graph = upload_all(s, wl)
        settled = settle(lambda: s.train(net, costs, 25, method=0, fresh=1, log=0, graph=graph), lambda: None,
                         settle_ms)
        settled['epochs'] *= 25
        s.train(net, costs, warmup, method=0, fresh=1, log=0, graph=graph)
        t0 = time.perf_counter()
        s.train(net, costs, steps, method=0, fresh=0, log=0, graph=graph)
        wall = time.perf_counter() - t0
        value, _ = s.graph_eval(net, costs, graph, gradient=False)
    with tempfile.TemporaryDirectory() as tmp:
        path = Path(tmp) / 'trace.json'
        env = dict(os.environ, CPDE_TRACE_FILE=str(path))
        with wire.Session(SERVER, env=env) as s:
            net, costs, graph = upload_all(s, wl)
            s.train(net, costs, trace_steps, method=0, fresh=1, log=0, graph=graph)
        report = {k: tuple(v) for k, v in json.loads(path.read_text()).items()}
    return wall * 1e3 / steps, None, value, 'device 0 (protocol server)', report, settled


def other_workloads(names, settle_ms):
    """The other configurations (same step, same clock settling; the larger
    ones for a few epochs), so that their roofline fractions come from this
    run too."""
    out = {}
    for name in names:
        spec = WORKLOADS[name]
        wl = spec.make()
        run = run_server if spec.server else run_direct
        ms, device_ms, _, _, report, settled = run(wl, spec.steps, spec.warmup, spec.trace_steps, settle_ms)
        t_roof = wl.flops_per_epoch() / PEAK_FP32_MFMA + wl.bytes_per_epoch() / PEAK_HBM
        out[name] = {'config': describe(wl, name), 'steps': spec.steps, 'warmup': spec.warmup,
                     'ms_per_step': round(ms, 4),
                     'device_ms_per_step': None if device_ms is None else round(device_ms, 4),
                     'value': round(point_rows(wl) / (ms / 1e3), 1), 'unit': 'points·derivs/s',
                     'epoch_roofline': {'t_roof_ms': round(t_roof * 1e3, 3), 'frac': round(t_roof / (ms / 1e3), 4)},
                     'roofline': roofline(report, name), 'clock_settle': settled,
                     'kernels': {k: {'launches_per_step': v[0] / spec.trace_steps,
                                     'us_per_step': round(v[1] * 1e3 / spec.trace_steps, 3)}
                                 for k, v in sorted(report.items(), key=lambda kv: -kv[1][1])}}
    return out


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=None, help='timed epochs (default: per workload)')
    ap.add_argument('--warmup', type=int, default=None)
    ap.add_argument('--workload', default='fourier_fit_order6', choices=sorted(WORKLOADS))
    ap.add_argument('--trace-steps', type=int, default=None)
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--no-op90', action='store_true', help='skip the protocol-server timing (op 90)')
    ap.add_argument('--settle-ms', type=float, default=250.0,
                    help='untimed epochs for this long before the warm-ups, so the GPU leaves its idle clocks')
    ap.add_argument('--no-other-workloads', action='store_true',
                    help='skip the other configurations (order-2 fit, Poisson graph epoch, 3D order 4, 2->256^4->1 order 6) timed after the main line')
    ap.add_argument('--copy-calibration', action='store_true',
                    help='only run a plain 256 MiB device copy five times (the reference for HBM byte counters)')
    args = ap.parse_args(argv)
    if args.copy_calibration:
        return copy_calibration()
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py measures one GPU only: the cPDE hot path runs on a single device '
              '(multi-GPU point sharding is a design, not a build, here); run with --gpus 1', file=sys.stderr)
        return 2
    spec = WORKLOADS[args.workload]
    steps = args.steps if args.steps is not None else spec.steps
    warmup = args.warmup if args.warmup is not None else spec.warmup
    trace_steps = args.trace_steps if args.trace_steps is not None else spec.trace_steps

    wl = spec.make()
    # The protocol server runs as a child process, started before this process
    # touches the device.
    op90 = None if args.no_op90 or spec.op90 is None else server_op90(wl, *spec.op90)
    runner = run_server if spec.server else run_direct
    ms, device_ms, loss, device, report, settled = runner(wl, steps, warmup, trace_steps, args.settle_ms)

    value = point_rows(wl) / (ms / 1e3)
    t_roof = wl.flops_per_epoch() / PEAK_FP32_MFMA + wl.bytes_per_epoch() / PEAK_HBM
    out = {
        'metric': METRIC,
        'value': round(value, 1),
        'unit': 'points·derivs/s',
        'n_gpus': 1,
        'steps': steps,
        'warmup': warmup,
        'ms_per_step': round(ms, 5),
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': round(value / PUBLISHED_POINTS_DERIVS_PER_S, 3) if args.workload == 'fourier_fit_order6'
        else None,
        'dtype': 'f32',
        'data': 'synthetic (seeded Fourier-sum targets with analytic derivatives / seeded Gaussian sources, '
                'Xavier-uniform weights)',
        'config': describe(wl, args.workload),
        'device': device,
        'device_ms_per_step': None if device_ms is None else round(device_ms, 5),
        'epoch_roofline': {'t_roof_us': round(t_roof * 1e6, 2), 'frac': round(t_roof / (ms / 1e3), 4),
                           'gflop': wl.flops_per_epoch() / 1e9, 'gbytes': wl.bytes_per_epoch() / 1e9},
        'loss_after_timed_steps': loss,
        'roofline': roofline(report, args.workload),
        'kernels': {k: {'launches_per_step': v[0] / trace_steps, 'us_per_step': round(v[1] * 1e3 / trace_steps, 3)}
                    for k, v in sorted(report.items(), key=lambda kv: -kv[1][1])},
        'op90': op90,
        'clock_settle': settled,
        'cpu_baseline': None,
    }
    if not args.no_cpu_baseline:
        out['cpu_baseline'] = cpu_baseline(wl)
    if args.workload == 'fourier_fit_order6' and not args.no_other_workloads:
        out['other_workloads'] = other_workloads(['fourier_fit_order2', 'poisson_disk_order2', 'fourier_3d_order4',
                                                  'fourier_large_order6'], args.settle_ms)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == '__main__':
    sys.exit(main())
