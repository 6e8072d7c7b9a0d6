"""Per-phase clock stamps of the one-pass matching epoch kernel (diagnostics).

With ``CPDE_PHASE_STAMPS=1`` the library generates its one-pass epoch kernels
with a clock stamp after every phase (input layer, each hidden layer, output
layer, cost, output backward, each hidden backward, input gradient, and the
barriers between them); lane 0 of each workgroup writes them over the block's
output stack when the epoch ends: cycles since the workgroup began, then the
100 MHz real-time clock at its start and at its end.  This script trains the
named workload for a while, downloads the stamps of a number of epochs and
prints, per phase, the median cycles of the workgroups dispatched first,
second and third on their compute units (blocks 0-255, 256-511, 512-...), and
the spread of the workgroups' end times.  The output stack holds stamps, not
outputs, in this mode: it is for measurement only.

    CPDE_PHASE_STAMPS=1 python3 -m cpde_amd.stamps --workload fourier_fit_order6
"""
from __future__ import annotations

import argparse
import os
import sys

import numpy as np

from . import hip, workloads


def phase_names(neurons):
    """The stamps' phases in the order the one-pass matching epoch runs them."""
    h = len(neurons) - 3
    names = ['input layer', 'barrier']
    names += [f'hidden {t} forward' for t in range(1, h + 1)]
    names += ['output layer', 'barrier', 'matching cost', 'output backward']
    names += [f'hidden {t} backward' for t in range(h, 0, -1)]
    names += ['input gradient']
    return names


def collect(workload, warmup, epochs):
    dev = hip.Device(0)
    run = hip.MatchingRun(dev, workload)
    for _ in range(warmup):
        run.step(update=True)
    dev.synchronize()
    R, n_out = len(workload.cost_schema), workload.neurons[-1]
    dest = hip.Buffer(dev, R * workload.size * n_out * 4)
    rows = np.arange(R, dtype=np.int32)
    out = []
    for _ in range(epochs):
        run.step(update=True)
        dev.synchronize()
        run.plan.output(dest, workload.size, rows, 0, workload.size)
        stack = dest.download(np.float32, R * workload.size * n_out).reshape(R, workload.size, n_out)
        out.append(stack[:, :, 0].view(np.uint32).copy())
    dest.free()
    dev.close()
    return np.stack(out)  # [epoch][slot][point]


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split('\n\n')[0])
    ap.add_argument('--workload', default='fourier_fit_order6', choices=[f'fourier_fit_order{k}' for k in range(5, 7)])
    ap.add_argument('--warmup', type=int, default=300)
    ap.add_argument('--epochs', type=int, default=20)
    ap.add_argument('--save', default=None, help='also write the raw stamps (.npy: epoch x slot x point)')
    args = ap.parse_args(argv)
    if os.environ.get('CPDE_PHASE_STAMPS') != '1':
        sys.exit('set CPDE_PHASE_STAMPS=1: the stamps are generated into the kernels only then')
    wl = workloads.fourier_fit(int(args.workload[-1]))
    names = phase_names(wl.neurons)
    n = len(names)
    u = collect(wl, args.warmup, args.epochs).astype(np.int64)
    if args.save:
        np.save(args.save, u)
    t = u[:, :n, :]
    w0, w1 = u[:, n, :], u[:, n + 1, :]
    if not (np.diff(t, axis=1) >= 0).all() or not (w1 > w0).all():
        sys.exit('the output stack does not hold phase stamps (was the module generated with CPDE_PHASE_STAMPS=1?)')
    waves = 4
    hw = u[:, n + 2:n + 2 + waves, :]  # hardware id register of each wave
    simd = (hw >> 4) & 3
    d = np.diff(np.concatenate([np.zeros_like(t[:, :1, :]), t], axis=1), axis=1)
    blocks = t.shape[2]
    tiers = [(f'blocks {a}-{min(b, blocks) - 1}', slice(a, min(b, blocks))) for a, b in ((0, 256), (256, 512), (512, 768))
             if a < blocks]
    print(f'{args.workload}: {blocks} workgroups, {args.epochs} epochs after {args.warmup}')
    print('| phase | ' + ' | '.join(name for name, _ in tiers) + ' |')
    print('|---|' + '---:|' * len(tiers))
    for k in range(n):
        print(f'| {names[k]} | ' + ' | '.join(f'{np.median(d[:, k, s]):.0f}' for _, s in tiers) + ' |')
    print('| total | ' + ' | '.join(f'{np.median(t[:, n - 1, s]):.0f}' for _, s in tiers) + ' |')
    span = (w1 - w0.min(axis=1, keepdims=True)) * 0.01  # µs
    life = (w1 - w0) * 0.01
    print(f'workgroup end (µs after the first start), median over epochs: '
          f'min {np.median(span.min(axis=1)):.1f}, median {np.median(np.median(span, axis=1)):.1f}, '
          f'max {np.median(span.max(axis=1)):.1f}')
    for name, s in tiers:
        print(f'{name}: lifetime median {np.median(life[:, s]):.1f} µs; cycles per µs '
              f'{np.median(t[:, n - 1, s]) / np.median(life[:, s]):.0f}')
    print('SIMD of waves 0-3 (share of workgroups per SIMD):')
    for w in range(waves):
        share = [float((simd[:, w, :] == k).mean()) for k in range(4)]
        print(f'  wave {w}: ' + ', '.join(f'SIMD {k} {share[k]:.2f}' for k in range(4)))


if __name__ == '__main__':
    main()
