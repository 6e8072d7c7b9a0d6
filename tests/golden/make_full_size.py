"""Writes the full-size golden vectors of the two largest workloads by driving
the reference CPU server (``make -C oracle ref``) through this package's wire
client:

  * ``fourier3d_full``: 3->128x5->1 sigmoid, all mixed partials through order 4
    (35 rows), 32,768 points on the 32^3 grid;
  * ``large_full``: 2->256x4->1 sigmoid, order 6 (28 rows), 262,144 points on
    the 512^2 grid.

The reference server is single-threaded (portable serial BLAS), so the epoch is
cut into point slices that run in parallel server processes.  Each slice is an
op-14 evaluation with gradient (cuda/cpde_server.cu:535-551) of the same cost
(same network, row weights and targets) on its own points; the matching cost
and its weight gradient are sums over points, so the epoch's loss and gradient
are the sums of the slices' (in float64 here; the reference itself adds chunks
in fp32, which differs only in rounding).  Stored per case:

  * ``loss``;
  * per transition: the full gradient when it has at most 1,024 entries,
    otherwise its projections onto the fixed probe vectors of make_golden.py
    and its norm (``grad{t}_probes``, ``grad{t}_norm``);
  * ``outputs`` at 64 evenly spaced points (op 4 + op 5), [row][point][out];
  * checksums of the generated inputs, so the tests can rebuild them.

    make -C oracle ref && python tests/golden/make_full_size.py [case ...] [--workers N]
"""
from __future__ import annotations

import argparse
import multiprocessing as mp
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(HERE))

from cpde_amd import wire, workloads as W  # noqa: E402
from make_golden import SERVER, SINGLE_LEAF, checksum, probes  # noqa: E402

CASES = {
    # name: (generator, slice points)
    'fourier3d_full': ('fourier_3d', 4096),
    'large_full': ('fourier_large', 8192),
}
SAMPLED = 64


def build(generator):
    return getattr(W, generator)()


def slice_workload(wl, begin, end):
    return W.MatchingWorkload(f'{wl.name}[{begin}:{end}]', wl.neurons, wl.points[begin:end], wl.schema,
                              wl.target[:, begin:end], wl.row_weights, wl.init)


def run_slice(job):
    generator, begin, end = job
    wl = slice_workload(build(generator), begin, end)
    t0 = time.time()
    with wire.Session(SERVER) as s:
        ids = wl.upload(s, 0)
        value, grads = s.graph_eval(ids['net'], [ids['cost']], SINGLE_LEAF, gradient=True)
    print(f'[golden] {generator} points {begin}:{end} loss {value!r} {time.time() - t0:.0f} s', flush=True)
    return begin, value, [np.asarray(g, np.float64) for g in grads]


def sampled_outputs(wl, idx):
    x = W.MatchingWorkload('sampled', wl.neurons, wl.points[idx], wl.schema, wl.target[:, idx], wl.row_weights,
                           wl.init)
    with wire.Session(SERVER) as s:
        d = s.data(x.inputs, x.schema)
        n = s.network(x.neurons, x.linear, x.init)
        out = s.eval(n, d, 0)
        return s.download(out).reshape(x.rows, len(idx), x.neurons[-1])


def make(name, workers):
    generator, step = CASES[name]
    wl = build(generator)
    jobs = [(generator, b, min(b + step, wl.size)) for b in range(0, wl.size, step)]
    t0 = time.time()
    with mp.get_context('spawn').Pool(workers) as pool:
        parts = sorted(pool.map(run_slice, jobs, chunksize=1), key=lambda p: p[0])
    loss = float(sum(p[1] for p in parts))
    grads = [sum(p[2][t] for p in parts) for t in range(len(wl.neurons) - 1)]
    idx = np.linspace(0, wl.size - 1, SAMPLED).astype(int)
    rec = dict(generator=np.array(generator), generator_args=np.array('{}'), loss=np.float64(loss),
               slices=np.int32(len(jobs)), sampled=idx.astype(np.int64), outputs=sampled_outputs(wl, idx),
               checksums=np.stack([checksum(wl.points), checksum(wl.target), checksum(wl.row_weights),
                                   checksum(np.concatenate(wl.init))]))
    for t, g in enumerate(grads):
        if g.size <= 1024:
            rec[f'grad{t}'] = g.astype(np.float32)
        else:
            rec[f'grad{t}_probes'] = probes(g.size) @ g
            rec[f'grad{t}_norm'] = np.float64(np.linalg.norm(g))
    np.savez_compressed(HERE / f'{name}.npz', **rec)
    print(f'[golden] {name}: {len(jobs)} slices, loss {loss!r}, {time.time() - t0:.0f} s', flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('cases', nargs='*')
    ap.add_argument('--workers', type=int, default=4)
    args = ap.parse_args()
    if not SERVER.exists():
        raise SystemExit(f'{SERVER} missing: run make -C oracle ref')
    for name in args.cases or list(CASES):
        make(name, args.workers)


if __name__ == '__main__':
    main()
