"""The reference's published Fourier benchmark workload, regenerated to pin the
published losses (test fixture generator, not part of the package).

Reproducing the published numbers bit for bit needs the same random draws and
the same arithmetic as the reference's own benchmark script and Python
initialiser, so these two functions restate them:

  * ``reference_init``: cpde/api.py:277-280 -- U(+-2/sqrt(fan_in)) weights in
    column-major order, then U(+-0.1) biases, from one generator;
  * ``reference_benchmark``: scripts/benchmark_fourier_performance.py:20-57 --
    27x27 grid in [-1,1]^2, a 10x10 grid of Fourier coefficients (seed 2026)
    with analytic derivatives, rows weighted by 1/var, weights from
    ``reference_init`` with seed 3407.

``PUBLISHED_LOSSES`` are the losses at initial weights for orders 0..6 of the
RTX 3090 CUDA build (docs/benchmarks/fourier-rtx3090.json:159,189,219,249,279,
309,339).
"""
from __future__ import annotations

import numpy as np

from cpde_amd import workloads as W

PUBLISHED_LOSSES = [1519.6657229734592, 2989.1356939971447, 5187.967334091663, 8111.595301151276,
                    11767.45415353775, 16145.947476387024, 21259.16511631012]


def reference_init(neurons, seed):
    rng = np.random.default_rng(seed)
    blocks = []
    for fan_in, fan_out in zip(neurons, neurons[1:]):
        bound = 2 / np.sqrt(fan_in)
        weights = rng.uniform(-bound, bound, fan_out * fan_in)
        biases = rng.uniform(-.1, .1, fan_out)
        blocks.append(np.concatenate((weights, biases)).astype(np.float32))
    return blocks


def reference_benchmark(order):
    neurons = [2, 128, 128, 128, 128, 1]
    schema = W.closed_schema(2, [(i, order - i) for i in range(order + 1)])
    x, y = np.meshgrid(np.linspace(-1, 1, 27), np.linspace(-1, 1, 27), indexing='ij')
    pts = np.column_stack((x.ravel(), y.ravel())).astype(np.float32)
    px, py = pts.astype(float).T
    coef = np.random.default_rng(2026).uniform(-1, 1, (4, 10, 10))
    target = np.zeros((len(schema), len(pts)))
    for row, (_, dx, dy) in enumerate(schema):
        for n in range(1, 11):
            for k in range(1, 11):
                a, b, c, d = coef[:, n - 1, k - 1] * n ** int(dx) * k ** int(dy) / (n * k)
                sx, cx = np.sin(n * px + dx * np.pi / 2), np.cos(n * px + dx * np.pi / 2)
                sy, cy = np.sin(k * py + dy * np.pi / 2), np.cos(k * py + dy * np.pi / 2)
                target[row] += a * sx * sy + b * sx * cy + c * cx * sy + d * cx * cy
    weights = (1 / target.std(axis=1) ** 2).astype(np.float32)
    return W.MatchingWorkload(f'reference_fourier_order{order}', neurons, pts, schema, target.astype(np.float32),
                              weights, reference_init(neurons, 3407))
