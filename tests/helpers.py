"""Shared numerics helpers and golden-record loading for the parity tests."""
import ast
from pathlib import Path

import numpy as np
import pytest

from cpde_amd import workloads as W

GOLDEN = Path(__file__).resolve().parent / 'golden'


def scaled_error(got, want, axis=None):
    """max |got-want| / max(|want|, rms of the row): a relative error that does
    not blow up on entries that cancel to ~0 inside a derivative row."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    if axis is None:
        scale = np.maximum(np.abs(want), np.sqrt(np.mean(want ** 2)) + 1e-30)
    else:
        rms = np.sqrt(np.mean(want ** 2, axis=axis, keepdims=True)) + 1e-30
        scale = np.maximum(np.abs(want), rms)
    return float(np.max(np.abs(got - want) / scale))


def rel_l2(got, want):
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def checksum(a):
    a = np.asarray(a, np.float64).ravel()
    return np.array([a.size, a.sum(), (a * a).sum(), (a * np.arange(a.size) / max(a.size, 1)).sum()])


def probes(count, seed=2718):
    """The fixed probe vectors of tests/golden/make_golden.py."""
    return np.random.default_rng(seed).standard_normal((64, count))


def load_golden(name):
    """A golden record; records of generated workloads get their inputs rebuilt
    by the workload generator and checked against the stored checksums."""
    path = GOLDEN / f'{name}.npz'
    if not path.exists():
        pytest.skip(f'{path.name} not generated')
    g = dict(np.load(path, allow_pickle=False))
    if 'generator' in g:
        wl = getattr(W, str(g['generator']))(**ast.literal_eval(str(g['generator_args'])))
        got = np.stack([checksum(wl.points), checksum(wl.target), checksum(wl.row_weights),
                        checksum(np.concatenate(wl.init))])
        assert np.allclose(got, g['checksums'], rtol=1e-12, atol=0), 'workload generator drifted'
        g.update(schema=wl.schema, points=wl.points, target=wl.target, row_weights=wl.row_weights)
        for t, w in enumerate(wl.init):
            g[f'init{t}'] = w
    return g


def golden_workload(g):
    """MatchingWorkload of a golden record."""
    T = len(g['neurons']) - 1
    return W.MatchingWorkload('golden', list(g['neurons']), g['points'], g['schema'], g['target'],
                              g['row_weights'], [g[f'init{t}'] for t in range(T)], chunk=int(g['chunk']))


def golden_form(g, prefix):
    """MatchingWorkload of a record written by make_golden.workload_record."""
    T = len(g[f'{prefix}_neurons']) - 1
    return W.MatchingWorkload(prefix, list(g[f'{prefix}_neurons']), g[f'{prefix}_points'], g[f'{prefix}_schema'],
                              g[f'{prefix}_target'], g[f'{prefix}_weights'], [g[f'{prefix}_init{t}'] for t in range(T)],
                              chunk=int(g[f'{prefix}_chunk']), linear=g[f'{prefix}_linear'], rows=g[f'{prefix}_rows'],
                              target_schema=g[f'{prefix}_target_schema'], target_rows=g[f'{prefix}_target_rows'])


def oracle_epoch(wl, outputs=False):
    """The oracle's epoch of a MatchingWorkload: loss, gradients, outputs."""
    import oracle
    return oracle.matching_epoch(wl.neurons, wl.linear, wl.init, wl.cost_schema, wl.inputs.transpose(0, 2, 1),
                                 wl.target[:, :, None], wl.weight_block(), chunk=wl.chunk, rows=wl.cost_rows,
                                 target_rows=wl.target_rows, weight_samples=wl.weight_samples, outputs=outputs)


def check_gradient(g, t, grad, tol):
    """Relative L2 of a transition's gradient against the record (full vector,
    or its probe projections and norm)."""
    if f'grad{t}' in g:
        err = rel_l2(grad, g[f'grad{t}'])
    else:
        p = probes(grad.size) @ np.asarray(grad, np.float64)
        err = max(np.linalg.norm(p - g[f'grad{t}_probes']) / np.linalg.norm(g[f'grad{t}_probes']),
                  abs(np.linalg.norm(np.asarray(grad, np.float64)) / g[f'grad{t}_norm'] - 1))
    assert err < tol, (t, err)
    return err
