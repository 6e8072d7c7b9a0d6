"""Pins the oracle's optimizers (RPROP, step set/restore, Adam) against
multi-epoch trajectories of the reference CPU server (tests/golden/optimizer.npz,
written by tests/golden/make_golden.py).

Each trajectory stores, for every epoch, the gradient that the epoch's update
consumed (an op-14 evaluation at the same weights) and the whole optimizer
state after it.  Replaying the updates through the oracle from the initial
state must reproduce every state bit for bit: weights, steps or moments, both
gradient buffers and the active flags.  CPU only."""
import numpy as np
import pytest

import oracle
from cpde_amd import wire
from helpers import load_golden

RUNS = {
    # prefix: (reset_steps, restore_every, restore_step)
    'rprop': (0.0, 0, 0.0),
    'bigstep': (0.05, 0, 0.0),
    'restore': (2e-4, 2, 1e-3),
}


# transitions each trajectory must exercise (grow x1.2, rollback x0.5, plain):
# the large reset step reverses signs within six epochs, the default step
# and the restored floor do not
MIN_TRANSITIONS = {'rprop': (20, 0, 20), 'bigstep': (20, 20, 20), 'restore': (0, 0, 0)}


def initial_state(g):
    T = len(g['neurons']) - 1
    return [dict(W=np.array(g[f'init{t}'], np.float32), buf={1: np.zeros_like(g[f'init{t}']),
                                                            2: np.zeros_like(g[f'init{t}'])},
                 S=np.full_like(g[f'init{t}'], 0.002), active=1) for t in range(T)]


def compare(state, blob, where):
    _, layers = wire.decode_state(bytes(blob))
    for t, (ours, ref) in enumerate(zip(state, layers)):
        W, b1, b2, S = ref['buffers']
        np.testing.assert_array_equal(ours['W'], W, err_msg=f'{where} W{t}')
        np.testing.assert_array_equal(ours['buf'][1], b1, err_msg=f'{where} buffer 1 of {t}')
        np.testing.assert_array_equal(ours['buf'][2], b2, err_msg=f'{where} buffer 2 of {t}')
        np.testing.assert_array_equal(ours['S'], S, err_msg=f'{where} step{t}')
        assert ours['active'] == ref['active'], where


def branch_counts(g, gprev, W, S):
    """Entries taking each RPROP transition (cuda/derivative_kernels_v4.cu:752-778)."""
    prod = (g * gprev).astype(np.float32)
    grow = prod > 0
    rollback = prod < 0
    plain = (prod == 0) & (g != 0)
    return np.array([grow.sum(), rollback.sum(), plain.sum()])


@pytest.mark.parametrize('prefix', list(RUNS))
def test_rprop_trajectory_matches_reference(prefix):
    """RPROP epochs replayed through orc_rprop (and orc_set_steps /
    orc_restore_steps where the run asks for them) against the reference's
    state after every epoch; the trajectories must exercise growth (x1.2),
    rollback (x0.5) and plain steps."""
    g = load_golden('optimizer')
    reset, every, floor = RUNS[prefix]
    state = initial_state(g)
    if reset:
        for L in state:
            L['S'], L['buf'][1], L['buf'][2] = oracle.set_steps(reset, L['S'], L['buf'][1], L['buf'][2])
    counts = np.zeros(3, np.int64)
    for k in range(int(g[f'{prefix}_epochs'])):
        for t, L in enumerate(state):
            act, inact = L['active'], 3 - L['active']
            grad = g[f'{prefix}_grad{k}_{t}']
            counts += branch_counts(grad, L['buf'][inact], L['W'], L['S'])
            W, S, ga, gi = oracle.rprop(L['W'], L['S'], grad, L['buf'][inact])
            L['W'], L['S'], L['buf'][act], L['buf'][inact] = W, S, ga, gi
            L['active'] = inact
        if every and (k + 1) % every == 0:
            for L in state:
                L['S'], L['buf'][1], L['buf'][2] = oracle.restore_steps(floor, L['S'], L['buf'][1], L['buf'][2])
        compare(state, g[f'{prefix}_state{k}'], f'{prefix} epoch {k + 1}')
    print(f'[rprop {prefix}] grow/rollback/plain transitions: {counts.tolist()}')
    assert (counts >= MIN_TRANSITIONS[prefix]).all(), counts


def test_adam_trajectory_matches_reference():
    """Three Adam epochs (lr 0.01) replayed through orc_adam: weights, both
    moments and the untouched gradient buffer bit-identical to the
    reference's state after every epoch (ADAM_k, cuda/derivative_kernels_v4.cu:780-799;
    M in the step buffer, V in the inactive gradient buffer,
    cuda/cpde_engine.cuh:1008-1011)."""
    g = load_golden('optimizer')
    state = initial_state(g)
    for L in state:
        L['S'] = np.zeros_like(L['S'])
    for k in range(int(g['adam_epochs'])):
        for t, L in enumerate(state):
            grad = g[f'adam_grad{k}_{t}']
            L['W'], L['S'], L['buf'][2] = oracle.adam(L['W'], grad, L['S'], L['buf'][2], np.float32(0.01), k + 1)
            L['buf'][1] = np.array(grad, np.float32)
        compare(state, g[f'adam_state{k}'], f'adam epoch {k + 1}')
    meta, _ = wire.decode_state(bytes(g['adam_state2']))
    assert meta['adam_step'] == 3 and meta['optimizer'] == 1


def test_adam_moment_bias_correction_closed_form():
    """One Adam step from zero moments is w - lr * g / (|g| + 1e-8) to within
    the fp32 rounding of the moments: a dropped bias correction (a factor 10
    in m-hat) or a wrong second moment fails it."""
    rng = np.random.default_rng(5)
    g = rng.standard_normal(1000).astype(np.float32)
    W = rng.uniform(-1, 1, 1000).astype(np.float32)
    W1, m, v = oracle.adam(W, g, np.zeros_like(W), np.zeros_like(W), np.float32(0.01), 1)
    # the betas are the fp32 constants 0.9f and 0.999f
    np.testing.assert_allclose(m, (1 - np.float64(np.float32(0.9))) * g, rtol=1e-6)
    np.testing.assert_allclose(v, (1 - np.float64(np.float32(0.999))) * g.astype(np.float64) ** 2, rtol=1e-6)
    expected = W - 0.01 * g / (np.abs(g.astype(np.float64)) + 1e-8)
    np.testing.assert_allclose(W1, expected, rtol=0, atol=2e-7)
