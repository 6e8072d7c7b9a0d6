"""Pins the oracle against what the mathematics fixes (CPU only).

* composition: every row of d^alpha sigma(z) against a float64 Taylor-jet
  composition (tests/jet.py), for 1-3 variables through order 6 and a
  non-full (Poisson) closure; the single-variable rows also against the closed
  forms of sigma^(k);
* the jet of sigma'(z): against sigma(1-sigma) as a series and against
  d y / d z_0 from the complex-step Jacobian;
* adjoint: against J^T g with J the complex-step Jacobian of the jet
  composition -- a dropped pair, a wrong binomial or a transposed index fails;
* products: the serial column-major SGEMM against a float64 matmul;
* matching cost: against a direct numpy statement, including zero weights,
  padding lanes and the first non-finite location;
* RPROP: the reference's known answers (tests/test_rprop.py:42-150 in the
  reference), restated at the update level;
* gradient statistics: known answers (tests/reduction_probe.cu:29-87).
"""
import numpy as np
import pytest

import oracle
from cpde_amd import workloads as W
from jet import compose_jacobian, compose_prime_stack, compose_stack

SCHEMAS = {
    '1var_order6': W.full_schema(1, 6),
    '2var_order6': W.full_schema(2, 6),
    '3var_order4': W.full_schema(3, 4),
    '3var_order3': W.full_schema(3, 3),
    'poisson': W.closed_schema(2, [(2, 0), (0, 2)]),
    'mixed_closure': W.closed_schema(2, [(3, 1), (0, 4)]),
}


def random_stacks(schema, count, seed):
    rng = np.random.default_rng(seed)
    z = rng.standard_normal((len(schema), count)) * 0.8
    z[0] = rng.uniform(-3, 3, count)
    return z.astype(np.float32)


@pytest.mark.parametrize('name', list(SCHEMAS))
def test_composition_against_taylor_jet(name):
    schema = SCHEMAS[name]
    z = random_stacks(schema, 6, 1)
    y = oracle.compose(schema, z)
    for e in range(z.shape[1]):
        want = compose_stack(schema, z[:, e].astype(np.float64))
        scale = np.maximum(np.abs(want), np.sqrt(np.mean(want ** 2)))
        err = np.max(np.abs(y[:, e] - want) / scale)
        assert err < 2e-5, (name, e, err)


@pytest.mark.parametrize('name', list(SCHEMAS))
def test_sigma_prime_jet(name):
    """The jet of sigma'(z) (what the adjoint contracts with) against sigma(1-sigma)
    composed as a float64 series, and against the first column of the
    complex-step Jacobian of the composition (d y_alpha / d z_0)."""
    schema = SCHEMAS[name]
    z = random_stacks(schema, 4, 5)
    u = oracle.compose_prime(schema, z)
    for e in range(z.shape[1]):
        zz = z[:, e].astype(np.float64)
        for want in (compose_prime_stack(schema, zz), compose_jacobian(schema, zz)[:, 0]):
            scale = np.maximum(np.abs(want), np.sqrt(np.mean(want ** 2)))
            err = np.max(np.abs(u[:, e] - want) / scale)
            assert err < 2e-5, (name, e, err)


def test_sigma_closed_forms():
    """One variable, unit first derivative, zero higher input rows: row k is
    sigma^(k)(z) exactly (d^k/dz^k of 1/(1+e^-z), from float64 recurrences)."""
    schema = W.full_schema(1, 6)
    zs = np.linspace(-6, 6, 13)
    z = np.zeros((7, zs.size), np.float32)
    z[0], z[1] = zs, 1
    y = oracle.compose(schema, z)
    s = 1 / (1 + np.exp(-zs))
    # polynomial recurrence: sigma^(k+1) = P_k'(s) s (1-s) with sigma^(k) = P_k(s)
    P = np.polynomial.Polynomial([0, 1])
    ds = np.polynomial.Polynomial([0, 1, -1])
    for k in range(7):
        assert np.allclose(y[k], P(s), rtol=2e-5, atol=2e-6), k
        P = P.deriv() * ds


@pytest.mark.parametrize('name', list(SCHEMAS))
def test_adjoint_against_complex_step(name):
    schema = SCHEMAS[name]
    R = len(schema)
    z = random_stacks(schema, 3, 2)
    rng = np.random.default_rng(3)
    gy = rng.standard_normal((R, 3)).astype(np.float32)
    gz = oracle.compose_adjoint(schema, z, gy)
    for e in range(3):
        J = compose_jacobian(schema, z[:, e].astype(np.float64))
        want = J.T @ gy[:, e].astype(np.float64)
        scale = np.maximum(np.abs(want), np.sqrt(np.mean(want ** 2)))
        err = np.max(np.abs(gz[:, e] - want) / scale)
        assert err < 5e-5, (name, e, err)


def test_pair_tables_small_case():
    """dTab/Crs for {1, x, y, xx, xy}: the pair (x, xy) differs by y with C=1,
    (x, xx) by x with C=2 (cuda/cpde_engine.cuh:476-498)."""
    schema = W.closed_schema(2, [(2, 0), (1, 1)])   # rows: 1, y, x, xy, xx (counts (cx, cy))
    keys = [tuple(r[1:]) for r in schema]
    d, c = oracle.pair_tables(schema)
    i, j = keys.index((1, 0)), keys.index((2, 0))
    assert d[i, j] == keys.index((1, 0)) and c[i, j] == 2
    j = keys.index((1, 1))
    assert d[i, j] == keys.index((0, 1)) and c[i, j] == 1
    assert d[j, i] == -1


@pytest.mark.parametrize('ta,tb', [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_gemm_against_float64(ta, tb):
    rng = np.random.default_rng(4)
    m, n, k = 7, 9, 13
    A = rng.standard_normal((m, k)).astype(np.float32)
    B = rng.standard_normal((k, n)).astype(np.float32)
    C0 = rng.standard_normal((m, n)).astype(np.float32)
    a = (A.T if ta == 0 else A).copy()   # column-major storage of A (or of A^T when ta)
    b = (B.T if tb == 0 else B).copy()
    lda, ldb = (m if ta == 0 else k), (k if tb == 0 else n)
    got = oracle.gemm(ta, tb, m, n, k, 1.0, a, lda, b, ldb, 0.5, C0.T.copy(), m).reshape(n, m).T
    want = A.astype(np.float64) @ B.astype(np.float64) + 0.5 * C0
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5)


def test_matching_cost_direct():
    rng = np.random.default_rng(5)
    R, width, valid, samples, offset = 4, 6, 4, 10, 3
    y = rng.standard_normal((R, width, 1)).astype(np.float32)
    target = rng.standard_normal((R + 1, samples, 1)).astype(np.float32)
    trows = np.array([1, 0, 3, 4], np.int32)
    w = np.array([1.0, 0.0, 0.5, 2.0], np.float32).reshape(R, 1, 1)
    loss, g, bs, bc = oracle.matching(y, target, trows, w, 1, width, valid, offset, samples)
    r = y[:, :valid, 0].astype(np.float64) - target[trows, offset:offset + valid, 0]
    assert np.isclose(loss, np.sum(w[:, 0, 0, None] * r ** 2), rtol=1e-6)
    assert np.allclose(g[:, :valid, 0], 2 * w[:, 0, 0, None] * r, rtol=1e-6)
    assert np.all(g[:, valid:] == 0) and np.all(g[1] == 0)
    assert bs == 0x7fffffff
    y[2, 1, 0] = np.inf
    _, _, bs, bc = oracle.matching(y, target, trows, w, 1, width, valid, offset, samples)
    assert (bs, bc) == (offset + 1, -1)


def test_matching_cost_per_sample_weights_direct():
    """The [R][P][outputs] weight layout (weight_samples = P): the weight of
    (row d, chunk lane p, output o) is weights[d][offset + p][o] -- the sample
    index, not the lane -- and a zero weight drops the term and its gradient.
    Two outputs so that a swapped (sample, output) index also fails."""
    rng = np.random.default_rng(6)
    R, width, valid, samples, offset, outputs = 3, 5, 4, 11, 6, 2
    y = rng.standard_normal((R, width, outputs)).astype(np.float32)
    target = rng.standard_normal((R + 2, samples, outputs)).astype(np.float32)
    trows = np.array([4, 0, 2], np.int32)
    w = rng.uniform(0.5, 2.0, (R, samples, outputs)).astype(np.float32)
    w[1, offset + 2, 0] = 0
    w[:, offset + 1, :] = 0
    loss, g, bs, bc = oracle.matching(y, target, trows, w, samples, width, valid, offset, samples)
    ws = w[:, offset:offset + valid, :].astype(np.float64)
    r = y[:, :valid, :].astype(np.float64) - target[trows, offset:offset + valid, :]
    assert np.isclose(loss, np.sum(ws * r ** 2), rtol=1e-6)
    assert np.allclose(g[:, :valid, :], 2 * ws * r, rtol=1e-6)
    assert g[1, 2, 0] == 0 and np.all(g[:, 1, :] == 0) and np.all(g[:, valid:, :] == 0)
    # a lane-indexed weight (wp = p instead of offset + p) gives another loss
    lane = w[:, :valid, :].astype(np.float64)
    assert not np.isclose(loss, np.sum(lane * r ** 2), rtol=1e-3)
    assert bs == 0x7fffffff
    # the first bad component of the first bad sample: (row 2, output 1) at lane 3
    y[2, 3, 1] = np.inf
    _, _, bs, bc = oracle.matching(y, target, trows, w, samples, width, valid, offset, samples)
    assert (bs, bc) == (offset + 3, -1)


def test_rprop_known_answers():
    # bound rejection: w=19, step=100, previous -1, current gradient of (w-100)^2
    W_, S, ga, gi = oracle.rprop([19.0], [100.0], [2 * (19 - 100)], [-1.0])
    assert W_[0] == 19 and S[0] == np.float32(0.1) and ga[0] == 0
    # next epoch (buffers switched): gradient of (w-0)^2, previous cleared
    W_, S, ga, gi = oracle.rprop(W_, S, [2 * 19.0], ga)
    assert np.isclose(W_[0], 18.9, atol=1e-5)
    # the mirrored bound
    W_, S, ga, gi = oracle.rprop([-19.0], [100.0], [2 * (-19 + 100)], [1.0])
    assert W_[0] == -19 and S[0] == np.float32(0.1)
    # accepted step, then a sign reversal rolls it back with a halved step
    W_, S, ga, gi = oracle.rprop([0.5], [0.1], [2 * (0.5 - 1)], [0.0])
    assert np.isclose(W_[0], 0.6, atol=1e-6)
    W_, S, ga2, gi = oracle.rprop(W_, S, [2 * (W_[0] + 1)], ga)
    assert np.isclose(W_[0], 0.5, atol=1e-6) and np.isclose(S[0], 0.05) and ga2[0] == 0
    # zero gradient: nothing moves
    W_, S, ga, gi = oracle.rprop([0.0], [2.0], [0.0], [0.0])
    assert W_[0] == 0 and S[0] == 2


def test_restore_and_set_steps():
    floor = np.float32(1e-5)
    S, ga, gi = oracle.restore_steps(floor, [0, floor], [3, 4], [5, 6])
    assert list(S) == [floor, floor] and list(ga) == [0, 4] and list(gi) == [0, 6]
    S, ga, gi = oracle.restore_steps(floor, [floor / 2, 2 * floor], [3, 4], [5, 6])
    assert list(S) == [floor, 2 * floor] and list(ga) == [0, 4]
    S, ga, gi = oracle.set_steps(2e-4, [1, 2], [3, 4], [5, 6])
    assert np.all(S == np.float32(2e-4)) and not ga.any() and not gi.any()


def test_gradient_stats_known_answers():
    g = np.zeros(1100, np.float32)
    g[12], g[7] = 12, -5
    s = oracle.gradient_stats(g)
    assert s['squared_norm'] == 169 and s['max_abs'] == 12 and s['nonfinite'] == 0 and s['first'] == -1
    g[1025], g[1099] = np.nan, np.inf
    s = oracle.gradient_stats(g)
    assert s['nonfinite'] == 2 and s['first'] == 1025 and s['squared_norm'] == 169
