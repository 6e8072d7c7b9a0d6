"""Attached variations, frozen components and the full-size Poisson graph on
the MI355X server against the reference CPU server
(tests/golden/variations.npz, tests/golden/poisson_full.npz).

* A frozen component (expression IR Component with b = 1) contributes its
  value but no adjoint (cuda/expression_program.hpp:46); a leaf whose
  components are all frozen has a zero gradient.
* Attach (graph op 15) passes the first operand's value and both operands'
  adjoints (cuda/cost_graph.cuh:13-14,22-23): a variation cancelled by its
  own negation keeps its value with a zero gradient
  (tests/test_audit_fixes.py:69-77); nested variations with shared leaves
  have value-dependent multipliers (tests/test_integrals.py:176-186).

Bars: objectives relative 1e-4, gradients relative L2 1e-3; structural zeros
exact."""
import numpy as np
import pytest

from cpde_amd import wire, workloads as W
from cpde_amd.build import SERVER
from helpers import checksum, load_golden, rel_l2

pytestmark = pytest.mark.gpu

SINGLE_LEAF = wire.graph_bytes([(1, 0, 0)], [0.0], 0)


@pytest.fixture(scope='module')
def server():
    if not SERVER.exists():
        pytest.fail('protocol server not built: python -m cpde_amd.build')
    s = wire.Session(SERVER)
    yield s
    s.close()


def check(value, grads, g, key):
    print(f'[result] {key} {value!r} reference {float(g[f"{key}_value"])!r}', flush=True)
    assert abs(value / g[f'{key}_value'] - 1) < 1e-4
    for t, grad in enumerate(grads):
        ref = g[f'{key}_grad{t}']
        if not ref.any():
            np.testing.assert_array_equal(grad, 0)
        else:
            assert rel_l2(grad, ref) < 1e-3, (key, t)


@pytest.mark.parametrize('name', ['a', 'correction', 'frozen', 'free'])
def test_leaves_with_frozen_components(server, name):
    g = load_golden('variations')
    vw = W.VariationWorkload()
    n, d, costs = vw.upload(server)
    value, grads = server.graph_eval(n, [costs[name]], SINGLE_LEAF, gradient=True)
    check(value, grads, g, name)
    if name == 'frozen':
        # u**2 with u frozen: the value of u**2, no gradient at all
        free, _ = server.graph_eval(n, [costs['free']], SINGLE_LEAF, gradient=False)
        assert value == free
        for grad in grads:
            np.testing.assert_array_equal(grad, 0)


def test_cancelled_variation_keeps_value_with_zero_gradient(server):
    g = load_golden('variations')
    vw = W.VariationWorkload()
    n, d, costs = vw.upload(server)
    value, grads = server.graph_eval(n, [costs['a']], vw.cancelled_graph(), gradient=True)
    check(value, grads, g, 'cancelled')
    a, _ = server.graph_eval(n, [costs['a']], SINGLE_LEAF, gradient=False)
    assert value == a
    for grad in grads:
        np.testing.assert_array_equal(grad, 0)


def test_nested_variations_with_shared_leaves(server):
    """(a*a).with_variation(correction.with_variation(a)) + correction + a:
    value A^2 + B + A, gradient (2A + 2) grad a + 2 grad b (B's u_x frozen)."""
    g = load_golden('variations')
    vw = W.VariationWorkload()
    n, d, costs = vw.upload(server)
    value, grads = server.graph_eval(n, [costs['a'], costs['correction']], vw.nested_graph(), gradient=True)
    check(value, grads, g, 'nested')
    A, ga = server.graph_eval(n, [costs['a']], SINGLE_LEAF, gradient=True)
    B, gb = server.graph_eval(n, [costs['correction']], SINGLE_LEAF, gradient=True)
    assert value == pytest.approx(A * A + B + A, rel=1e-12)
    for t, grad in enumerate(grads):
        assert rel_l2(grad, (2 * A + 2) * ga[t].astype(np.float64) + 2 * gb[t].astype(np.float64)) < 1e-6
    res = server.train(n, [costs['a'], costs['correction']], 2, method=0, fresh=1, log=1, graph=vw.nested_graph())
    reports = np.asarray([(e['completed'], e['updates'], e['after'], e['total']) for e in res['events']
                          if e['kind'] == 6])
    np.testing.assert_array_equal(reports[:, :3], g['nested_reports'][:, :3])
    np.testing.assert_allclose(reports[:, 3], g['nested_reports'][:, 3], rtol=1e-4)
    ours = wire.decode_state(server.snapshot(n))
    ref = wire.decode_state(bytes(g['nested_state']))
    assert ours[0] == ref[0]
    for a, b in zip(ours[1], ref[1]):
        assert rel_l2(a['buffers'][0], b['buffers'][0]) < 1e-5


def test_poisson_at_full_size(server):
    """The Poisson workload at its full size (64 x 64 interior quadrature
    points, 256 boundary points): objective, both leaves, gradient, and two
    RPROP epochs (reports and state)."""
    g = load_golden('poisson_full')
    pw = W.PoissonWorkload()
    got = np.stack([checksum(pw.interior), checksum(pw.interior_w), checksum(pw.boundary), checksum(pw.f),
                    checksum(np.concatenate(pw.init))])
    assert np.allclose(got, g['checksums'], rtol=1e-12, atol=0), 'workload generator drifted'
    ids = pw.upload(server)
    value, grads = server.graph_eval(ids['net'], ids['costs'], pw.graph(), gradient=True)
    print(f'[result] poisson objective {value!r} reference {float(g["loss"])!r}', flush=True)
    assert abs(value / g['loss'] - 1) < 1e-4
    for t, grad in enumerate(grads):
        e = rel_l2(grad, g[f'grad{t}'])
        print(f'[result] transition {t} gradient rel-L2 {e:.3e}', flush=True)
        assert e < 1e-3
    for leaf in range(2):
        v, _ = server.graph_eval(ids['net'], [ids['costs'][leaf]], SINGLE_LEAF, gradient=False)
        assert abs(v / g[f'leaf{leaf}'] - 1) < 1e-4
    res = server.train(ids['net'], ids['costs'], 2, method=0, fresh=1, steps=2e-4, log=1, graph=pw.graph())
    reports = np.asarray([(e['completed'], e['updates'], e['after'], e['total']) for e in res['events']
                          if e['kind'] == 6])
    np.testing.assert_array_equal(reports[:, :3], g['reports'][:, :3])
    np.testing.assert_allclose(reports[:, 3], g['reports'][:, 3], rtol=1e-4)
    ours = wire.decode_state(server.snapshot(ids['net']))
    ref = wire.decode_state(bytes(g['state']))
    assert ours[0] == ref[0]
    for a, b in zip(ours[1], ref[1]):
        assert rel_l2(a['buffers'][0], b['buffers'][0]) < 1e-5


def run_nested(env, trace=None):
    """Value, gradients and a two-epoch RPROP state of the nested-variation
    graph (three chunks per leaf) in a fresh server with `env`; the server's
    per-kernel launch counts when `trace` names a file."""
    import json
    import os
    extra = dict(env)
    if trace:
        extra['CPDE_TRACE_FILE'] = str(trace)
    s = wire.Session(SERVER, env=dict(os.environ, **extra))
    try:
        vw = W.VariationWorkload()
        n, d, costs = vw.upload(s)
        value, grads = s.graph_eval(n, [costs['a'], costs['correction']], vw.nested_graph(), gradient=True)
        s.train(n, [costs['a'], costs['correction']], 2, method=0, fresh=1, log=1, graph=vw.nested_graph())
        state = s.snapshot(n)
    finally:
        s.close()
    launches = json.loads(trace.read_text()) if trace else None
    return value, grads, state, launches


def test_retained_forwards_match_recomputed(tmp_path):
    """Leaves with value-dependent multipliers keep every chunk's forward in a
    stack set of its own until their backward, instead of recomputing it as
    the reference does (CPDE_RETAIN_MB=0), unless their backward runs as one
    launch with a small forward inside it.  With the one-launch epochs off
    (CPDE_ONE_PASS=0) this graph's leaves keep their forwards: fewer forward
    launches, the same value, and the gradient to rounding (the recomputing
    run sums the chunks' backwards in another order: it starts with the last
    chunk of its costliest leaf, whose forward is still in place).  With them
    on, both runs recompute."""
    for serial in ({'CPDE_ONE_PASS': '0'}, {}):
        kept = run_nested(serial, tmp_path / 'kept.json')
        again = run_nested(dict(serial, CPDE_RETAIN_MB='0'), tmp_path / 'again.json')
        assert kept[0] == again[0]
        for a, b in zip(kept[1], again[1]):
            assert rel_l2(a, b) < 1e-6
        ours, theirs = wire.decode_state(kept[2]), wire.decode_state(again[2])
        assert ours[0] == theirs[0]
        for a, b in zip(ours[1], theirs[1]):
            assert rel_l2(a['buffers'][0], b['buffers'][0]) < 1e-6
        forwards = [sum(v[0] for k, v in r[3].items() if k in ('network_forward', 'fused_forward', 'gemm_forward'))
                    for r in (kept, again)]
        print(f'[result] {serial} forward launches retained {forwards[0]} recomputed {forwards[1]}', flush=True)
        if serial:
            assert forwards[0] < forwards[1]
