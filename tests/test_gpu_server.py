"""The MI355X protocol server against the reference CPU server's golden vectors,
over the wire protocol exactly as the reference's Python client drives it.

Bars: objectives relative 1e-4, gradients and outputs relative L2 1e-3 (the
order-6 bars); RPROP weights bit-identical wherever the reference gradient
exceeds 1e-3 of its largest entry; state blobs identical in their metadata."""
import numpy as np
import pytest

from cpde_amd import wire
from cpde_amd.build import SERVER
from helpers import golden_workload, load_golden, rel_l2

pytestmark = pytest.mark.gpu

SINGLE_LEAF = wire.graph_bytes([(1, 0, 0)], [0.0], 0)


@pytest.fixture(scope='module')
def server():
    if not SERVER.exists():
        pytest.fail('protocol server not built: python -m cpde_amd.build')
    s = wire.Session(SERVER)
    yield s
    s.close()


def check_sure_weights(after, ref_after, ref_grad):
    sure = np.abs(ref_grad) > 1e-3 * np.abs(ref_grad).max()
    np.testing.assert_array_equal(after[sure], ref_after[sure])


def test_matching_cost_gradient_outputs_and_first_update(server):
    g = load_golden('tiny_order6')
    wl = golden_workload(g)
    ids = wl.upload(server, 0)
    value, grads = server.graph_eval(ids['net'], [ids['cost']], SINGLE_LEAF, gradient=True)
    print(f'[result] loss {value!r} reference {float(g["loss"])!r}', flush=True)
    assert abs(value / g['loss'] - 1) < 1e-4
    for t, grad in enumerate(grads):
        assert rel_l2(grad, g[f'grad{t}']) < 1e-3
    out = server.eval(ids['net'], ids['data'], 0)
    outputs = server.download(out).reshape(wl.rows, wl.size, 1)
    assert max(rel_l2(outputs[r], g['outputs'][r]) for r in range(wl.rows)) < 1e-3
    res = server.train(ids['net'], [ids['cost']], 1, method=0, fresh=1, log=1)
    assert res['completed'] == 1 and res['stopped'] == 0
    meta, layers = wire.decode_state(server.snapshot(ids['net']))
    assert meta['updates'] == 1 and meta['optimizer'] == 0
    for t, layer in enumerate(layers):
        check_sure_weights(layer['buffers'][0], g[f'after{t}'], g[f'grad{t}'])
        assert layer['active'] == int(g[f'active{t}'])


def test_chunked_cost(server):
    g = load_golden('tiny_order6')
    wl = golden_workload(g)
    ids = wl.upload(server, 7)
    value, grads = server.graph_eval(ids['net'], [ids['cost']], SINGLE_LEAF, gradient=True)
    assert abs(value / g['chunk7_loss'] - 1) < 1e-4
    for t, grad in enumerate(grads):
        assert rel_l2(grad, g[f'chunk7_grad{t}']) < 1e-3


def test_expression_costs_and_graph(server):
    """Poisson on the disk: (u_xx + u_yy + f)^2 over quadrature points plus u^2 on
    the boundary, compiled with hipRTC, combined by the scalar cost graph."""
    from cpde_amd import workloads as W
    g = load_golden('poisson')
    pw = W.PoissonWorkload(radial=int(g['radial']), angular=int(g['angular']), boundary=int(g['boundary']))
    ids = pw.upload(server)
    value, grads = server.graph_eval(ids['net'], ids['costs'], pw.graph(), gradient=True)
    print(f'[result] poisson objective {value!r} reference {float(g["loss"])!r}', flush=True)
    assert abs(value / g['loss'] - 1) < 1e-4
    for t, grad in enumerate(grads):
        assert rel_l2(grad, g[f'grad{t}']) < 1e-3
    for leaf in range(2):
        v, _ = server.graph_eval(ids['net'], [ids['costs'][leaf]], SINGLE_LEAF, gradient=False)
        assert abs(v / g[f'leaf{leaf}'] - 1) < 1e-4
    source, _ = server.inspect(ids['costs'][0], compile=True)
    assert 'expression' in source


def test_one_pass_expression_epoch_matches_separate_launches(server):
    """The Poisson objective and gradient with the one-pass expression epoch
    (forward, per-sample expression and backward in one launch per leaf) against
    a second server that runs them as separate launches (CPDE_ONE_PASS=0): the
    same adjoint and backward, so bit-identical gradients; the objective
    differs only in its fp64 summation order.  Then three RPROP epochs on each,
    whose weights must stay bit-identical."""
    import os
    from cpde_amd import workloads as W
    g = load_golden('poisson')
    pw = W.PoissonWorkload(radial=int(g['radial']), angular=int(g['angular']), boundary=int(g['boundary']))
    separate = wire.Session(SERVER, env=dict(os.environ, CPDE_ONE_PASS='0'))
    try:
        results = []
        for s in (server, separate):
            ids = pw.upload(s)
            value, grads = s.graph_eval(ids['net'], ids['costs'], pw.graph(), gradient=True)
            s.train(ids['net'], ids['costs'], 3, method=0, fresh=1, log=1, graph=pw.graph())
            results.append((value, grads, wire.decode_state(s.snapshot(ids['net']))))
    finally:
        separate.close()
    (v1, g1, st1), (v2, g2, st2) = results
    print(f'[result] one-pass objective {v1!r} separate {v2!r}', flush=True)
    assert abs(v1 / v2 - 1) < 1e-12
    for a, b in zip(g1, g2):
        np.testing.assert_array_equal(a, b)
    assert st1[0] == st2[0]
    for a, b in zip(st1[1], st2[1]):
        np.testing.assert_array_equal(a['buffers'][0], b['buffers'][0])


def test_paired_aliased_expression_epoch(server):
    """The Poisson objective on a server whose network kernels are forced to
    two points per workgroup with one LDS tile (the one-pass expression epoch
    then keeps its per-point double and flag records in a scratch apart from
    the tiles): the reference's objective and gradients, and the same
    gradients as the default form to the fp32 bar."""
    import os
    from cpde_amd import workloads as W
    g = load_golden('poisson')
    pw = W.PoissonWorkload(radial=int(g['radial']), angular=int(g['angular']), boundary=int(g['boundary']))
    forced = wire.Session(SERVER, env=dict(os.environ, CPDE_FUSED='2', CPDE_NET_POINTS='2', CPDE_NET_ALIAS='1',
                                           CPDE_NET_COLTILE='16', CPDE_NET_SPLIT='1', CPDE_NET_SPLIT_ADJOINT='1'))
    try:
        ids = pw.upload(forced)
        value, grads = forced.graph_eval(ids['net'], ids['costs'], pw.graph(), gradient=True)
    finally:
        forced.close()
    print(f'[result] paired aliased poisson objective {value!r} reference {float(g["loss"])!r}', flush=True)
    assert abs(value / g['loss'] - 1) < 1e-4
    for t, grad in enumerate(grads):
        assert rel_l2(grad, g[f'grad{t}']) < 1e-3


def test_graph_without_leaf_dependence_zeroes_the_gradient(server):
    """A root that depends on no leaf: every multiplier is known to be 0, no
    leaf runs a backward pass, and the gradient must come back zero although
    the previous evaluation left a nonzero one (the only case in which the
    server still zero-fills before the passes)."""
    from cpde_amd import workloads as W
    g = load_golden('poisson')
    pw = W.PoissonWorkload(radial=int(g['radial']), angular=int(g['angular']), boundary=int(g['boundary']))
    ids = pw.upload(server)
    _, grads = server.graph_eval(ids['net'], ids['costs'], pw.graph(), gradient=True)
    assert all(np.abs(x).max() > 0 for x in grads)
    constant = wire.graph_bytes([(1, 0, 0), (1, 1, 0), (0, 0, 0)], [0.0, 0.0, 5.0], 2)
    value, grads = server.graph_eval(ids['net'], ids['costs'], constant, gradient=True)
    assert value == 5.0
    for x in grads:
        np.testing.assert_array_equal(x, np.zeros_like(x))


def test_value_dependent_graph_multipliers(server):
    """root = leaf0 / leaf1 + log(leaf0) + leaf1 ** 1.5: the leaf multipliers are
    known only after the forward passes, so every leaf runs a second, backward
    pass scaled by its multiplier (one leaf reusing its last forward chunk).
    Objective, gradients, two training epochs' reports and the final state
    against the reference server."""
    from cpde_amd import workloads as W
    g = load_golden('poisson')
    pw = W.PoissonWorkload(radial=int(g['radial']), angular=int(g['angular']), boundary=int(g['boundary']))
    graph = W.PoissonWorkload.value_dependent_graph()
    ids = pw.upload(server)
    value, grads = server.graph_eval(ids['net'], ids['costs'], graph, gradient=True)
    print(f'[result] objective {value!r} reference {float(g["vgraph_loss"])!r}', flush=True)
    assert abs(value / g['vgraph_loss'] - 1) < 1e-4
    for t, grad in enumerate(grads):
        assert rel_l2(grad, g[f'vgraph_grad{t}']) < 1e-3
    res = server.train(ids['net'], ids['costs'], 2, method=0, fresh=1, log=1, graph=graph)
    reports = np.asarray([(e['completed'], e['updates'], e['after'], e['total']) for e in res['events']
                          if e['kind'] == 6])
    assert reports.shape == g['vgraph_reports'].shape
    np.testing.assert_array_equal(reports[:, :3], g['vgraph_reports'][:, :3])
    np.testing.assert_allclose(reports[:, 3], g['vgraph_reports'][:, 3], rtol=1e-4)
    ours = wire.decode_state(server.snapshot(ids['net']))
    ref = wire.decode_state(bytes(g['vgraph_state']))
    assert ours[0] == ref[0]
    for a, b in zip(ours[1], ref[1]):
        assert rel_l2(a['buffers'][0], b['buffers'][0]) < 1e-5


def test_polynomial_cost(server):
    g = load_golden('polynomial')
    schema = g['schema']
    from cpde_amd import workloads as W
    inputs = W.input_stack(g['points'], schema)
    neurons = list(g['neurons'])
    T = len(neurons) - 1
    d = server.data(inputs, schema)
    n = server.network(neurons, W.linear_flags(neurons), [g[f'init{t}'] for t in range(T)])
    c = server.polynomial_cost(n, d, list(range(len(schema))), 2, g['terms'], g['coeffs'], g['rhs'], g['weights'],
                               chunk=int(g['chunk']))
    value, grads = server.graph_eval(n, [c], SINGLE_LEAF, gradient=True)
    assert abs(value / g['loss'] - 1) < 1e-4
    for t, grad in enumerate(grads):
        assert rel_l2(grad, g[f'grad{t}']) < 1e-3
    server.train(n, [c], 1, method=0, fresh=1, log=1)
    _, layers = wire.decode_state(server.snapshot(n))
    for t, layer in enumerate(layers):
        check_sure_weights(layer['buffers'][0], g[f'after{t}'], g[f'grad{t}'])


def test_training_reports_diagnostics_and_adam(server):
    g = load_golden('training')
    wl = golden_workload(g)
    ids = wl.upload(server, int(g['chunk']))
    res = server.train(ids['net'], [ids['cost']], 3, method=0, fresh=1, log=1, diagnostics=1, eval_every=2)
    reports = np.asarray([(e['completed'], e['updates'], e['after'], e['values'][0]) for e in res['events']
                          if e['kind'] == 2])
    assert reports.shape == g['reports'].shape
    np.testing.assert_array_equal(reports[:, :3], g['reports'][:, :3])
    np.testing.assert_allclose(reports[:, 3], g['reports'][:, 3], rtol=1e-4)
    diag = np.asarray([(e['epoch'], e['layers'][0]['sq'], e['layers'][0]['max']) for e in res['events']
                       if e['kind'] == 5])
    np.testing.assert_array_equal(diag[:, 0], g['diagnostics'][:, 0])
    np.testing.assert_allclose(diag[:, 1:], g['diagnostics'][:, 1:], rtol=2e-3)
    ours = wire.decode_state(server.snapshot(ids['net']))
    ref = wire.decode_state(bytes(g['rprop_state']))
    assert ours[0] == ref[0]
    for a, b in zip(ours[1], ref[1]):
        assert a['active'] == b['active']
        assert rel_l2(a['buffers'][0], b['buffers'][0]) < 1e-5
    # Adam from a fresh network
    ids2 = wl.upload(server, int(g['chunk']))
    res2 = server.train(ids2['net'], [ids2['cost']], 2, method=1, fresh=1, lr=0.01, log=1)
    adam = np.asarray([(e['completed'], e['updates'], e['after'], e['values'][0]) for e in res2['events']
                       if e['kind'] == 2])
    np.testing.assert_array_equal(adam[:, :3], g['adam_reports'][:, :3])
    np.testing.assert_allclose(adam[:, 3], g['adam_reports'][:, 3], rtol=1e-4)
    ours = wire.decode_state(server.snapshot(ids2['net']))
    ref = wire.decode_state(bytes(g['adam_state']))
    assert ours[0] == ref[0]
    for a, b in zip(ours[1], ref[1]):
        assert rel_l2(a['buffers'][0], b['buffers'][0]) < 1e-4


def test_restore_reference_checkpoint(server):
    """A state blob written by the reference server restores here and reads back
    byte for byte."""
    g = load_golden('training')
    wl = golden_workload(g)
    ids = wl.upload(server, int(g['chunk']))
    blob = bytes(g['rprop_state'])
    server.restore(ids['net'], blob)
    assert server.snapshot(ids['net']) == blob


def test_timing_command_matches_evaluation(server):
    g = load_golden('tiny_order6')
    wl = golden_workload(g)
    ids = wl.upload(server, 0)
    r = server.timing(ids['net'], ids['cost'], warm=2, iterations=5, batches=2, layers=len(wl.neurons) - 1)
    assert len(r['wall_ms']) == 2 and all(t > 0 for t in r['gpu_ms'])
    assert abs(r['loss'] / g['loss'] - 1) < 1e-4
    for t, grad in enumerate(r['gradients']):
        assert rel_l2(grad, g[f'grad{t}']) < 1e-3


def test_close_semantics(server):
    g = load_golden('tiny_order6')
    ids = golden_workload(g).upload(server, 0)
    with pytest.raises(wire.ServerError, match='retained by a cost'):
        server.close_object(0, ids['data'])
    with pytest.raises(wire.ServerError, match='retained by a cost'):
        server.close_object(1, ids['net'])
    server.close_object(2, ids['cost'])
    server.close_object(0, ids['data'])
    server.close_object(1, ids['net'])
    with pytest.raises(wire.ServerError, match='unknown or released'):
        server.snapshot(ids['net'])


def test_nonfinite_objective_is_rejected_and_state_kept(server):
    """A non-finite objective stops training before the optimizer: weights,
    steps and counters stay as they were, and the session stays usable."""
    g = load_golden('tiny_order6')
    wl = golden_workload(g)
    ids = wl.upload(server, 0)
    server.train(ids['net'], [ids['cost']], 1, method=0, fresh=1, log=1)
    meta0, before = wire.decode_state(server.snapshot(ids['net']))
    bad = wl.inputs.copy()
    bad[0, 0, 3] = np.nan
    server.replace(ids['data'], bad)
    with pytest.raises(wire.ServerError, match='non-finite'):
        server.train(ids['net'], [ids['cost']], 1, method=0, fresh=0, log=1)
    meta1, after = wire.decode_state(server.snapshot(ids['net']))
    assert meta1['updates'] == meta0['updates']
    for a, b in zip(before, after):
        np.testing.assert_array_equal(a['buffers'][0], b['buffers'][0])
        np.testing.assert_array_equal(a['buffers'][3], b['buffers'][3])
    server.replace(ids['data'], wl.inputs)
    res = server.train(ids['net'], [ids['cost']], 1, method=0, fresh=0, log=1)
    assert res['completed'] == 1
