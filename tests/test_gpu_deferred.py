"""Backward passes that share a reduction launch (the protocol server defers
each pass's gradient reduction so that the next pass over the same network
joins it, and the scalar graph rides in it) against one launch per pass
(CPDE_DEFER_REDUCE=0): every frame and the final state byte for byte.  Cases:
the Poisson disk graph (two leaves with known multipliers), the nested
variation graph (value-dependent multipliers, three chunks per leaf: with the
one-pass epochs, with separate network launches, and on the table-driven and
layer-fused kernels), and two expression costs trained without a graph.
The same cases check one-pass expression epochs of two plans that share one
launch against separate launches, and training epochs in halves (the next
epoch's first passes sent before this epoch's scalars are back) against whole
epochs, with an epoch rejected after the next one's first half went out."""
import json
import os

import numpy as np
import pytest

from cpde_amd import wire, workloads as W
from cpde_amd.build import SERVER

pytestmark = pytest.mark.gpu


def canonical(events):
    out = []
    for e in events:
        item = []
        for k in sorted(e):
            v = e[k]
            if isinstance(v, np.ndarray):
                v = (v.dtype.str, v.shape, v.tobytes())
            elif isinstance(v, (list, tuple)):
                v = tuple(x.tobytes() if isinstance(x, np.ndarray) else x for x in v)
            item.append((k, v))
        out.append(tuple(item))
    return out


def run(env, body, trace):
    s = wire.Session(SERVER, env=dict(os.environ, CPDE_TRACE_FILE=str(trace), **env))
    try:
        result = body(s)
    finally:
        s.close()
    return result, json.loads(trace.read_text())


def poisson(s):
    pw = W.PoissonWorkload(radial=16, angular=16, boundary=64)
    ids = pw.upload(s)
    value, grads = s.graph_eval(ids['net'], ids['costs'], pw.graph(), gradient=True)
    res = s.train(ids['net'], ids['costs'], 6, method=0, fresh=1, log=1, graph=pw.graph())
    return value, [g.tobytes() for g in grads], canonical(res['events']), s.snapshot(ids['net'])


def nested(s):
    vw = W.VariationWorkload()
    n, _, costs = vw.upload(s)
    leaves = [costs['a'], costs['correction']]
    value, grads = s.graph_eval(n, leaves, vw.nested_graph(), gradient=True)
    res = s.train(n, leaves, 5, method=0, fresh=1, log=1, graph=vw.nested_graph())
    return value, [g.tobytes() for g in grads], canonical(res['events']), s.snapshot(n)


def two_costs(s):
    vw = W.VariationWorkload()
    n, _, costs = vw.upload(s)
    res = s.train(n, [costs['a'], costs['free']], 5, method=0, fresh=1, log=1)
    return canonical(res['events']), s.snapshot(n)


@pytest.mark.parametrize('name,body,env', [
    ('poisson', poisson, {}),
    ('nested', nested, {}),
    ('nested-separate', nested, {'CPDE_ONE_PASS': '0'}),
    ('nested-table', nested, {'CPDE_FUSED': '0'}),             # table-driven kernels
    ('nested-layer', nested, {'CPDE_FUSED': '1'}),             # layer-fused kernels
    ('two-costs', two_costs, {}),
])
def test_shared_reductions_match_one_per_pass(tmp_path, name, body, env):
    shared, t1 = run(env, body, tmp_path / 'shared.json')
    alone, t0 = run(dict(env, CPDE_DEFER_REDUCE='0'), body, tmp_path / 'alone.json')
    launches = [t['split_reduce'][0] for t in (t1, t0)]
    print(f'[result] {name}: reduction launches shared {launches[0]} alone {launches[1]}', flush=True)
    assert shared == alone
    assert launches[0] < launches[1]


@pytest.mark.parametrize('name,body', [('poisson', poisson), ('nested', nested), ('two-costs', two_costs)])
def test_paired_epochs_match_separate_launches(tmp_path, name, body):
    """One-pass expression epochs of two plans in one launch (the first held
    back while reductions are deferred) against each in its own launch
    (CPDE_EPOCH_PAIRS=0): every frame and the final state byte for byte, and
    on the Poisson graph half the network-epoch launches."""
    paired, t1 = run({}, body, tmp_path / 'paired.json')
    alone, t0 = run({'CPDE_EPOCH_PAIRS': '0'}, body, tmp_path / 'alone.json')
    launches = [t['network_epoch'][0] for t in (t1, t0)]
    print(f'[result] {name}: network epoch launches paired {launches[0]} alone {launches[1]}', flush=True)
    assert paired == alone
    if name == 'poisson':
        assert launches[0] < launches[1]


def run_counted(env, body, counts):
    s = wire.Session(SERVER, env=dict(os.environ, CPDE_REPLAY_FILE=str(counts), **env))
    try:
        result = body(s)
    finally:
        s.close()
    return result, json.loads(counts.read_text())


def rejected_at_epoch_one(method, diagnostics=1):
    """u = w x + b on one point, w = 0, b = 1, cost (k u)^2: epoch 0 is clean;
    its update moves w, so epoch 1 overflows and is rejected -- after epoch
    1's first passes went out behind epoch 0's update.  RPROP: x = 1e30, k = 1
    (epoch 0: dE/dw 2e30; epoch 1's objective overflows).  Adam: x = 1e22,
    k^2 = 5e-4 (epoch 0: dE/dw 1e19, whose square Adam's second moment still
    holds; a first step of about lr makes epoch 1's dE/dw about -1e39).
    diagnostics=0: the update launches test the gradients themselves, and the
    rejected epoch's report takes its statistics afterwards."""
    x, k = (1e30, 1.0) if method == 0 else (1e22, np.sqrt(5e-4))

    def body(s):
        n = s.network([1, 1], [1, 1], [np.array([0.0, 1.0], np.float32)])
        d = s.data(np.array([[[x]]], np.float32), np.array([[0, 0]], np.int32))
        c = s.polynomial_cost(n, d, [0], 1, [[0, 0, -1]], np.full((1, 1), k, np.float32),
                              np.zeros((1, 1), np.float32), np.ones((1, 1), np.float32))
        with pytest.raises(wire.ServerError) as err:
            s.train(n, [c], 4, method=method, fresh=1, lr=0.01, log=1, diagnostics=diagnostics)
        return str(err.value), canonical(err.value.events), s.snapshot(n)
    return body


SQUARE = ([(1, 0, 0), (7, 0, -1)], [0.0, 2.0])  # u ** 2 (scalar ops Component 1, Power 7)


def rejected_integrals(method, layout, diagnostics=1):
    """u = w x + b (w = 0, b = 1) under integral costs q u**2: epoch 0 is clean;
    its update moves w, so epoch 1's dE/dw = 2 u q x overflows in fp32 and is
    rejected, after epoch 2's first half went out behind epoch 1's update.
    That first half launches reductions before its scalars are back:
      * 'graph': two leaves summed by a graph, which rides in the reduction
        and launches it;
      * 'chunks': one leaf over three samples in one-sample chunks, whose third
        backward pass launches the first two's reduction.
    RPROP: x = 1e30, q = 1.  Adam: x = 1e22 and q = 5e-4 / samples, so that
    epoch 0's dE/dw is 1e19, whose square Adam's second moment still holds,
    and a first step of about lr gives epoch 1 a dE/dw of about -1e39.
    diagnostics=0: as in rejected_at_epoch_one."""
    samples = 2 if layout == 'graph' else 3
    x, q = (1e30, 1.0) if method == 0 else (1e22, 5e-4 / samples)

    def body(s):
        n = s.network([1, 1], [1, 1], [np.array([0.0, 1.0], np.float32)])
        table = np.array([[0, 0]], np.int32)
        if layout == 'graph':
            ds = [s.data(np.array([[[x]]], np.float32), table) for _ in range(2)]
            costs = [s.integral_cost(n, d, *SQUARE, np.zeros((0, 1)), [q]) for d in ds]
            graph = W.PoissonWorkload.graph()
        else:
            d = s.data(np.full((1, 1, 3), x, np.float32), table)
            costs = [s.integral_cost(n, d, *SQUARE, np.zeros((0, 3)), [q] * 3, chunk=1)]
            graph = None
        with pytest.raises(wire.ServerError) as err:
            s.train(n, costs, 6, method=method, fresh=1, lr=0.01, log=1, diagnostics=diagnostics, graph=graph)
        return str(err.value), canonical(err.value.events), s.snapshot(n)
    return body


def two_costs_adam(s):
    vw = W.VariationWorkload()
    n, _, costs = vw.upload(s)
    res = s.train(n, [costs['a'], costs['free']], 5, method=1, fresh=1, lr=0.01, log=1)
    return canonical(res['events']), s.snapshot(n)


@pytest.mark.parametrize('name,body', [('poisson', poisson), ('nested', nested), ('two-costs', two_costs),
                                       ('two-costs-adam', two_costs_adam),
                                       ('rejected', rejected_at_epoch_one(0)),
                                       ('rejected-adam', rejected_at_epoch_one(1)),
                                       ('rejected-graph', rejected_integrals(0, 'graph')),
                                       ('rejected-graph-adam', rejected_integrals(1, 'graph')),
                                       ('rejected-chunks', rejected_integrals(0, 'chunks')),
                                       ('rejected-chunks-adam', rejected_integrals(1, 'chunks')),
                                       ('rejected-short', rejected_at_epoch_one(0, 0)),
                                       ('rejected-graph-short', rejected_integrals(0, 'graph', 0)),
                                       ('rejected-chunks-adam-short', rejected_integrals(1, 'chunks', 0))])
def test_epochs_in_halves_match_whole_epochs(tmp_path, name, body):
    """Training (RPROP and Adam) with each epoch's first passes sent before
    the previous epoch's scalars are back (its update guarded on the device)
    against whole epochs (CPDE_EPOCH_HALVES=0): every frame, the final state
    (all four buffers of every transition) and, for a rejected epoch, the
    error byte for byte; first halves were sent ahead."""
    halves, c1 = run_counted({}, body, tmp_path / 'halves.json')
    whole, c0 = run_counted({'CPDE_EPOCH_HALVES': '0'}, body, tmp_path / 'whole.json')
    print(f'[result] {name}: first halves sent ahead {c1["ahead"]} (whole epochs {c0["ahead"]})', flush=True)
    if name.startswith('rejected'):
        print(f'[result] {name}: {halves[0]}', flush=True)
        meta, _ = wire.decode_state(bytes(halves[2]))
        assert meta['updates'] == 1
    assert halves == whole
    assert c1['ahead'] > 0 and c0['ahead'] == 0


def test_stop_with_halves_leaves_the_state_of_whole_epochs(tmp_path):
    """op 99 sent on the first report of a long call with nothing that keeps
    the next first half back (no saves, evaluations or restores): the call
    stops after some small number of epochs k -- one more than whole epochs
    would run when the next epoch's first half was already out, as if the
    stop had arrived during that epoch -- and the state is byte for byte that
    of k whole epochs (the metadata's remaining count aside)."""
    def stopped(s):
        vw = W.VariationWorkload()
        n, _, costs = vw.upload(s)

        def on_event(session, ev):
            if ev['kind'] == 6 and not getattr(session, '_stop_sent', False):
                session._stop_sent = True
                session.stop()
        res = s.train(n, [costs['a'], costs['correction']], 100000, method=0, fresh=1, log=1,
                      graph=vw.nested_graph(), on_event=on_event)
        return res['completed'], res['stopped'], s.snapshot(n)

    (k, flag, blob), counts = run_counted({}, stopped, tmp_path / 'stopped.json')
    print(f'[result] stopped after {k} epochs, first halves sent ahead {counts["ahead"]}', flush=True)
    assert flag == 1 and 1 <= k < 100000
    meta, _ = wire.decode_state(bytes(blob))
    assert meta['updates'] == k

    def whole(s):
        vw = W.VariationWorkload()
        n, _, costs = vw.upload(s)
        res = s.train(n, [costs['a'], costs['correction']], k, method=0, fresh=1, log=1, graph=vw.nested_graph())
        return res['completed'], s.snapshot(n)

    (k0, blob0), _ = run_counted({'CPDE_EPOCH_HALVES': '0'}, whole, tmp_path / 'whole.json')
    assert k0 == k
    (m1, l1), (m0, l0) = wire.decode_state(bytes(blob)), wire.decode_state(bytes(blob0))
    assert m1.pop('remaining') == 100000 - k and m0.pop('remaining') == 0
    assert m1 == m0
    for a, b in zip(l1, l0):
        assert a['active'] == b['active']
        for x, y in zip(a['buffers'], b['buffers']):
            assert x.tobytes() == y.tobytes()
