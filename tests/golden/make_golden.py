"""Writes the golden vectors under tests/golden/ by driving the reference CPU
server (built from the reference sources by ``make -C oracle ref``) through this
package's own wire client.  Run in a container that has the reference tree:

    make -C oracle ref && python tests/golden/make_golden.py [case ...]

Each case is one .npz with the inputs that define it (network, schema, points,
targets, weights) and the server's answers:
  * ``loss``, ``grad{t}``  - op 14 (graph evaluation with gradient) at the
                             initial weights: forward + cost + weight gradient
                             (cuda/cpde_server.cu:535-551);
  * ``outputs``            - op 4 evaluation + op 5 download, [row][sample][out];
  * ``after{t}``/``step{t}`` - weights and RPROP steps after one op-8 training
                             epoch from a fresh optimizer state, via op 9;
  * ``published_losses``   - the losses of the reference's Fourier benchmark
                             workload at orders 0..6.
"""
from __future__ import annotations

import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(HERE))

from cpde_amd import wire, workloads as W  # noqa: E402
from published_workload import PUBLISHED_LOSSES, reference_benchmark  # noqa: E402

SERVER = ROOT / 'oracle' / '_ref' / 'cpde_cpu_server'
SINGLE_LEAF = wire.graph_bytes([(1, 0, 0)], [0.0], 0)


def session():
    if not SERVER.exists():
        raise SystemExit(f'{SERVER} missing: run make -C oracle ref')
    return wire.Session(SERVER)


def checksum(a):
    a = np.asarray(a, np.float64).ravel()
    return np.array([a.size, a.sum(), (a * a).sum(), (a * np.arange(a.size) / max(a.size, 1)).sum()])


PROBES = 64


def probes(count, seed=2718):
    """Fixed random probe vectors: a large gradient is stored as its
    projections onto these (any plausible error changes many of them)."""
    return np.random.default_rng(seed).standard_normal((PROBES, count))


def matching_fixture(s, wl, chunk=0, outputs=True, rprop=True, generator=None, project=()):
    """``generator``: (name, kwargs) of the workloads function that rebuilds
    the inputs; then only checksums of the inputs are stored.  Gradients of the
    transitions listed in ``project`` are stored as probe projections."""
    ids = wl.upload(s, chunk)
    rec = dict(neurons=np.asarray(wl.neurons, np.int32), linear=np.asarray(wl.linear, np.int32),
               chunk=np.int32(chunk))
    if generator is None:
        rec.update(schema=wl.schema, points=wl.points, target=wl.target, row_weights=wl.row_weights)
        for t, w in enumerate(wl.init):
            rec[f'init{t}'] = np.asarray(w, np.float32)
    else:
        rec['generator'] = np.array(generator[0])
        rec['generator_args'] = np.array(repr(generator[1]))
        rec['checksums'] = np.stack([checksum(wl.points), checksum(wl.target), checksum(wl.row_weights),
                                     checksum(np.concatenate(wl.init))])
    value, grads = s.graph_eval(ids['net'], [ids['cost']], SINGLE_LEAF, gradient=True)
    rec['loss'] = np.float64(value)
    for t, g in enumerate(grads):
        if t in project:
            rec[f'grad{t}_probes'] = probes(g.size) @ g.astype(np.float64)
            rec[f'grad{t}_norm'] = np.float64(np.linalg.norm(g.astype(np.float64)))
        else:
            rec[f'grad{t}'] = g
    if outputs:
        out = s.eval(ids['net'], ids['data'], chunk)
        rec['outputs'] = s.download(out).reshape(wl.rows, wl.size, wl.neurons[-1])
        s.close_object(0, out)
    if rprop:
        s.train(ids['net'], [ids['cost']], 1, method=0, fresh=1, log=1)
        meta, layers = wire.decode_state(s.snapshot(ids['net']))
        for t, layer in enumerate(layers):
            rec[f'after{t}'] = layer['buffers'][0]
            rec[f'step{t}'] = layer['buffers'][3]
            rec[f'active{t}'] = np.int32(layer['active'])
    for kind, key in ((2, 'cost'), (1, 'net'), (0, 'data'), (0, 'target')):
        s.close_object(kind, ids[key])
    return rec


def case_tiny_order6(s):
    neurons = [2, 8, 8, 1]
    schema = W.full_schema(2, 6)
    rng = np.random.default_rng(11)
    pts = rng.uniform(0, 1, (30, 2))
    freq, coef, phase = W.fourier_modes(2, 3, 3, 11)
    target = W.fourier_target(pts, schema, freq, coef, phase)
    wl = W.MatchingWorkload('tiny_order6', neurons, pts, schema, target, 1.0 / target.var(axis=1),
                            W.xavier_weights(neurons, 11))
    rec = matching_fixture(s, wl)
    # the same epoch in chunks of 7 points (zero-padded final chunk)
    wl2 = W.MatchingWorkload('tiny_order6', neurons, pts, schema, target, 1.0 / target.var(axis=1),
                             W.xavier_weights(neurons, 11))
    ids = wl2.upload(s, 7)
    value, grads = s.graph_eval(ids['net'], [ids['cost']], SINGLE_LEAF, gradient=True)
    rec['chunk7_loss'] = np.float64(value)
    for t, g in enumerate(grads):
        rec[f'chunk7_grad{t}'] = g
    return rec


def case_tiny_3var_order4(s):
    neurons = [3, 12, 10, 1]
    schema = W.full_schema(3, 4)
    rng = np.random.default_rng(12)
    pts = rng.uniform(0, 1, (24, 3))
    freq, coef, phase = W.fourier_modes(3, 3, 3, 12)
    target = W.fourier_target(pts, schema, freq, coef, phase)
    wl = W.MatchingWorkload('tiny_3var_order4', neurons, pts, schema, target, 1.0 / target.var(axis=1),
                            W.xavier_weights(neurons, 12))
    return matching_fixture(s, wl)


def case_fourier_order2(s):
    return matching_fixture(s, W.fourier_fit(2), rprop=False, generator=('fourier_fit', dict(order=2)))


def case_fourier_order6(s):
    return matching_fixture(s, W.fourier_fit(6), rprop=False, generator=('fourier_fit', dict(order=6)))


def case_fourier3d_reduced(s):
    return matching_fixture(s, W.fourier_3d(points=256), rprop=False,
                            generator=('fourier_3d', dict(points=256)), project=(1, 2, 3, 4))


def case_large_reduced(s):
    wl = W.fourier_large(points=192)
    return matching_fixture(s, wl, chunk=80, rprop=False, generator=('fourier_large', dict(points=192)),
                            project=(1, 2, 3))


def case_published(s):
    losses = []
    for order in range(7):
        wl = reference_benchmark(order)
        ids = wl.upload(s, 0)
        value, _ = s.graph_eval(ids['net'], [ids['cost']], SINGLE_LEAF, gradient=False)
        losses.append(value)
        for kind, key in ((2, 'cost'), (1, 'net'), (0, 'data'), (0, 'target')):
            s.close_object(kind, ids[key])
    return dict(published_losses=np.asarray(losses, np.float64),
                published_reference=np.asarray(PUBLISHED_LOSSES, np.float64))


def case_poisson(s):
    pw = W.PoissonWorkload(radial=16, angular=16, boundary=64)
    ids = pw.upload(s)
    value, grads = s.graph_eval(ids['net'], ids['costs'], pw.graph(), gradient=True)
    rec = dict(neurons=np.asarray(pw.neurons, np.int32), radial=np.int32(16), angular=np.int32(16),
               boundary=np.int32(64), loss=np.float64(value))
    for t, w in enumerate(pw.init):
        rec[f'init{t}'] = np.asarray(w, np.float32)
    for t, g in enumerate(grads):
        rec[f'grad{t}'] = g
    # each leaf alone
    for leaf in range(2):
        v, _ = s.graph_eval(ids['net'], [ids['costs'][leaf]], SINGLE_LEAF, gradient=False)
        rec[f'leaf{leaf}'] = np.float64(v)
    # a graph whose leaf multipliers depend on the leaf values (second backward
    # pass, cuda/cpde_server.cu:279-316): leaf0 / leaf1 + log(leaf0) + leaf1 ** 1.5
    graph = W.PoissonWorkload.value_dependent_graph()
    value, grads = s.graph_eval(ids['net'], ids['costs'], graph, gradient=True)
    rec['vgraph_loss'] = np.float64(value)
    for t, g in enumerate(grads):
        rec[f'vgraph_grad{t}'] = g
    res = s.train(ids['net'], ids['costs'], 2, method=0, fresh=1, log=1, graph=graph)
    rec['vgraph_reports'] = np.asarray([(e['completed'], e['updates'], e['after'], e['total'])
                                        for e in res['events'] if e['kind'] == 6], np.float64)
    rec['vgraph_state'] = np.frombuffer(s.snapshot(ids['net']), np.uint8)
    return rec


def tiny_workload(seed=11, order=6, neurons=(2, 8, 8, 1), points=30):
    schema = W.full_schema(2, order)
    rng = np.random.default_rng(seed)
    pts = rng.uniform(0, 1, (points, 2))
    freq, coef, phase = W.fourier_modes(2, 3, 3, seed)
    target = W.fourier_target(pts, schema, freq, coef, phase)
    return W.MatchingWorkload('tiny', list(neurons), pts, schema, target, 1.0 / target.var(axis=1),
                              W.xavier_weights(list(neurons), seed))


def case_polynomial(s):
    """Sparse residuals (op 7 kind 1) on an order-2 schema: equation 0 is
    linear, c0 u_xx + c1 u_yy - rhs0; equation 1 quadratic, c2 u u_x - rhs1."""
    wl = tiny_workload(seed=21, order=2, neurons=(2, 10, 9, 1), points=25)
    rng = np.random.default_rng(21)
    P = wl.size
    keys = [tuple(r[1:]) for r in wl.schema]
    xx, yy, x, v = keys.index((2, 0)), keys.index((0, 2)), keys.index((1, 0)), keys.index((0, 0))
    terms = np.array([[0, xx, -1], [0, yy, -1], [1, v, x]], np.int32)
    coeffs = rng.uniform(0.5, 1.5, (3, P)).astype(np.float32)
    rhs = rng.standard_normal((2, P)).astype(np.float32)
    weights = rng.uniform(0.2, 1.0, (2, P)).astype(np.float32)
    weights[1, :3] = 0
    d = s.data(wl.inputs, wl.schema)
    n = s.network(wl.neurons, wl.linear, wl.init)
    rows = list(range(wl.rows))
    c = s.polynomial_cost(n, d, rows, 2, terms, coeffs, rhs, weights, chunk=10)
    value, grads = s.graph_eval(n, [c], SINGLE_LEAF, gradient=True)
    rec = dict(neurons=np.asarray(wl.neurons, np.int32), schema=wl.schema, points=wl.points, terms=terms,
               coeffs=coeffs, rhs=rhs, weights=weights, chunk=np.int32(10), loss=np.float64(value))
    for t, w in enumerate(wl.init):
        rec[f'init{t}'] = np.asarray(w, np.float32)
    for t, g in enumerate(grads):
        rec[f'grad{t}'] = g
    s.train(n, [c], 1, method=0, fresh=1, log=1)
    _, layers = wire.decode_state(s.snapshot(n))
    for t, layer in enumerate(layers):
        rec[f'after{t}'] = layer['buffers'][0]
    return rec


def case_training(s):
    """Three RPROP epochs with per-epoch reports and gradient diagnostics, then
    two Adam epochs (lr 0.01) on a fresh network: reported objectives and the
    final state blobs."""
    wl = tiny_workload(seed=31, order=4, neurons=(2, 12, 12, 1), points=40)
    ids = wl.upload(s, 16)
    res = s.train(ids['net'], [ids['cost']], 3, method=0, fresh=1, log=1, diagnostics=1, eval_every=2)
    reports = [(e['completed'], e['updates'], e['after'], e['values'][0]) for e in res['events'] if e['kind'] == 2]
    diag = [(e['epoch'], e['layers'][0]['sq'], e['layers'][0]['max']) for e in res['events'] if e['kind'] == 5]
    rprop_state = s.snapshot(ids['net'])
    wl2 = tiny_workload(seed=31, order=4, neurons=(2, 12, 12, 1), points=40)
    ids2 = wl2.upload(s, 16)
    res2 = s.train(ids2['net'], [ids2['cost']], 2, method=1, fresh=1, lr=0.01, log=1)
    adam_reports = [(e['completed'], e['updates'], e['after'], e['values'][0]) for e in res2['events']
                    if e['kind'] == 2]
    adam_state = s.snapshot(ids2['net'])
    rec = dict(neurons=np.asarray(wl.neurons, np.int32), schema=wl.schema, points=wl.points, target=wl.target,
               row_weights=wl.row_weights, chunk=np.int32(16),
               reports=np.asarray(reports, np.float64), diagnostics=np.asarray(diag, np.float64),
               rprop_state=np.frombuffer(rprop_state, np.uint8), adam_reports=np.asarray(adam_reports, np.float64),
               adam_state=np.frombuffer(adam_state, np.uint8),
               completed=np.int64(res['completed']), stopped=np.int32(res['stopped']))
    for t, w in enumerate(wl.init):
        rec[f'init{t}'] = np.asarray(w, np.float32)
    return rec


def state_arrays(blob):
    """(metadata, [per transition: W, buffer 1, buffer 2, step/m, active])."""
    meta, layers = wire.decode_state(blob)
    return meta, [(*layer['buffers'], layer['active']) for layer in layers]


def stepped_run(s, ids, epochs, first, later, prefix, rec):
    """``epochs`` single-epoch op-8 calls (``first`` the first call's keyword
    arguments, ``later`` the others'), each preceded by an op-14 gradient at
    the current weights and followed by an op-9 snapshot: the exact gradient
    every update consumed and the state it left."""
    for k in range(epochs):
        _, grads = s.graph_eval(ids['net'], [ids['cost']], SINGLE_LEAF, gradient=True)
        for t, g in enumerate(grads):
            rec[f'{prefix}_grad{k}_{t}'] = g
        s.train(ids['net'], [ids['cost']], 1, log=1, **(first if k == 0 else later))
        rec[f'{prefix}_state{k}'] = np.frombuffer(s.snapshot(ids['net']), np.uint8)
    rec[f'{prefix}_epochs'] = np.int32(epochs)


def case_optimizer(s):
    """Optimizer trajectories with the gradient each update consumed:
      * ``rprop``: six RPROP epochs from a fresh state (initial step 0.002);
      * ``bigstep``: six RPROP epochs after reset_steps=0.05, so that sign
        reversals (rollback, x0.5) occur early;
      * ``restore``: four RPROP epochs with reset_steps=2e-4 and
        restore_every=2, restore_step=1e-3 (cuda/cpde_server.cu:377,415-418);
      * ``adam``: three Adam epochs with lr 0.01.
    The initial weights and the state blob after every epoch are stored."""
    wl = tiny_workload(seed=41, order=4, neurons=(2, 12, 12, 1), points=40)
    rec = dict(neurons=np.asarray(wl.neurons, np.int32), schema=wl.schema, points=wl.points, target=wl.target,
               row_weights=wl.row_weights, chunk=np.int32(16))
    for t, w in enumerate(wl.init):
        rec[f'init{t}'] = np.asarray(w, np.float32)
    runs = [('rprop', dict(method=0, fresh=1), dict(method=0, fresh=0), 6),
            ('bigstep', dict(method=0, fresh=1, steps=0.05), dict(method=0, fresh=0), 6),
            ('restore', dict(method=0, fresh=1, steps=2e-4, restore_every=2, restore_step=1e-3),
             dict(method=0, fresh=0, restore_every=2, restore_step=1e-3), 4),
            ('adam', dict(method=1, fresh=1, lr=0.01), dict(method=1, fresh=0), 3)]
    for prefix, first, later, epochs in runs:
        ids = wl.upload(s, 16)
        stepped_run(s, ids, epochs, first, later, prefix, rec)
        for kind, key in ((2, 'cost'), (1, 'net'), (0, 'data'), (0, 'target')):
            s.close_object(kind, ids[key])
    return rec


def events_record(res, ids_to_index):
    """Event frames as arrays: kinds in order, report rows (completed, updates,
    after, values...), state blobs and output frames (cost index, values)."""
    kinds = np.asarray([e['kind'] for e in res['events']], np.int32)
    reports = [(e['completed'], e['updates'], e['after'], *e['values']) for e in res['events'] if e['kind'] == 2]
    blobs = [np.frombuffer(e['blob'], np.uint8) for e in res['events'] if e['kind'] == 3]
    outputs = [(ids_to_index[e['cost']], e['outputs']) for e in res['events'] if e['kind'] == 4]
    return kinds, np.asarray(reports, np.float64), blobs, outputs


def linear_unit(s, weight, bias, x):
    """The reference tests' one-input linear network u = weight*x + bias
    (tests/test_interface.py:290-325) on a single value-row sample."""
    n = s.network([1, 1], [1, 1], [np.array([weight, bias], np.float32)])
    d = s.data(np.array([[[x]]], np.float32), np.array([[0, 0]], np.int32))
    return n, d


def case_protocol(s):
    """Training-loop surface against the reference server:
      * save_every=2, eval_every=2 and print_outputs over five epochs
        (kind-2 reports, kind-3 snapshots, kind-4 outputs, cuda/cpde_server.cu:419-433);
      * op 99 sent on the first kind-3 frame of a 100,000-epoch call, then a
        resume of two remaining epochs from the stopped state
        (tests/test_interface.py:204-222);
      * non-finite weight gradient (u = 1e10 at x = 1e30: dE/dW overflows)
        and non-finite dE/dY with a finite objective (1e30 * u at u = 1e-20),
        both rejected before any update (tests/test_interface.py:290-325)."""
    wl = tiny_workload(seed=51, order=2, neurons=(2, 10, 10, 1), points=30)
    rec = dict(neurons=np.asarray(wl.neurons, np.int32), schema=wl.schema, points=wl.points, target=wl.target,
               row_weights=wl.row_weights, chunk=np.int32(16))
    for t, w in enumerate(wl.init):
        rec[f'init{t}'] = np.asarray(w, np.float32)
    ids = wl.upload(s, 16)
    res = s.train(ids['net'], [ids['cost']], 5, method=0, fresh=1, log=2, eval_every=2, outputs=1, save=2)
    kinds, reports, blobs, outputs = events_record(res, {ids['cost']: 0})
    rec.update(periodic_kinds=kinds, periodic_reports=reports, periodic_completed=np.int64(res['completed']))
    for i, b in enumerate(blobs):
        rec[f'periodic_blob{i}'] = b
    for i, (c, o) in enumerate(outputs):
        rec[f'periodic_outputs{i}'] = o
    rec['periodic_final'] = np.frombuffer(s.snapshot(ids['net']), np.uint8)

    # stop at the first checkpoint of a long call, then resume two epochs
    stop_ids = wl.upload(s, 16)

    def stop_on_checkpoint(session, ev):
        if ev['kind'] == 3 and not getattr(session, '_stop_sent', False):
            session._stop_sent = True
            session.stop()

    s._stop_sent = False
    res = s.train(stop_ids['net'], [stop_ids['cost']], 100000, method=1, fresh=1, lr=0.01, log=1, save=1,
                  stage='stop-test', on_event=stop_on_checkpoint)
    stopped_blob = s.snapshot(stop_ids['net'])
    meta, layers = wire.decode_state(stopped_blob)
    kinds = np.asarray([e['kind'] for e in res['events']], np.int32)
    rec.update(stop_completed=np.int64(res['completed']), stop_stopped=np.int32(res['stopped']), stop_kinds=kinds,
               stop_meta=np.asarray([meta['updates'], meta['adam_step'], meta['stage_done'], meta['remaining']],
                                    np.int64))
    meta['remaining'] = 2
    s.restore(stop_ids['net'], wire.encode_state(meta, layers))
    res = s.train(stop_ids['net'], [stop_ids['cost']], 2, method=1, fresh=0, log=1, stage='stop-test')
    meta2, _ = wire.decode_state(s.snapshot(stop_ids['net']))
    rec.update(resume_completed=np.int64(res['completed']), resume_stopped=np.int32(res['stopped']),
               resume_meta=np.asarray([meta2['updates'], meta2['adam_step'], meta2['stage_done'],
                                       meta2['remaining']], np.int64))

    # non-finite weight gradient: objective and dE/dY finite, x * dE/dY overflows
    n, d = linear_unit(s, 0.0, 1e10, 1e30)
    c = s.polynomial_cost(n, d, [0], 1, [[0, 0, -1]], np.ones((1, 1), np.float32), np.zeros((1, 1), np.float32),
                          np.ones((1, 1), np.float32))
    before = s.snapshot(n)
    try:
        s.train(n, [c], 1, method=1, fresh=1, lr=0.01, log=1)
        raise SystemExit('reference accepted a non-finite weight gradient')
    except wire.ServerError as e:
        rec['weight_gradient_error'] = np.array(str(e))
        diag = [ev for ev in e.events if ev['kind'] == 5]
        rec['weight_gradient_diag'] = np.asarray([(l['nonfinite'], l['first'], l['max']) for l in diag[0]['layers']],
                                                 np.float64)
    rec['weight_gradient_before'] = np.frombuffer(before, np.uint8)
    rec['weight_gradient_after'] = np.frombuffer(s.snapshot(n), np.uint8)

    # non-finite dE/dY with a finite objective
    n, d = linear_unit(s, 0.0, 1e-20, 0.0)
    c = s.polynomial_cost(n, d, [0], 1, [[0, 0, -1]], np.full((1, 1), 1e30, np.float32),
                          np.zeros((1, 1), np.float32), np.ones((1, 1), np.float32))
    before = s.snapshot(n)
    try:
        s.train(n, [c], 1, method=1, fresh=1, lr=0.01, log=1)
        raise SystemExit('reference accepted a non-finite output gradient')
    except wire.ServerError as e:
        rec['output_gradient_error'] = np.array(str(e))
    rec['output_gradient_before'] = np.frombuffer(before, np.uint8)
    rec['output_gradient_after'] = np.frombuffer(s.snapshot(n), np.uint8)
    return rec


def case_variations(s):
    """Attached variations and frozen components: each leaf alone, the nested
    variation graph (value-dependent multipliers, shared leaves), the cancelled
    variation, and two RPROP epochs of the nested graph."""
    vw = W.VariationWorkload()
    n, d, costs = vw.upload(s)
    rec = dict(neurons=np.asarray(vw.neurons, np.int32), points=vw.points, quadrature=vw.weights)
    for t, w in enumerate(vw.init):
        rec[f'init{t}'] = np.asarray(w, np.float32)
    for name in ('a', 'correction', 'frozen', 'free'):
        value, grads = s.graph_eval(n, [costs[name]], SINGLE_LEAF, gradient=True)
        rec[f'{name}_value'] = np.float64(value)
        for t, g in enumerate(grads):
            rec[f'{name}_grad{t}'] = g
    value, grads = s.graph_eval(n, [costs['a'], costs['correction']], vw.nested_graph(), gradient=True)
    rec['nested_value'] = np.float64(value)
    for t, g in enumerate(grads):
        rec[f'nested_grad{t}'] = g
    value, grads = s.graph_eval(n, [costs['a']], vw.cancelled_graph(), gradient=True)
    rec['cancelled_value'] = np.float64(value)
    for t, g in enumerate(grads):
        rec[f'cancelled_grad{t}'] = g
    res = s.train(n, [costs['a'], costs['correction']], 2, method=0, fresh=1, log=1, graph=vw.nested_graph())
    rec['nested_reports'] = np.asarray([(e['completed'], e['updates'], e['after'], e['total'])
                                        for e in res['events'] if e['kind'] == 6], np.float64)
    rec['nested_state'] = np.frombuffer(s.snapshot(n), np.uint8)
    return rec


def case_poisson_full(s):
    """The Poisson workload at full size: 64 Gauss-Legendre radii x 64 angles
    plus 256 boundary points.  Objective, leaves, gradient, and the state after
    two RPROP epochs (reset_steps 2e-4)."""
    pw = W.PoissonWorkload()
    ids = pw.upload(s)
    value, grads = s.graph_eval(ids['net'], ids['costs'], pw.graph(), gradient=True)
    rec = dict(loss=np.float64(value))
    for t, g in enumerate(grads):
        rec[f'grad{t}'] = g
    for leaf in range(2):
        v, _ = s.graph_eval(ids['net'], [ids['costs'][leaf]], SINGLE_LEAF, gradient=False)
        rec[f'leaf{leaf}'] = np.float64(v)
    res = s.train(ids['net'], ids['costs'], 2, method=0, fresh=1, steps=2e-4, log=1, graph=pw.graph())
    rec['reports'] = np.asarray([(e['completed'], e['updates'], e['after'], e['total'])
                                 for e in res['events'] if e['kind'] == 6], np.float64)
    rec['state'] = np.frombuffer(s.snapshot(ids['net']), np.uint8)
    rec['checksums'] = np.stack([checksum(pw.interior), checksum(pw.interior_w), checksum(pw.boundary),
                                 checksum(pw.f), checksum(np.concatenate(pw.init))])
    return rec


def closure_indices(schema, requested):
    """Indices into ``schema`` of the closure of the requested count tuples."""
    keys = [tuple(r[1:]) for r in schema]
    return np.array([keys.index(tuple(r[1:])) for r in W.closed_schema(schema.shape[1] - 1, requested)], np.int32)


def form_workload(order, points, seed, neurons, requested=None, reverse_target=False, per_sample=False, chunk=0):
    """A matching workload on random points of [0,1]^2: data with the full
    schema of ``order``; the cost over the closure of ``requested`` (default:
    every row); targets in a data object whose rows are reversed when
    ``reverse_target``; one weight per row (1/var) or, with ``per_sample``,
    per row and sample, U(0.2, 1.5) with a fifth of them zero."""
    schema = W.full_schema(2, order)
    rng = np.random.default_rng(seed)
    pts = rng.uniform(0, 1, (points, 2))
    freq, coef, phase = W.fourier_modes(2, 3, 3, seed)
    target = W.fourier_target(pts, schema, freq, coef, phase)
    rows = np.arange(len(schema), dtype=np.int32) if requested is None else closure_indices(schema, requested)
    perm = np.arange(len(schema))[::-1] if reverse_target else np.arange(len(schema))
    target_rows = np.array([int(np.flatnonzero(perm == r)[0]) for r in rows], np.int32)
    if per_sample:
        weights = rng.uniform(0.2, 1.5, (len(rows), points))
        weights[rng.random(weights.shape) < 0.2] = 0
    else:
        weights = 1.0 / target[rows].var(axis=1)
    return W.MatchingWorkload('form', neurons, pts, schema, target[perm], weights, W.xavier_weights(neurons, seed),
                              chunk=chunk, rows=rows, target_schema=schema[perm], target_rows=target_rows)


FORMS = {
    # name: form_workload arguments
    'persample': dict(order=6, points=30, seed=71, neurons=(2, 8, 8, 1), per_sample=True, chunk=7),
    'subset': dict(order=2, points=40, seed=72, neurons=(2, 10, 9, 1), requested=[(2, 0)], reverse_target=True),
    'subset_persample': dict(order=4, points=33, seed=73, neurons=(2, 9, 8, 1), requested=[(1, 2)],
                             reverse_target=True, per_sample=True, chunk=9),
}


def workload_record(wl, prefix):
    rec = {f'{prefix}_{k}': v for k, v in dict(
        neurons=np.asarray(wl.neurons, np.int32), linear=np.asarray(wl.linear, np.int32), schema=wl.schema,
        points=wl.points, target=wl.target, target_schema=wl.target_schema, rows=wl.cost_rows,
        target_rows=wl.target_rows, weights=wl.row_weights, chunk=np.int32(wl.chunk)).items()}
    for t, w in enumerate(wl.init):
        rec[f'{prefix}_init{t}'] = np.asarray(w, np.float32)
    return rec


def epoch_record(s, wl, prefix, outputs=False):
    """op 14 (value and gradient), optionally op 4 outputs, and the weights
    after one RPROP epoch from a fresh state."""
    rec = workload_record(wl, prefix)
    ids = wl.upload(s)
    value, grads = s.graph_eval(ids['net'], [ids['cost']], SINGLE_LEAF, gradient=True)
    rec[f'{prefix}_loss'] = np.float64(value)
    for t, g in enumerate(grads):
        rec[f'{prefix}_grad{t}'] = g
    if outputs:
        out = s.eval(ids['net'], ids['data'], wl.chunk)
        rec[f'{prefix}_outputs'] = s.download(out).reshape(len(wl.schema), wl.size, wl.neurons[-1])
        s.close_object(0, out)
    s.train(ids['net'], [ids['cost']], 1, method=0, fresh=1, log=1)
    _, layers = wire.decode_state(s.snapshot(ids['net']))
    for t, layer in enumerate(layers):
        rec[f'{prefix}_after{t}'] = layer['buffers'][0]
    for kind, key in ((2, 'cost'), (1, 'net'), (0, 'data'), (0, 'target')):
        s.close_object(kind, ids[key])
    return rec


def case_matching_forms(s):
    """Matching-cost requests the client sends (cpde/api.py:350-362) in forms the
    other cases leave out, each as op 14 (value + gradient) and one RPROP
    epoch:
      * ``persample``: one weight per row and sample (weight_samples = P, the
        [R][P][1] layout, cuda/cost_kernels.cuh:17-19), a fifth of them zero,
        order 6 on 30 points in chunks of 7, so the sample index is offset + p;
      * ``subset``: data with the full order-2 schema, a cost over the closure
        of {xx} = rows (1, x, xx), not a prefix, and targets in a data object
        whose rows run in reverse order, so target_rows remaps
        (cuda/cost_kernels.cuh:20);
      * ``subset_persample``: both at order 4, the closure of {x y^2}, chunks
        of 9."""
    rec = {}
    for name, kwargs in FORMS.items():
        rec.update(epoch_record(s, form_workload(**kwargs), name))
    return rec


LINEAR_HIDDEN = {
    # name: (neurons, linear flags, order, points, chunk)
    'inner': ((2, 8, 6, 8, 1), (1, 0, 1, 0, 1), 4, 25, 10),
    'first': ((2, 10, 8, 1), (1, 1, 0, 1), 6, 20, 0),
}


def case_linear_hidden(s):
    """Networks with linear hidden layers, which the client accepts
    (cpde/api.py:270-272) and whose composition the reference skips
    (cuda/cpde_engine.cuh:894-909,973-987): 2->8->6(linear)->8->1 at order 4
    in chunks of 10, and 2->10(linear)->8->1 at order 6.  op 14 value and
    gradient, outputs (op 4 + op 5) and one RPROP epoch."""
    rec = {}
    for name, (neurons, linear, order, points, chunk) in LINEAR_HIDDEN.items():
        schema = W.full_schema(2, order)
        rng = np.random.default_rng(81 + order)
        pts = rng.uniform(0, 1, (points, 2))
        freq, coef, phase = W.fourier_modes(2, 3, 3, 81 + order)
        target = W.fourier_target(pts, schema, freq, coef, phase)
        wl = W.MatchingWorkload(name, neurons, pts, schema, target, 1.0 / target.var(axis=1),
                                W.xavier_weights(neurons, 81 + order), chunk=chunk, linear=linear)
        rec.update(epoch_record(s, wl, name, outputs=True))
    return rec


def empty_integral_graphs():
    """Graphs over leaf 0 (a sampled integral) and leaf 1 (an empty one):
    ``constant``: leaf0 + 3 exp(leaf1), multipliers known; ``dependent``:
    leaf0 * (leaf1 + 2), leaf 0's multiplier depends on leaf 1's value."""
    constant = wire.graph_bytes([(1, 0, 0), (1, 1, 0), (9, 1, 0), (0, 0, 0), (5, 2, 3), (3, 0, 4)],
                                [0.0, 0.0, 0.0, 3.0, 0.0, 0.0], 5)
    dependent = wire.graph_bytes([(1, 0, 0), (1, 1, 0), (0, 0, 0), (3, 1, 2), (5, 0, 3)],
                                 [0.0, 0.0, 2.0, 0.0, 0.0], 4)
    return dict(constant=constant, dependent=dependent)


def empty_integral_costs(s, vw, n, d):
    """Leaf 0: u**2 over the variation workload's points in chunks of 5; leaf 1:
    an empty integral (op 12 with samples = 0 and no input data,
    cuda/cpde_server.cu:491-497), whose pass does nothing (:226), so its value
    stays 0."""
    leaf0 = s.integral_cost(n, d, *vw.FREE, np.zeros((0, len(vw.points))), vw.weights, chunk=5)
    leaf1 = s.integral_cost(n, 0, [(0, 0, 0)], [1.0], np.zeros((0, 0)), np.zeros(0))
    return [leaf0, leaf1]


def case_empty_integral(s):
    """An empty integral as a graph leaf: op 14 value and gradient of both
    graphs of ``empty_integral_graphs`` and the state after two RPROP epochs
    of the value-dependent one."""
    vw = W.VariationWorkload()
    rec = dict(neurons=np.asarray(vw.neurons, np.int32), points=vw.points, quadrature=vw.weights)
    for t, w in enumerate(vw.init):
        rec[f'init{t}'] = np.asarray(w, np.float32)
    d = s.data(W.input_stack(vw.points, vw.schema), vw.schema)
    n = s.network(vw.neurons, W.linear_flags(vw.neurons), vw.init)
    leaves = empty_integral_costs(s, vw, n, d)
    for name, graph in empty_integral_graphs().items():
        value, grads = s.graph_eval(n, leaves, graph, gradient=True)
        rec[f'{name}_value'] = np.float64(value)
        for t, g in enumerate(grads):
            rec[f'{name}_grad{t}'] = g
    res = s.train(n, leaves, 2, method=0, fresh=1, log=1, graph=empty_integral_graphs()['dependent'])
    rec['reports'] = np.asarray([(e['completed'], e['updates'], e['after'], *e['values'], e['total'])
                                 for e in res['events'] if e['kind'] == 6], np.float64)
    rec['state'] = np.frombuffer(s.snapshot(n), np.uint8)
    return rec


CASES = {
    'tiny_order6': case_tiny_order6,
    'tiny_3var_order4': case_tiny_3var_order4,
    'fourier_order2': case_fourier_order2,
    'fourier_order6': case_fourier_order6,
    'fourier3d_reduced': case_fourier3d_reduced,
    'large_reduced': case_large_reduced,
    'published': case_published,
    'poisson': case_poisson,
    'polynomial': case_polynomial,
    'training': case_training,
    'optimizer': case_optimizer,
    'protocol': case_protocol,
    'variations': case_variations,
    'poisson_full': case_poisson_full,
    'matching_forms': case_matching_forms,
    'linear_hidden': case_linear_hidden,
    'empty_integral': case_empty_integral,
}


def main(names):
    names = names or list(CASES)
    with session() as s:
        print(f'[golden] server {s.protocol} v{s.version} caps {s.capabilities}', flush=True)
        for name in names:
            t0 = time.time()
            rec = CASES[name](s)
            np.savez_compressed(HERE / f'{name}.npz', **rec)
            print(f'[golden] {name}: {time.time() - t0:.1f} s', flush=True)


if __name__ == '__main__':
    main(sys.argv[1:])
