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

from cpde_amd import wire, workloads as W  # noqa: E402

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
        wl = W.reference_benchmark(order)
        ids = wl.upload(s, 0)
        value, _ = s.graph_eval(ids['net'], [ids['cost']], SINGLE_LEAF, gradient=False)
        losses.append(value)
        for kind, key in ((2, 'cost'), (1, 'net'), (0, 'data'), (0, 'target')):
            s.close_object(kind, ids[key])
    return dict(published_losses=np.asarray(losses, np.float64),
                published_reference=np.asarray(W.PUBLISHED_LOSSES, np.float64))


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
