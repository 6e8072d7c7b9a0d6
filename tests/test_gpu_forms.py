"""Request forms the reference client sends that the workload goldens leave
out, against the reference CPU server's answers (tests/golden/make_golden.py:
matching_forms, linear_hidden, empty_integral):

  * matching weights per sample (weight_samples = P, the [R][P][1] layout,
    cuda/cost_kernels.cuh:17-19) with zero entries, in chunks;
  * a matching cost on a non-prefix subset of the data's rows, with targets in
    a data object whose rows run in another order (target_rows remaps,
    cuda/cost_kernels.cuh:20);
  * networks with linear hidden layers (cuda/cpde_engine.cuh:894-909,973-987);
  * an empty integral as a graph leaf (op 12 with no samples,
    cuda/cpde_server.cu:491-497), with known and value-dependent multipliers.

Through the C ABI on every kernel family, one-pass and separate launches, and
through the protocol server.  Bars: loss relative error <= 1e-4, every
gradient and output row relative L2 <= 1e-3; after one RPROP epoch, every
weight whose reference gradient exceeds 1e-3 of the largest bit-identical.
"""
import numpy as np
import pytest

from cpde_amd import hip, wire, workloads as W
from cpde_amd.build import SERVER
from helpers import golden_form, load_golden, rel_l2

pytestmark = pytest.mark.gpu

FORMS = [('matching_forms', 'persample'), ('matching_forms', 'subset'), ('matching_forms', 'subset_persample'),
         ('linear_hidden', 'inner'), ('linear_hidden', 'first')]
SINGLE_LEAF = wire.graph_bytes([(1, 0, 0)], [0.0], 0)


def outputs_of(device, run, wl):
    """Forward every chunk on the data's full schema and gather the output stack."""
    R, n_out = len(wl.schema), wl.neurons[-1]
    plan = hip.Plan(run.net, wl.schema, run.width, False)
    dest = hip.Buffer(device, R * wl.size * n_out * 4)
    rows = np.arange(R, dtype=np.int32)
    for offset in range(0, wl.size, run.width):
        valid = min(run.width, wl.size - offset)
        plan.activate(run.data, wl.size, rows, offset, valid)
        plan.forward()
        plan.output(dest, wl.size, rows, offset, valid)
    out = dest.download(np.float32, R * wl.size * n_out).reshape(R, wl.size, n_out)
    dest.free()
    plan.destroy()
    return out


def sure(grad):
    return np.abs(grad) > 1e-3 * np.abs(grad).max()


@pytest.mark.parametrize('one_pass', [True, False], ids=['one-pass', 'separate'])
@pytest.mark.parametrize('record,prefix', FORMS)
def test_forms_through_the_abi(device, path, record, prefix, one_pass):
    g = load_golden(record)
    wl = golden_form(g, prefix)
    print(f'[case] {record}/{prefix} path={path} one_pass={one_pass} neurons={wl.neurons} linear={wl.linear} '
          f'rows={wl.cost_rows.tolist()} target_rows={wl.target_rows.tolist()} weight_samples={wl.weight_samples} '
          f'P={wl.size} chunk={wl.chunk}', flush=True)
    run = hip.MatchingRun(device, wl, one_pass=one_pass)
    run.step()
    device.synchronize()
    loss = run.loss()
    rel = abs(loss / g[f'{prefix}_loss'] - 1)
    print(f'[result] loss {loss!r} reference {float(g[f"{prefix}_loss"])!r} rel {rel:.2e}', flush=True)
    assert rel < 1e-4
    grads = run.gradients()
    for t, grad in enumerate(grads):
        err = rel_l2(grad, g[f'{prefix}_grad{t}'])
        print(f'[result] transition {t} gradient rel-L2 {err:.2e}', flush=True)
        assert err < 1e-3
    if f'{prefix}_outputs' in g:
        out = outputs_of(device, run, wl)
        worst = max(rel_l2(out[r], g[f'{prefix}_outputs'][r]) for r in range(len(wl.schema)))
        print(f'[result] worst output row rel-L2 {worst:.2e}', flush=True)
        assert worst < 1e-3
    # one RPROP update from the fresh state on the reference's own gradient signs
    run.net.rprop()
    device.synchronize()
    for t in range(len(wl.neurons) - 1):
        keep = sure(g[f'{prefix}_grad{t}'])
        np.testing.assert_array_equal(run.net.state(t, 0)[keep], g[f'{prefix}_after{t}'][keep])
    run.close()


@pytest.fixture(scope='module')
def server():
    s = wire.Session(SERVER)
    yield s
    s.close()


@pytest.mark.parametrize('record,prefix', FORMS)
def test_forms_through_the_server(server, record, prefix):
    """The same requests as the client sends them: op 7 with rows, target_rows
    and weight_samples, then op 14 and one op-8 RPROP epoch."""
    g = load_golden(record)
    wl = golden_form(g, prefix)
    ids = wl.upload(server)
    value, grads = server.graph_eval(ids['net'], [ids['cost']], SINGLE_LEAF, gradient=True)
    print(f'[result] {record}/{prefix}: objective {value!r} reference {float(g[f"{prefix}_loss"])!r}', flush=True)
    assert abs(value / g[f'{prefix}_loss'] - 1) < 1e-4
    for t, grad in enumerate(grads):
        assert rel_l2(grad, g[f'{prefix}_grad{t}']) < 1e-3
    if f'{prefix}_outputs' in g:
        out = server.eval(ids['net'], ids['data'], wl.chunk)
        got = server.download(out).reshape(len(wl.schema), wl.size, wl.neurons[-1])
        server.close_object(0, out)
        assert max(rel_l2(got[r], g[f'{prefix}_outputs'][r]) for r in range(len(wl.schema))) < 1e-3
    server.train(ids['net'], [ids['cost']], 1, method=0, fresh=1, log=1)
    _, layers = wire.decode_state(server.snapshot(ids['net']))
    for t, layer in enumerate(layers):
        keep = sure(g[f'{prefix}_grad{t}'])
        np.testing.assert_array_equal(layer['buffers'][0][keep], g[f'{prefix}_after{t}'][keep])
    for kind, key in ((2, 'cost'), (1, 'net'), (0, 'data'), (0, 'target')):
        server.close_object(kind, ids[key])


def empty_integral_setup(s):
    """The objects of make_golden.case_empty_integral, on this server."""
    from make_golden import empty_integral_costs, empty_integral_graphs
    vw = W.VariationWorkload()
    d = s.data(W.input_stack(vw.points, vw.schema), vw.schema)
    n = s.network(vw.neurons, W.linear_flags(vw.neurons), vw.init)
    return n, empty_integral_costs(s, vw, n, d), empty_integral_graphs()


def test_empty_integral_leaf(server):
    """An empty integral's value is 0 and it adds no pass; with a graph over it
    and a sampled leaf, the objective, gradient, two training epochs' reports
    and the final state match the reference server."""
    g = load_golden('empty_integral')
    n, leaves, graphs = empty_integral_setup(server)
    for name, graph in graphs.items():
        value, grads = server.graph_eval(n, leaves, graph, gradient=True)
        print(f'[result] {name}: objective {value!r} reference {float(g[f"{name}_value"])!r}', flush=True)
        assert abs(value / g[f'{name}_value'] - 1) < 1e-4
        for t, grad in enumerate(grads):
            assert rel_l2(grad, g[f'{name}_grad{t}']) < 1e-3
    res = server.train(n, leaves, 2, method=0, fresh=1, log=1, graph=graphs['dependent'])
    reports = np.asarray([(e['completed'], e['updates'], e['after'], *e['values'], e['total'])
                          for e in res['events'] if e['kind'] == 6])
    assert reports.shape == g['reports'].shape
    np.testing.assert_array_equal(reports[:, :3], g['reports'][:, :3])
    np.testing.assert_array_equal(reports[:, 4], g['reports'][:, 4])  # the empty leaf: exactly 0
    np.testing.assert_allclose(reports[:, [3, 5]], g['reports'][:, [3, 5]], rtol=1e-4)
    ours = wire.decode_state(server.snapshot(n))
    ref = wire.decode_state(bytes(g['state']))
    assert ours[0] == ref[0]
    for a, b in zip(ours[1], ref[1]):
        assert rel_l2(a['buffers'][0], b['buffers'][0]) < 1e-5
