"""The training loop's protocol surface against the reference CPU server
(tests/golden/protocol.npz): periodic reports, snapshots and outputs
(save_every, eval_every, print_outputs), op 99 stop and resume, and the two
rejections that happen after a finite objective (a non-finite weight gradient,
a non-finite dE/dY), each of which must leave the state untouched.

Reference behaviour: cuda/cpde_server.cu:364-435 (train), :557-576 (the reader
thread that turns op 99 into a stop flag), tests/test_interface.py:120-146,
204-222 and 290-325."""
import numpy as np
import pytest

from cpde_amd import wire
from cpde_amd.build import SERVER
from helpers import golden_workload, load_golden, rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope='module')
def server():
    if not SERVER.exists():
        pytest.fail('protocol server not built: python -m cpde_amd.build')
    s = wire.Session(SERVER)
    yield s
    s.close()


def same_state(blob, ref_blob, rtol=1e-5):
    meta, layers = wire.decode_state(bytes(blob))
    ref_meta, ref_layers = wire.decode_state(bytes(ref_blob))
    assert meta == ref_meta
    for a, b in zip(layers, ref_layers):
        assert a['active'] == b['active']
        assert rel_l2(a['buffers'][0], b['buffers'][0]) < rtol


def test_periodic_reports_snapshots_and_outputs(server):
    """save_every=2, eval_every=2, print_outputs and log every 2 over five
    epochs: the same frame sequence as the reference, report values at the
    objective bar, snapshots with the reference's metadata, and every output
    frame equal to an evaluation at the weights its epoch's snapshot holds."""
    g = load_golden('protocol')
    wl = golden_workload(g)
    ids = wl.upload(server, int(g['chunk']))
    res = server.train(ids['net'], [ids['cost']], 5, method=0, fresh=1, log=2, eval_every=2, outputs=1, save=2)
    kinds = [e['kind'] for e in res['events']]
    print(f'[result] frames {kinds}', flush=True)
    assert kinds == g['periodic_kinds'].tolist()
    assert res['completed'] == int(g['periodic_completed']) and res['stopped'] == 0
    reports = np.asarray([(e['completed'], e['updates'], e['after'], *e['values']) for e in res['events']
                          if e['kind'] == 2])
    np.testing.assert_array_equal(reports[:, :3], g['periodic_reports'][:, :3])
    np.testing.assert_allclose(reports[:, 3:], g['periodic_reports'][:, 3:], rtol=1e-4)
    blobs = [e['blob'] for e in res['events'] if e['kind'] == 3]
    outputs = [e for e in res['events'] if e['kind'] == 4]
    assert len(blobs) == len(outputs) == 3
    for i, (blob, out) in enumerate(zip(blobs, outputs)):
        same_state(blob, g[f'periodic_blob{i}'])
        assert out['cost'] == ids['cost']
        assert rel_l2(out['outputs'], g[f'periodic_outputs{i}']) < 1e-3
    # the last periodic snapshot is the final state
    final = server.snapshot(ids['net'])
    assert final == blobs[-1]
    same_state(final, g['periodic_final'])
    # each output frame is the evaluation at its epoch's weights
    for blob, out in zip(blobs, outputs):
        server.restore(ids['net'], blob)
        ev = server.eval(ids['net'], ids['data'], int(g['chunk']))
        np.testing.assert_array_equal(server.download(ev), out['outputs'])
        server.close_object(0, ev)


def test_stop_and_resume(server):
    """op 99 on the first checkpoint of a 100,000-epoch call stops after the
    epoch in progress: the reply says stopped, the counters and the remaining
    epochs agree with the epochs done (the reference's relations, checked on its
    own record too), the state equals an uninterrupted run of as many epochs,
    and a resume of two remaining epochs completes them."""
    g = load_golden('protocol')
    # the reference's relations on its own record
    done = int(g['stop_completed'])
    assert int(g['stop_stopped']) == 1 and done > 0
    assert g['stop_meta'].tolist() == [done, done, done, 100000 - done]
    assert g['stop_kinds'].tolist() == [2, 3] * done + [2]
    assert int(g['resume_completed']) == 2 and int(g['resume_stopped']) == 0
    assert g['resume_meta'].tolist() == [done + 2, done + 2, done + 2, 0]

    wl = golden_workload(g)
    ids = wl.upload(server, int(g['chunk']))
    sent = []

    def stop_on_checkpoint(session, ev):
        if ev['kind'] == 3 and not sent:
            sent.append(1)
            session.stop()

    res = server.train(ids['net'], [ids['cost']], 100000, method=1, fresh=1, lr=0.01, log=1, save=1,
                       stage='stop-test', on_event=stop_on_checkpoint)
    n = res['completed']
    print(f'[result] stopped after {n} epochs', flush=True)
    assert res['stopped'] == 1 and 0 < n < 100000
    assert [e['kind'] for e in res['events']] == [2, 3] * n + [2]
    meta, layers = wire.decode_state(server.snapshot(ids['net']))
    assert [meta['updates'], meta['adam_step'], meta['stage_done'], meta['remaining']] == [n, n, n, 100000 - n]
    assert res['metadata'] == meta
    # an uninterrupted run of n epochs from the same start gives the same state
    ids2 = wl.upload(server, int(g['chunk']))
    server.train(ids2['net'], [ids2['cost']], n, method=1, fresh=1, lr=0.01, log=0, stage='stop-test')
    _, straight = wire.decode_state(server.snapshot(ids2['net']))
    for a, b in zip(layers, straight):
        for x, y in zip(a['buffers'], b['buffers']):
            np.testing.assert_array_equal(x, y)
    # resume the two remaining epochs of the stopped stage
    meta['remaining'] = 2
    server.restore(ids['net'], wire.encode_state(meta, layers))
    res = server.train(ids['net'], [ids['cost']], 2, method=1, fresh=0, log=1, stage='stop-test')
    assert res['completed'] == 2 and res['stopped'] == 0
    m2 = res['metadata']
    assert [m2['updates'], m2['adam_step'], m2['stage_done'], m2['remaining']] == [n + 2, n + 2, n + 2, 0]
    # a stop that arrives while no training runs is ignored
    server.stop()
    res = server.train(ids['net'], [ids['cost']], 1, method=1, fresh=0, log=1, stage='stop-test')
    assert res['completed'] == 1 and res['stopped'] == 0


def linear_unit(s, weight, bias, x):
    n = s.network([1, 1], [1, 1], [np.array([weight, bias], np.float32)])
    d = s.data(np.array([[[x]]], np.float32), np.array([[0, 0]], np.int32))
    return n, d


def unit_cost(s, n, d, coefficient):
    return s.polynomial_cost(n, d, [0], 1, [[0, 0, -1]], np.full((1, 1), coefficient, np.float32),
                             np.zeros((1, 1), np.float32), np.ones((1, 1), np.float32))


def assert_untouched(blob, ref_before, ref_after):
    """Weights, moments and counters as the reference left them."""
    meta, layers = wire.decode_state(blob)
    ref_meta, ref_layers = wire.decode_state(bytes(ref_after))
    _, before = wire.decode_state(bytes(ref_before))
    assert meta == ref_meta
    assert meta['updates'] == 0 and meta['adam_step'] == 0
    for a, b, c in zip(layers, ref_layers, before):
        np.testing.assert_array_equal(a['buffers'][0], b['buffers'][0])
        np.testing.assert_array_equal(a['buffers'][0], c['buffers'][0])
        np.testing.assert_array_equal(a['buffers'][3], b['buffers'][3])
        np.testing.assert_array_equal(a['buffers'][2], b['buffers'][2])
        assert a['active'] == b['active']


def test_nonfinite_weight_gradient_is_rejected(server):
    """u = 1e10 at x = 1e30: the objective (1e20) and dE/dY (2e10) are finite,
    dE/dW = x dE/dY overflows.  The same message as the reference, a gradient
    report naming the entry, no update; then the session recovers."""
    g = load_golden('protocol')
    n, d = linear_unit(server, 0.0, 1e10, 1e30)
    c = unit_cost(server, n, d, 1.0)
    with pytest.raises(wire.ServerError) as err:
        server.train(n, [c], 1, method=1, fresh=1, lr=0.01, log=1)
    assert str(err.value) == str(g['weight_gradient_error'])
    diag = [e for e in err.value.events if e['kind'] == 5]
    assert len(diag) == 1
    got = np.asarray([(l['nonfinite'], l['first'], l['max']) for l in diag[0]['layers']], np.float64)
    np.testing.assert_array_equal(got, g['weight_gradient_diag'])
    assert_untouched(server.snapshot(n), g['weight_gradient_before'], g['weight_gradient_after'])
    # recovery: zero weights and input, clean history; the next epoch is clean
    meta, layers = wire.decode_state(server.snapshot(n))
    for layer in layers:
        layer['buffers'] = [np.zeros_like(b) for b in layer['buffers']]
    server.restore(n, wire.encode_state(meta, layers))
    server.replace(d, np.zeros((1, 1, 1), np.float32))
    res = server.train(n, [c], 1, method=1, fresh=0, log=1, diagnostics=1)
    layer = [e for e in res['events'] if e['kind'] == 5][0]['layers'][0]
    assert (layer['sq'], layer['max'], layer['nonfinite'], layer['first']) == (0.0, 0.0, 0, -1)


def test_nonfinite_output_gradient_is_rejected(server):
    """1e30 * u at u = 1e-20: the objective is 1e20, dE/dY = 2e40 overflows
    in fp32.  The same message as the reference and no update."""
    g = load_golden('protocol')
    n, d = linear_unit(server, 0.0, 1e-20, 0.0)
    c = unit_cost(server, n, d, 1e30)
    with pytest.raises(wire.ServerError) as err:
        server.train(n, [c], 1, method=1, fresh=1, lr=0.01, log=1)
    assert str(err.value) == str(g['output_gradient_error'])
    assert_untouched(server.snapshot(n), g['output_gradient_before'], g['output_gradient_after'])
