"""Optimizer parity on the GPU.

* Crafted states through the C ABI: weights, steps and both gradient buffers
  are written through the state pointers so that every RPROP transition is
  taken (growth x1.2, rollback x0.5, plain step, zero gradient, a step
  rejected at |w| > 20, float products that underflow to zero, infinities),
  then cpde_rprop / cpde_set_steps / cpde_restore_steps / cpde_adam (and
  cpde_scalars_download_rprop, which updates only on clean scalars) run once
  and must match the oracle bit for bit (the oracle's optimizers are pinned
  against the reference server's trajectories in test_oracle_optimizer.py).
* The protocol server against the reference server's optimizer trajectories
  (tests/golden/optimizer.npz): per epoch from the reference's own state, and
  free running.  RPROP weights and steps must be bit-identical wherever the
  gradient is sure (above 1e-3 of its largest entry): sign decisions
  bit-exact wherever the gradient exceeds the tolerance.
"""
import numpy as np
import pytest

import oracle
from cpde_amd import hip, wire
from cpde_amd import workloads as W
from cpde_amd.build import SERVER
from helpers import golden_workload, load_golden, rel_l2

pytestmark = pytest.mark.gpu

SINGLE_LEAF = wire.graph_bytes([(1, 0, 0)], [0.0], 0)
NEURONS = [3, 40, 33, 7, 2]


def crafted(count, seed):
    """Weights, steps, current and previous gradients that reach every RPROP
    transition (cuda/derivative_kernels_v4.cu:752-778)."""
    rng = np.random.default_rng(seed)
    W_ = rng.uniform(-1.5, 1.5, count)
    S = 10.0 ** rng.uniform(-5, -0.5, count)
    mag = 10.0 ** rng.uniform(-6, 3, (2, count))
    g, gi = mag * rng.choice([-1.0, 1.0], (2, count))
    kind = rng.integers(0, 10, count)
    g[kind == 0] = 0.0                                    # no gradient: nothing moves
    gi[kind == 1] = 0.0                                   # no history: plain step
    # near the bound: the outward step is rejected (step -> 0.1), the inward kept
    edge = kind == 2
    W_[edge] = rng.choice([-19.99, 19.99, -20.0, 20.0], edge.sum())
    S[edge] = rng.uniform(0.005, 0.05, edge.sum())
    # products that underflow to +-0 in fp32 although both signs are set
    tiny = kind == 3
    g[tiny] = 1e-25 * rng.choice([-1.0, 1.0], tiny.sum())
    gi[tiny] = 1e-24 * rng.choice([-1.0, 1.0], tiny.sum())
    # subnormal gradients, infinite gradients
    g[kind == 4] = 1e-40 * rng.choice([-1.0, 1.0], (kind == 4).sum())
    inf = kind == 5
    g[inf] = np.inf * rng.choice([-1.0, 1.0], inf.sum())
    return [np.asarray(a, np.float32) for a in (W_, S, g, gi)]


@pytest.fixture
def net(device):
    n = hip.Net(device, NEURONS, W.linear_flags(NEURONS), W.xavier_weights(NEURONS, 2))
    yield n
    n.destroy()


def load_state(net, t, W_, S, ga, gi):
    act = net.active(t)
    net.set_state(t, 0, W_)
    net.set_state(t, 3, S)
    net.set_state(t, act, ga)
    net.set_state(t, 3 - act, gi)


def test_rprop_every_transition_bit_exact(device, net):
    T = len(NEURONS) - 1
    states = []
    for t in range(T):
        count = NEURONS[t + 1] * (NEURONS[t] + 1)
        st = crafted(count, 100 + t)
        load_state(net, t, *st)
        states.append((net.active(t), st))
    net.rprop()
    device.synchronize()
    for t, (act, (W_, S, ga, gi)) in enumerate(states):
        rW, rS, rga, rgi = oracle.rprop(W_, S, ga, gi)
        print(f'[case] rprop transition {t}: {W_.size} entries, rejected at the bound '
              f'{int(((rS == 0.1) & (S != 0.1)).sum())}, rolled back {int((ga * gi < 0).sum())}', flush=True)
        assert net.active(t) == 3 - act
        np.testing.assert_array_equal(net.state(t, 0), rW)
        np.testing.assert_array_equal(net.state(t, 3), rS)
        np.testing.assert_array_equal(net.state(t, act), rga)
        np.testing.assert_array_equal(net.state(t, 3 - act), rgi)


def test_download_rprop_updates_only_on_clean_scalars(device, net):
    """cpde_scalars_download_rprop: with every gradient finite, the weights,
    steps, both gradient buffers and the buffer switch of cpde_rprop, bit for
    bit against the oracle, and updated = 1; with infinite gradient entries
    (the crafted states' own), nothing changes and updated = 0 -- the state a
    rejected epoch keeps."""
    T = len(NEURONS) - 1
    for clean in (True, False):
        states = []
        for t in range(T):
            count = NEURONS[t + 1] * (NEURONS[t] + 1)
            st = crafted(count, 300 + t)
            if clean:
                st[2][~np.isfinite(st[2])] = np.float32(1.5)
            load_state(net, t, *st)
            states.append((net.active(t), st))
        net.inspect_gradients()
        _, grads, updated = net.download_rprop(0)
        device.synchronize()
        nonfinite = sum(g.nonfinite_count for g in grads)
        print(f'[case] download_rprop clean={clean}: non-finite gradient entries {nonfinite}, updated {updated}',
              flush=True)
        assert updated == (1 if clean else 0)
        assert (nonfinite == 0) == clean
        for t, (act, (W_, S, ga, gi)) in enumerate(states):
            if clean:
                rW, rS, rga, rgi = oracle.rprop(W_, S, ga, gi)
                assert net.active(t) == 3 - act
            else:
                rW, rS, rga, rgi = W_, S, ga, gi
                assert net.active(t) == act
            np.testing.assert_array_equal(net.state(t, 0), rW)
            np.testing.assert_array_equal(net.state(t, 3), rS)
            np.testing.assert_array_equal(net.state(t, act), rga)
            np.testing.assert_array_equal(net.state(t, 3 - act), rgi)


@pytest.mark.parametrize('stats', ['full', 'short'])
@pytest.mark.parametrize('method', [0, 1], ids=['rprop', 'adam'])
@pytest.mark.parametrize('neurons', [NEURONS, [2, 128, 128, 128, 1]], ids=['tested', 'separate'])
def test_inspecting_update_matches_inspect_then_update(device, neurons, method, stats):
    """cpde_inspect_update_issue against cpde_inspect_gradients followed by
    cpde_update_issue on the same crafted states, clean and with infinite
    gradient entries: the same verdict and the same states, bit for bit.  The
    gradient totals are the same too, except where the update launch tested the
    gradients itself (3->40->33->7->2, 1,767 entries, short statistics asked
    for): then each transition's non-finite count is 1 if it has any non-finite
    entry, and the rest is left empty.  2->128->128->128->1 (33,537 entries in
    133 chunks of 256) is beyond the launch's chunk table of 40 and runs both
    launches."""
    T = len(neurons) - 1
    nets = [hip.Net(device, neurons, W.linear_flags(neurons), W.xavier_weights(neurons, 2)) for _ in range(2)]
    for clean in (True, False):
        for t in range(T):
            st = crafted(neurons[t + 1] * (neurons[t] + 1), 500 + t)
            if clean:
                st[2][~np.isfinite(st[2])] = np.float32(1.5)
            for n in nets:
                load_state(n, t, *st)
        nets[0].inspect_gradients()
        nets[0].issue_update(0, method, 1, 0.01)
        _, g0, u0 = nets[0].resolve_update(0)
        nets[1].issue_update(0, method, 1, 0.01, inspect=stats)
        _, g1, u1 = nets[1].resolve_update(0)
        device.synchronize()
        print(f'[case] neurons={neurons} method={method} stats={stats} clean={clean}: updated {u0} / {u1}, '
              f'non-finite {[g.nonfinite_count for g in g0]} / {[g.nonfinite_count for g in g1]}', flush=True)
        assert u0 == u1 == (1 if clean else 0)
        short = stats == 'short' and neurons == NEURONS
        for a, b in zip(g0, g1):
            if short:
                assert (b.nonfinite_count, b.first_nonfinite, b.squared_norm, b.max_abs) == \
                    (int(a.nonfinite_count > 0), 2**31 - 1, 0.0, 0.0)
            else:
                assert (a.nonfinite_count, a.first_nonfinite, a.squared_norm, a.max_abs) == \
                    (b.nonfinite_count, b.first_nonfinite, b.squared_norm, b.max_abs)
        for t in range(T):
            assert nets[0].active(t) == nets[1].active(t)
            for k in range(4):
                np.testing.assert_array_equal(nets[0].state(t, k), nets[1].state(t, k))
    for n in nets:
        n.destroy()


@pytest.mark.parametrize('mode', ['set', 'restore'])
def test_set_and_restore_steps_bit_exact(device, net, mode):
    T = len(NEURONS) - 1
    value = np.float32(1e-3)
    states = []
    for t in range(T):
        count = NEURONS[t + 1] * (NEURONS[t] + 1)
        W_, S, ga, gi = crafted(count, 200 + t)
        S[::7] = value                        # exactly at the floor: kept, histories kept
        load_state(net, t, W_, S, ga, gi)
        states.append((net.active(t), S, ga, gi))
    (net.set_steps if mode == 'set' else net.restore_steps)(float(value))
    device.synchronize()
    for t, (act, S, ga, gi) in enumerate(states):
        f = oracle.set_steps if mode == 'set' else oracle.restore_steps
        rS, rga, rgi = f(value, S, ga, gi)
        np.testing.assert_array_equal(net.state(t, 3), rS)
        np.testing.assert_array_equal(net.state(t, act), rga)
        np.testing.assert_array_equal(net.state(t, 3 - act), rgi)
        assert net.active(t) == act


def test_adam_bit_exact(device, net):
    """Adam step 3 from crafted moments: weights and both moments bit-identical
    to the oracle (fp32 moments without contraction, correctly rounded fp32
    division and square root, the update in double as the reference's double
    epsilon makes it)."""
    T = len(NEURONS) - 1
    rng = np.random.default_rng(7)
    states = []
    for t in range(T):
        count = NEURONS[t + 1] * (NEURONS[t] + 1)
        W_ = rng.uniform(-2, 2, count).astype(np.float32)
        W_[::11] = 19.9999                    # updates beyond the bound are dropped
        g = (rng.standard_normal(count) * 10.0 ** rng.uniform(-4, 1, count)).astype(np.float32)
        m = (rng.standard_normal(count) * 0.1).astype(np.float32)
        v = (rng.uniform(0, 1, count) * 0.01).astype(np.float32)
        act = net.active(t)
        net.set_state(t, 0, W_)
        net.set_state(t, act, g)
        net.set_state(t, 3, m)
        net.set_state(t, 3 - act, v)
        states.append((act, W_, g, m, v))
    net.adam(3, 0.01)
    device.synchronize()
    for t, (act, W_, g, m, v) in enumerate(states):
        rW, rm, rv = oracle.adam(W_, g, m, v, np.float32(0.01), 3)
        got = net.state(t, 0)
        ulp = np.abs(got.view(np.int32).astype(np.int64) - rW.view(np.int32).astype(np.int64)).max()
        print(f'[result] adam transition {t}: max weight difference {ulp} ulp', flush=True)
        np.testing.assert_array_equal(net.state(t, 3), rm)
        np.testing.assert_array_equal(net.state(t, 3 - act), rv)
        np.testing.assert_array_equal(got, rW)
        np.testing.assert_array_equal(net.state(t, act), g)


# ------------------------------------------------------------------ server trajectories
@pytest.fixture(scope='module')
def server():
    if not SERVER.exists():
        pytest.fail('protocol server not built: python -m cpde_amd.build')
    s = wire.Session(SERVER)
    yield s
    s.close()


RUNS = {
    'rprop': (dict(method=0, fresh=1), dict(method=0, fresh=0)),
    'bigstep': (dict(method=0, fresh=1, steps=0.05), dict(method=0, fresh=0)),
    'restore': (dict(method=0, fresh=1, steps=2e-4, restore_every=2, restore_step=1e-3),
                dict(method=0, fresh=0, restore_every=2, restore_step=1e-3)),
}


def sure(grad):
    return np.abs(grad) > 1e-3 * np.abs(grad).max()


@pytest.mark.parametrize('prefix', list(RUNS))
def test_rprop_decisions_from_reference_states(server, prefix):
    """Every epoch starts from the reference's own state after the previous
    epoch (op 10): the weights and steps after our update must equal the
    reference's bit for bit wherever the reference gradient is sure, and the
    metadata exactly."""
    g = load_golden('optimizer')
    wl = golden_workload(g)
    ids = wl.upload(server, int(g['chunk']))
    first, later = RUNS[prefix]
    checked = total = 0
    for k in range(int(g[f'{prefix}_epochs'])):
        if k:
            server.restore(ids['net'], bytes(g[f'{prefix}_state{k - 1}']))
        server.train(ids['net'], [ids['cost']], 1, log=1, **(first if k == 0 else later))
        meta, layers = wire.decode_state(server.snapshot(ids['net']))
        ref_meta, ref_layers = wire.decode_state(bytes(g[f'{prefix}_state{k}']))
        assert meta == ref_meta
        for t, (a, b) in enumerate(zip(layers, ref_layers)):
            mask = sure(g[f'{prefix}_grad{k}_{t}'])
            np.testing.assert_array_equal(a['buffers'][0][mask], b['buffers'][0][mask], err_msg=f'epoch {k} W{t}')
            np.testing.assert_array_equal(a['buffers'][3][mask], b['buffers'][3][mask], err_msg=f'epoch {k} S{t}')
            assert a['active'] == b['active']
            checked += int(mask.sum())
            total += mask.size
    print(f'[result] {prefix}: {checked} of {total} updates checked bit-exact', flush=True)
    assert checked > 0.8 * total


@pytest.mark.parametrize('prefix', list(RUNS))
def test_rprop_trajectory_free_running(server, prefix):
    """The same epochs without restoring: our own state carries from epoch to
    epoch.  An entry stays checked while its gradient has been sure at every
    epoch so far (one unsure decision may move it differently); those entries'
    weights and steps must be bit-identical, all weights close."""
    g = load_golden('optimizer')
    wl = golden_workload(g)
    ids = wl.upload(server, int(g['chunk']))
    first, later = RUNS[prefix]
    masks = None
    for k in range(int(g[f'{prefix}_epochs'])):
        server.train(ids['net'], [ids['cost']], 1, log=1, **(first if k == 0 else later))
        meta, layers = wire.decode_state(server.snapshot(ids['net']))
        ref_meta, ref_layers = wire.decode_state(bytes(g[f'{prefix}_state{k}']))
        assert meta == ref_meta
        step_masks = [sure(g[f'{prefix}_grad{k}_{t}']) for t in range(len(layers))]
        masks = step_masks if masks is None else [m & s for m, s in zip(masks, step_masks)]
        for t, (a, b, mask) in enumerate(zip(layers, ref_layers, masks)):
            np.testing.assert_array_equal(a['buffers'][0][mask], b['buffers'][0][mask], err_msg=f'epoch {k} W{t}')
            np.testing.assert_array_equal(a['buffers'][3][mask], b['buffers'][3][mask], err_msg=f'epoch {k} S{t}')
            assert rel_l2(a['buffers'][0], b['buffers'][0]) < 1e-4
    kept = sum(int(m.sum()) for m in masks) / sum(m.size for m in masks)
    print(f'[result] {prefix}: {kept:.3f} of the entries sure at every epoch', flush=True)
    assert kept > 0.5


def test_adam_from_reference_states(server):
    """Adam epochs from the reference's states: metadata exact, weights,
    first and second moments at the gradient bars."""
    g = load_golden('optimizer')
    wl = golden_workload(g)
    ids = wl.upload(server, int(g['chunk']))
    for k in range(int(g['adam_epochs'])):
        if k:
            server.restore(ids['net'], bytes(g[f'adam_state{k - 1}']))
        server.train(ids['net'], [ids['cost']], 1, log=1, method=1, fresh=int(k == 0), lr=0.01 if k == 0 else 0.0)
        meta, layers = wire.decode_state(server.snapshot(ids['net']))
        ref_meta, ref_layers = wire.decode_state(bytes(g[f'adam_state{k}']))
        assert meta == ref_meta
        for a, b in zip(layers, ref_layers):
            assert rel_l2(a['buffers'][0], b['buffers'][0]) < 1e-5
            assert rel_l2(a['buffers'][3], b['buffers'][3]) < 1e-3      # m
            assert rel_l2(a['buffers'][2], b['buffers'][2]) < 2e-3      # v
            assert rel_l2(a['buffers'][1], b['buffers'][1]) < 1e-3      # the gradient


def fourier_case(order, neurons, points, seed=9):
    schema = W.full_schema(neurons[0], order)
    rng = np.random.default_rng(seed)
    pts = rng.uniform(0, 1, (points, neurons[0]))
    freq, coef, phase = W.fourier_modes(neurons[0], 4, 3, seed)
    target = W.fourier_target(pts, schema, freq, coef, phase)
    return W.MatchingWorkload('fused', neurons, pts, schema, target, 1.0 / target.var(axis=1),
                              W.xavier_weights(neurons, seed))


@pytest.mark.parametrize('order, neurons, points, chunk, one_pass', [
    (6, [2, 64, 48, 1], 61, 0, '1'),        # one chunk, one-pass epoch
    (3, [2, 40, 40, 40, 1], 300, 128, '1'),  # three chunks: the update rides in the last one's reduction
    (2, [3, 32, 24, 1], 90, 0, '0'),        # no one-pass epoch: separate launches, then RPROP
])
def test_epoch_with_fused_rprop_matches_separate_update(device, monkeypatch, order, neurons, points, chunk, one_pass):
    """cpde_epoch_matching_rprop (the split reduction and RPROP in one launch)
    leaves weights, steps, both gradient buffers and the row-major weight copy
    bit-identical to cpde_epoch_matching followed by cpde_rprop, over five
    epochs (growth, rollback and plain steps all occur)."""
    monkeypatch.setenv('CPDE_ONE_PASS', one_pass)
    print(f'[case] fused rprop order={order} neurons={neurons} points={points} chunk={chunk} one_pass={one_pass}',
          flush=True)
    wl = fourier_case(order, neurons, points)
    runs = [hip.MatchingRun(device, wl, chunk=chunk or None) for _ in range(2)]
    losses = [[], []]
    for _ in range(5):
        runs[0].step(update=False)
        runs[0].net.rprop()
        runs[1].step(update=True)
        for k in range(2):
            losses[k].append(runs[k].loss())
    device.synchronize()
    assert losses[0] == losses[1]
    for t in range(len(neurons) - 1):
        for b in range(4):
            np.testing.assert_array_equal(runs[1].net.state(t, b), runs[0].net.state(t, b))
        assert runs[0].net.active(t) == runs[1].net.active(t)
    for r in runs:
        r.close()
