"""Kernel-level parity of the HIP path against the oracle, through the C ABI.

Tolerances (fp32 on both sides, different summation orders):
  * linear step:            scaled error <= 2e-5 against a float64 product;
  * composition / adjoint:  scaled error <= 1e-4 against the oracle on the same
                            GPU-produced z (error relative to max(|x|, row rms));
  * epoch:                  loss rel <= 1e-4, outputs and gradients rel-L2 <= 1e-3
                            (the order-6 bar), typically ~1e-6.
"""
import functools

import numpy as np
import pytest

import oracle
from cpde_amd import hip, workloads as W
from helpers import rel_l2, scaled_error

pytestmark = pytest.mark.gpu

SCHEMAS = {
    '2var_order6': W.full_schema(2, 6),
    '3var_order4': W.full_schema(3, 4),
    '1var_order6': W.full_schema(1, 6),
    'poisson_xx_yy': W.closed_schema(2, [(2, 0), (0, 2)]),
    '2var_order2': W.full_schema(2, 2),
    'value_only': W.full_schema(2, 0),
}


def random_layer(device, schema, n, points, seed, scale=0.7):
    """One sigmoid layer fed by random full stacks: returns net, plan, data."""
    rng = np.random.default_rng(seed)
    V = schema.shape[1] - 1
    R = len(schema)
    neurons, linear = [V, n, 1], [1, 0, 1]
    w0 = np.concatenate([rng.uniform(-1, 1, n * V), rng.uniform(-.5, .5, n)]).astype(np.float32)
    w1 = np.concatenate([rng.uniform(-1, 1, n), [0.1]]).astype(np.float32)
    net = hip.Net(device, neurons, linear, [w0, w1])
    plan = hip.Plan(net, schema, points, True)
    data = (rng.standard_normal((R, points, V)) * scale).astype(np.float32)   # [row][sample][channel]
    buf = hip.Buffer.of(device, data)
    plan.activate(buf, points, np.arange(R, dtype=np.int32), 0, points)
    return net, plan, buf, data, [w0, w1]


def linear_step(schema, data, w0, n):
    """z = W x (+ b on the value row) in float64, (points, R, n)."""
    V = schema.shape[1] - 1
    W0 = w0[:n * V].reshape(V, n).T.astype(np.float64)
    want = np.einsum('iv,rpv->pri', W0, data.astype(np.float64))
    want[:, 0, :] += w0[n * V:]
    return want


@pytest.mark.parametrize('name', list(SCHEMAS))
def test_linear_step_and_composition(device, path, name):
    """Network-fused plans keep u (the jet of sigma'(z)) instead of z: there y
    and u are checked against the oracle on the float64 linear step; the other
    families keep z, checked against float64 and then y against the oracle on
    that z."""
    schema = SCHEMAS[name]
    R = schema.shape[0]
    n, points = 64, 37
    print(f'[case] composition {name} R={R} n={n} points={points}', flush=True)
    net, plan, buf, data, (w0, w1) = random_layer(device, schema, n, points, 7)
    plan.forward()
    device.synchronize()
    want = linear_step(schema, data, w0, n)
    if path in ('network', 'partition'):
        zref = hip.stack_to_reference(want).reshape(R, -1).astype(np.float32)
        uref = oracle.compose_prime(schema, zref).reshape(R, points, n)
        u1 = hip.stack_to_reference(plan.unscaled_stack(1, 3))
        err = scaled_error(u1, uref, axis=(1, 2))
        print(f'[result] {name} sigma-prime jet scaled error {err:.3e}', flush=True)
        assert err < 1e-4
    else:
        z1 = plan.stack(1, 0)                   # (points, R, n)
        assert scaled_error(z1, want) < 2e-5
        zref = hip.stack_to_reference(z1).reshape(R, -1)
    y1 = plan.unscaled_stack(1, 1)
    yref = oracle.compose(schema, zref).reshape(R, points, n)
    err = scaled_error(hip.stack_to_reference(y1), yref, axis=(1, 2))
    print(f'[result] {name} composition scaled error {err:.3e}', flush=True)
    assert err < 1e-4
    plan.destroy(); net.destroy(); buf.free()


@pytest.mark.parametrize('name', list(SCHEMAS))
def test_adjoint_composition(device, path, name):
    schema = SCHEMAS[name]
    R = schema.shape[0]
    n, points = 64, 29
    print(f'[case] adjoint {name} R={R}', flush=True)
    net, plan, buf, data, (w0, w1) = random_layer(device, schema, n, points, 11)
    rng = np.random.default_rng(3)
    target = rng.standard_normal((R, points, 1)).astype(np.float32)
    tbuf = hip.Buffer.of(device, target)
    trows = hip.Buffer.of(device, np.arange(R, dtype=np.int32))
    wts = hip.Buffer.of(device, np.linspace(0.5, 1.5, R).astype(np.float32))
    device.costs_begin(1)
    plan.forward()
    plan.matching(tbuf, points, trows, wts, 1, 0, points, 0)
    plan.backward(False)
    device.synchronize()
    if path in ('network', 'partition'):  # z is not kept: the float64 linear step stands in
        z1 = hip.stack_to_reference(linear_step(schema, data, w0, n)).reshape(R, -1).astype(np.float32)
    else:
        z1 = hip.stack_to_reference(plan.stack(1, 0)).reshape(R, -1)
    g2 = plan.unscaled_stack(2, 2)[:, :, 0].astype(np.float64)         # (points, R)
    gy = np.einsum('i,pr->rpi', w1[:n].astype(np.float64), g2).reshape(R, -1).astype(np.float32)
    gz_ref = oracle.compose_adjoint(schema, z1, gy).reshape(R, points, n)
    gz = hip.stack_to_reference(plan.unscaled_stack(1, 2))
    err = scaled_error(gz, gz_ref, axis=(1, 2))
    print(f'[result] {name} adjoint scaled error {err:.3e}', flush=True)
    assert err < 1e-4
    for b in (tbuf, trows, wts, buf):
        b.free()
    plan.destroy(); net.destroy()


def small_workload(order, neurons, points, seed=5):
    schema = W.full_schema(2, order)
    rng = np.random.default_rng(seed)
    pts = rng.uniform(0, 1, (points, 2))
    freq, coef, phase = W.fourier_modes(2, 4, 3, seed)
    target = W.fourier_target(pts, schema, freq, coef, phase)
    return W.MatchingWorkload('small', neurons, pts, schema, target, 1.0 / target.var(axis=1),
                              W.xavier_weights(neurons, seed))


@pytest.mark.parametrize('order,neurons,points,chunk', [
    (6, [2, 32, 32, 1], 50, 0),
    (6, [2, 32, 32, 1], 50, 16),
    (2, [2, 48, 40, 24, 1], 101, 0),
    (4, [2, 16, 1], 64, 25),
    (5, [2, 80, 96, 1], 4101, 0),   # a long grid: two points per workgroup, one LDS tile, a lone last point
])
def test_epoch_matches_oracle(device, path, order, neurons, points, chunk):
    print(f'[case] epoch path={path} order={order} neurons={neurons} points={points} chunk={chunk}', flush=True)
    wl = small_workload(order, neurons, points)
    run = hip.MatchingRun(device, wl, chunk=chunk or None)
    run.step()
    device.synchronize()
    loss = run.loss()
    grads = run.gradients()
    ref_loss, ref_grads = oracle_epoch(order, tuple(neurons), points, chunk)
    print(f'[result] loss {loss!r} oracle {ref_loss!r}', flush=True)
    assert abs(loss / ref_loss - 1) < 1e-4
    for t, (g, r) in enumerate(zip(grads, ref_grads)):
        e = rel_l2(g, r)
        print(f'[result] transition {t} gradient rel-L2 {e:.3e}', flush=True)
        assert e < 1e-3
    run.close()


@pytest.mark.parametrize('order,neurons,points', [
    (4, [2, 128, 128, 1], 729),   # 64x64 tiles over short splits: direct tiles by default
    (0, [2, 128, 128, 128, 1], 729),  # one row: 64-column splits
    (6, [2, 64, 48, 1], 300),
    (3, [2, 30, 18, 1], 101),     # widths that are not multiples of 4: scalar operand loads
    (2, [2, 80, 96, 40, 1], 2000),
])
def test_weight_gradient_tile_forms(device, monkeypatch, order, neurons, points):
    """The weight gradient's direct tiles (operands from global memory straight
    into the matrix cores) and LDS-staged tiles, forced in turn
    (CPDE_WGRAD_DIRECT 2 and 0): each against the oracle, and the two within
    fp32 summation-order noise of each other."""
    print(f'[case] wgrad forms order={order} neurons={neurons} points={points}', flush=True)
    wl = small_workload(order, neurons, points)
    ref_loss, ref_grads = oracle_epoch(order, tuple(neurons), points, 0)
    got = {}
    for form in ('2', '0'):
        monkeypatch.setenv('CPDE_WGRAD_DIRECT', form)
        run = hip.MatchingRun(device, wl)
        run.step()
        device.synchronize()
        got[form] = run.gradients()
        assert abs(run.loss() / ref_loss - 1) < 1e-4
        run.close()
        for t, (g, r) in enumerate(zip(got[form], ref_grads)):
            e = rel_l2(g, r)
            print(f'[result] form {form} transition {t} gradient rel-L2 {e:.3e}', flush=True)
            assert e < 1e-3
    for a, b in zip(got['2'], got['0']):
        assert rel_l2(a, b) < 1e-5


@pytest.mark.parametrize('order,neurons,points,one_pass', [
    (6, [2, 64, 48, 32, 1], 61, '1'),     # one-pass epoch, scaled rows on three hidden layers
    (2, [2, 64, 64, 64, 1], 300, '1'),    # several points per workgroup
    (3, [2, 80, 96, 1], 97, '0'),         # separate forward and backward launches
    (0, [2, 64, 64, 64, 1], 256, '1'),    # the Poisson boundary leaf's shape: one row, eight points per workgroup
])
def test_weight_gradient_inside_the_backward(device, monkeypatch, order, neurons, points, one_pass):
    """Hidden transitions' weight-gradient partials written by the network
    backward itself (CPDE_INKERNEL_WGRAD=1) against the separate
    weight-gradient launch (=0): the same loss bit for bit, gradients within
    fp32 summation-order noise, and both against the oracle."""
    print(f'[case] in-kernel wgrad order={order} neurons={neurons} points={points} one_pass={one_pass}', flush=True)
    monkeypatch.setenv('CPDE_ONE_PASS', one_pass)
    wl = small_workload(order, neurons, points)
    ref_loss, ref_grads = oracle_epoch(order, tuple(neurons), points, 0)
    got, losses = {}, {}
    for form in ('1', '0'):
        monkeypatch.setenv('CPDE_INKERNEL_WGRAD', form)
        run = hip.MatchingRun(device, wl)
        run.step()
        device.synchronize()
        got[form], losses[form] = run.gradients(), run.loss()
        run.close()
        assert abs(losses[form] / ref_loss - 1) < 1e-4
        for t, (g, r) in enumerate(zip(got[form], ref_grads)):
            e = rel_l2(g, r)
            print(f'[result] in-kernel {form} transition {t} gradient rel-L2 {e:.3e}', flush=True)
            assert e < 1e-3
    assert losses['1'] == losses['0']
    for a, b in zip(got['1'], got['0']):
        assert rel_l2(a, b) < 1e-5


PAIRED_ALIASED = dict(CPDE_FUSED='2', CPDE_NET_POINTS='2', CPDE_NET_ALIAS='1', CPDE_NET_COLTILE='16',
                      CPDE_NET_SPLIT='1', CPDE_NET_SPLIT_ADJOINT='1')


@pytest.mark.parametrize('order,neurons,points', [
    (5, [2, 80, 96, 1], 4101),   # more workgroups than co-reside: separate forward and backward launches
    (5, [2, 80, 96, 1], 301),    # co-resident: the one-pass epoch, its cost scratch apart from the tiles
    (3, [2, 48, 32, 1], 257),    # few rows: two points share one 16-column tile pair
])
def test_paired_aliased_network_forms(device, monkeypatch, order, neurons, points):
    """The network kernels' two-points-per-workgroup, one-LDS-tile form forced
    by its tuning variables (by default it is chosen only on long grids of
    many-row points, depending on the CU count), with an odd point count so the
    last workgroup holds a lone point."""
    for k, v in PAIRED_ALIASED.items():
        monkeypatch.setenv(k, v)
    print(f'[case] paired aliased order={order} neurons={neurons} points={points}', flush=True)
    wl = small_workload(order, neurons, points)
    run = hip.MatchingRun(device, wl)
    run.step()
    device.synchronize()
    loss, grads = run.loss(), run.gradients()
    ref_loss, ref_grads = oracle_epoch(order, tuple(neurons), points, 0)
    print(f'[result] loss {loss!r} oracle {ref_loss!r}', flush=True)
    assert abs(loss / ref_loss - 1) < 1e-4
    for t, (g, r) in enumerate(zip(grads, ref_grads)):
        e = rel_l2(g, r)
        print(f'[result] transition {t} gradient rel-L2 {e:.3e}', flush=True)
        assert e < 1e-3
    run.close()


@pytest.mark.parametrize('order,neurons,points,per_block', [
    (6, [2, 128, 128, 128, 1], 100, 3),   # one-pass epoch, three points per 512-lane workgroup
    (4, [2, 64, 48, 1], 61, 2),
    (5, [2, 80, 96, 1], 4101, 2),         # separate forward and backward launches
])
def test_network_kernels_with_eight_waves(device, monkeypatch, order, neurons, points, per_block):
    """The network kernels on 512-lane workgroups (CPDE_NET_THREADS=512: eight
    waves share the products' row blocks) against the oracle."""
    monkeypatch.setenv('CPDE_FUSED', '2')
    monkeypatch.setenv('CPDE_NET_THREADS', '512')
    monkeypatch.setenv('CPDE_NET_POINTS', str(per_block))
    print(f'[case] eight waves order={order} neurons={neurons} points={points} per_block={per_block}', flush=True)
    wl = small_workload(order, neurons, points)
    run = hip.MatchingRun(device, wl)
    run.step()
    device.synchronize()
    loss, grads = run.loss(), run.gradients()
    ref_loss, ref_grads = oracle_epoch(order, tuple(neurons), points, 0)
    print(f'[result] loss {loss!r} oracle {ref_loss!r}', flush=True)
    assert abs(loss / ref_loss - 1) < 1e-4
    for t, (g, r) in enumerate(zip(grads, ref_grads)):
        assert rel_l2(g, r) < 1e-3, t
    run.close()


@pytest.mark.parametrize('order,neurons,points,split', [
    (6, [2, 128, 128, 1], 61, '2'),   # 28 rows: the scaled forward split over mirror lanes
    (5, [2, 64, 48, 32, 1], 40, '2'),
    (3, [2, 64, 64, 1], 300, '1'),    # several points per workgroup, whole compositions per lane
])
def test_network_kernels_composition_split(device, monkeypatch, order, neurons, points, split):
    """The network kernels with the forward compositions split over lanes
    (CPDE_NET_SPLIT=2, one point per workgroup: whole compositions are the
    default there) and unsplit where a split is the default, against the
    oracle."""
    monkeypatch.setenv('CPDE_FUSED', '2')
    monkeypatch.setenv('CPDE_NET_SPLIT', split)
    print(f'[case] composition split order={order} neurons={neurons} points={points} split={split}', flush=True)
    wl = small_workload(order, neurons, points)
    run = hip.MatchingRun(device, wl)
    run.step()
    device.synchronize()
    loss, grads = run.loss(), run.gradients()
    ref_loss, ref_grads = oracle_epoch(order, tuple(neurons), points, 0)
    print(f'[result] loss {loss!r} oracle {ref_loss!r}', flush=True)
    assert abs(loss / ref_loss - 1) < 1e-4
    for t, (g, r) in enumerate(zip(grads, ref_grads)):
        assert rel_l2(g, r) < 1e-3, t
    run.close()


@functools.lru_cache(maxsize=None)
def oracle_epoch(order, neurons, points, chunk):
    """The oracle's epoch of small_workload, computed once for all kernel families."""
    wl = small_workload(order, list(neurons), points)
    loss, grads, _ = oracle.matching_epoch(wl.neurons, wl.linear, wl.init, wl.schema, wl.inputs.transpose(0, 2, 1),
                                           wl.target[:, :, None], wl.row_weights[:, None, None], chunk=chunk)
    return loss, grads


@pytest.mark.parametrize('order,neurons,points,chunk,one_pass', [
    (4, [2, 32, 24, 3], 45, 0, True),
    (4, [2, 32, 24, 3], 45, 20, False),
    (3, [3, 16, 16, 2], 33, 16, True),
    (6, [2, 32, 32, 8], 20, 0, True),
    (6, [3, 24, 16, 2], 10, 0, True),     # 84 rows: beyond the network kernels' 64
    (2, [2, 320, 2], 20, 0, True),        # hidden width beyond the network kernels' 256
    (1, [2, 1040, 1], 8, 0, True),        # and beyond the layer-fused kernels' 1024
])
def test_multi_output_epoch_matches_oracle(device, path, order, neurons, points, chunk, one_pass):
    """Networks with several outputs (up to the eight the output layer takes):
    per-channel targets and row weights in the wire layouts [row][sample][channel]
    and [row][weight sample][channel], ragged last chunks, one-pass and separate
    launches."""
    print(f'[case] multi-output path={path} order={order} neurons={neurons} points={points} chunk={chunk} '
          f'one_pass={one_pass}', flush=True)
    V, n_out = neurons[0], neurons[-1]
    schema = W.full_schema(V, order)
    R = len(schema)
    pts = np.random.default_rng(11).uniform(0, 1, (points, V))
    target = np.stack([W.fourier_target(pts, schema, *W.fourier_modes(V, 3, 2, 40 + c)) for c in range(n_out)],
                      axis=2).astype(np.float32)                                   # (R, points, n_out)
    row_weights = (1.0 / target.var(axis=1, dtype=np.float64))[:, None, :].astype(np.float32)   # (R, 1, n_out)
    x = np.ascontiguousarray(W.input_stack(pts, schema).transpose(0, 2, 1), np.float32)      # (R, points, V)
    init = W.xavier_weights(neurons, 21)
    width = chunk or points
    net = hip.Net(device, neurons, W.linear_flags(neurons), init)
    plan = hip.Plan(net, schema, width, True)
    bufs = [hip.Buffer.of(device, a) for a in
            (x, target, np.arange(R, dtype=np.int32), row_weights)]
    data, tbuf, trows, wts = bufs
    rows = np.arange(R, dtype=np.int32)
    device.costs_begin(1)
    for offset in range(0, points, width):
        valid = min(width, points - offset)
        plan.activate(data, points, rows, offset, valid)
        if one_pass:
            plan.epoch_matching(tbuf, points, trows, wts, 1, offset, valid, 0, True, offset > 0)
        else:
            plan.forward()
            plan.matching(tbuf, points, trows, wts, 1, offset, valid, 0, True, True)
            plan.backward(offset > 0)
    device.synchronize()
    loss = device.scalars(1, 0)[0][0].value
    grads = [net.gradient(t) for t in range(len(neurons) - 1)]
    ref_loss, ref_grads, _ = oracle.matching_epoch(neurons, W.linear_flags(neurons), init, schema, x, target,
                                                   row_weights, chunk=chunk)
    print(f'[result] loss {loss!r} oracle {ref_loss!r}', flush=True)
    assert abs(loss / ref_loss - 1) < 1e-4
    for t, (g, r) in enumerate(zip(grads, ref_grads)):
        e = rel_l2(g, r)
        print(f'[result] transition {t} gradient rel-L2 {e:.3e}', flush=True)
        assert e < 1e-3
    for b in bufs:
        b.free()
    plan.destroy()
    net.destroy()


def test_deep_network_beyond_one_gradient_group(device):
    """41 transitions (the protocol takes up to 255): more than one grouped
    weight-gradient launch and reduction (32 transitions each), then RPROP and
    the gradient statistics over two launch groups as well.  Loss and every
    gradient against the oracle; the first RPROP step bit-exact against the
    oracle's on our gradients."""
    neurons = [2] + [6] * 40 + [1]
    print(f'[case] deep network {len(neurons) - 1} transitions', flush=True)
    wl = small_workload(1, neurons, 20, seed=9)
    # wide enough initial weights that the signal survives forty layers
    wl.init = [w * 3 for w in wl.init]
    run = hip.MatchingRun(device, wl)
    run.step()
    device.synchronize()
    loss, grads = run.loss(), run.gradients()
    ref_loss, ref_grads, _ = oracle.matching_epoch(wl.neurons, wl.linear, wl.init, wl.schema,
                                                   wl.inputs.transpose(0, 2, 1), wl.target[:, :, None],
                                                   wl.row_weights[:, None, None], outputs=False)
    print(f'[result] loss {loss!r} oracle {ref_loss!r}', flush=True)
    assert abs(loss / ref_loss - 1) < 1e-4
    errs = [rel_l2(g, r) for g, r in zip(grads, ref_grads)]
    print(f'[result] worst gradient rel-L2 {max(errs):.3e}', flush=True)
    assert max(errs) < 1e-3
    run.net.inspect_gradients()
    stats = device.scalars(0, len(neurons) - 1)[1]
    for s, g in zip(stats, grads):
        assert s.nonfinite_count == 0
        assert s.max_abs == np.abs(g).max()
    before = [run.net.state(t, 0) for t in range(len(neurons) - 1)]
    run.net.rprop()
    for t, (w, g) in enumerate(zip(before, grads)):
        rW, _, _, _ = oracle.rprop(w, np.full_like(w, 0.002), g, np.zeros_like(w))
        np.testing.assert_array_equal(run.net.state(t, 0), rW)
    run.close()


def test_oversized_chunk_is_rejected(device):
    """A chunk whose (point, row) pairs would overflow the kernels' 32-bit
    indexing is refused at plan creation, before any allocation, and the
    network stays usable."""
    neurons = [2, 8, 1]
    net = hip.Net(device, neurons, W.linear_flags(neurons), W.xavier_weights(neurons, 1))
    with pytest.raises(hip.CpdeError, match='chunk too large'):
        hip.Plan(net, W.full_schema(2, 6), 1 << 26, True)
    plan = hip.Plan(net, W.full_schema(2, 6), 64, True)
    plan.destroy()
    net.destroy()
