"""cpde_epoch_matching_static, the matching epoch that allocates nothing,
through the C ABI: its cost records and weight-gradient split partials live in
the library's static device scratch.  It runs the same kernels as
cpde_epoch_matching, so loss and gradients must be bit-identical to it, on two
calls in a row with different shapes (the second smaller, chunked), and its
refusals must leave the library usable."""
import numpy as np
import pytest

from cpde_amd import hip, workloads as W

pytestmark = pytest.mark.gpu


def small_workload(order, neurons, points, seed):
    schema = W.full_schema(2, order)
    rng = np.random.default_rng(seed)
    pts = rng.uniform(0, 1, (points, 2))
    freq, coef, phase = W.fourier_modes(2, 4, 3, seed)
    target = W.fourier_target(pts, schema, freq, coef, phase)
    return W.MatchingWorkload('small', neurons, pts, schema, target, 1.0 / target.var(axis=1),
                              W.xavier_weights(neurons, seed))


def epoch(device, wl, chunk, static):
    run = hip.MatchingRun(device, wl, chunk=chunk, static_scratch=static)
    try:
        run.step()
        device.synchronize()
        return run.loss(), run.gradients()
    finally:
        run.close()


def test_static_epoch_equals_the_allocating_epoch(device):
    """Two static-scratch epochs in a row -- 300 points at order 6, then 77
    points at order 3 in chunks of 32 (three launches, the last ragged) --
    each against cpde_epoch_matching on the same inputs: loss and every
    gradient bit-identical."""
    cases = [(small_workload(6, [2, 64, 48, 1], 300, 5), None),
             (small_workload(3, [2, 32, 40, 1], 77, 6), 32)]
    for wl, chunk in cases:
        print(f'[case] static epoch order={int(wl.schema[-1][0])} neurons={wl.neurons} points={wl.size} '
              f'chunk={chunk}', flush=True)
        ref_loss, ref_grads = epoch(device, wl, chunk, False)
        loss, grads = epoch(device, wl, chunk, True)
        print(f'[result] loss {loss!r} allocating epoch {ref_loss!r}', flush=True)
        assert loss == ref_loss
        for g, r in zip(grads, ref_grads):
            np.testing.assert_array_equal(g, r)


def test_static_epoch_refusals(device, monkeypatch):
    """A plan without the one-pass epoch and a plan whose split partials
    exceed the static scratch are refused with CPDE_EINVAL; the allocating
    epoch still works afterwards."""
    wl = small_workload(2, [2, 16, 16, 1], 40, 7)
    monkeypatch.setenv('CPDE_ONE_PASS', '0')
    run = hip.MatchingRun(device, wl, static_scratch=True)
    with pytest.raises(hip.CpdeError, match='one-pass epoch applies') as err:
        run.step()
    assert err.value.code == hip.EINVAL
    run.close()
    monkeypatch.delenv('CPDE_ONE_PASS')
    # 1 -> 256^6 -> 1 on the value row over four workgroups per CU of 32
    # points, on the LDS-staged weight-gradient tiles: five 256x256
    # transitions at 25 splits need 33 MB of partials (the direct tiles, one
    # per CU, need under 8 MB here)
    monkeypatch.setenv('CPDE_WGRAD_DIRECT', '0')
    _, cus = device.info()
    neurons = [1] + [256] * 6 + [1]
    points = 128 * cus
    x = np.linspace(0, 1, points)[:, None]
    schema = W.full_schema(1, 0)
    big = W.MatchingWorkload('big', neurons, x, schema, np.sin(x.T), np.ones(1), W.xavier_weights(neurons, 8))
    run = hip.MatchingRun(device, big, static_scratch=True)
    with pytest.raises(hip.CpdeError, match='static scratch') as err:
        run.step()
    assert err.value.code == hip.EINVAL
    run.close()
    monkeypatch.delenv('CPDE_WGRAD_DIRECT')
    loss, grads = epoch(device, wl, None, False)
    loss2, grads2 = epoch(device, wl, None, True)
    assert loss == loss2
