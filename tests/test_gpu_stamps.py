"""Phase clock stamps of the one-pass matching epoch (CPDE_PHASE_STAMPS=1,
diagnostics read by cpde_amd/stamps.py)."""
import numpy as np
import pytest

from cpde_amd import hip, stamps, workloads as W


def small_workload():
    neurons = [2, 32, 32, 1]
    schema = W.full_schema(2, 6)
    pts = np.random.default_rng(1).uniform(0, 1, (40, 2))
    freq, coef, phase = W.fourier_modes(2, 4, 3, 1)
    target = W.fourier_target(pts, schema, freq, coef, phase)
    return W.MatchingWorkload('stamps', neurons, pts, schema, target, 1.0 / target.var(axis=1),
                              W.xavier_weights(neurons, 1))


def epoch(device, wl):
    run = hip.MatchingRun(device, wl)
    run.step()
    device.synchronize()
    loss, grads = run.loss(), run.gradients()
    R = len(wl.cost_schema)
    dest = hip.Buffer(device, R * wl.size * 4)
    run.plan.output(dest, wl.size, np.arange(R, dtype=np.int32), 0, wl.size)
    stack = dest.download(np.float32, R * wl.size).reshape(R, wl.size)
    dest.free()
    run.close()
    return loss, grads, stack


@pytest.mark.gpu
def test_phase_stamps_over_the_output_stack(device, monkeypatch):
    """Every block's output stack holds one increasing cycle stamp per phase
    (the phases cpde_amd.stamps names) and the real-time clock at the block's
    start and end; the epoch's loss and gradients are those of the kernel
    without stamps, bit for bit."""
    wl = small_workload()
    print(f'[case] stamps on 2->32->32->1, {wl.size} points, {len(wl.cost_schema)} rows', flush=True)
    loss0, grads0, _ = epoch(device, wl)
    monkeypatch.setenv('CPDE_PHASE_STAMPS', '1')
    loss1, grads1, stack = epoch(device, wl)
    assert loss1 == loss0
    for g0, g1 in zip(grads0, grads1):
        assert np.array_equal(g0, g1)
    n = len(stamps.phase_names(wl.neurons))
    u = stack.view(np.uint32).astype(np.int64)  # [slot][point]: one point per workgroup here
    t = u[:n]
    assert (t[0] > 0).all() and (np.diff(t, axis=0) >= 0).all()
    assert (u[n + 1] > u[n]).all()
