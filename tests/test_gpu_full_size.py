"""Full-size checks of the two largest workloads:

  * against the reference CPU server at full size (tests/golden/
    make_full_size.py): the epoch's loss (relative 1e-4), every weight
    gradient (relative L2 1e-3, on probe projections and the norm for the
    large blocks) and the derivative outputs at 64 sampled points (relative L2
    per row 1e-3);

and through properties that need no full-size CPU reference:

  * 2->256x4->1 sigmoid, order 6 (28 rows), 262,144 points in 65,536-point
    chunks, and 3->128x5->1 sigmoid, order 4 (35 rows), 32,768 points;
  * every derivative output row at a fixed sample of 64 points equals the
    oracle's forward of those points (a point's derivative stack depends on
    that point alone): relative L2 per row <= 1e-3, the order-6 bar;
  * the chunked epoch's loss and weight gradient equal the sums of the
    per-chunk epochs run as separate workloads (chunk accumulation changes only
    the fp32 summation order): loss relative 1e-6, gradient relative L2 1e-5.
"""
import numpy as np
import pytest

import oracle
from cpde_amd import hip, workloads as W
from helpers import check_gradient, load_golden, rel_l2

pytestmark = pytest.mark.gpu

FULL = {'3d_order4': ('fourier3d_full', W.fourier_3d), 'large_order6': ('large_full', W.fourier_large)}


@pytest.mark.parametrize('name', list(FULL))
def test_full_size_epoch_against_reference_server(device, name):
    record, make = FULL[name]
    g = load_golden(record)
    wl = make()
    print(f'[case] {wl.name} neurons={wl.neurons} R={wl.rows} P={wl.size} chunk={wl.chunk}', flush=True)
    run = hip.MatchingRun(device, wl)
    run.step()
    device.synchronize()
    loss = run.loss()
    rel = abs(loss / g['loss'] - 1)
    print(f'[result] loss {loss!r} reference {float(g["loss"])!r} rel {rel:.2e}', flush=True)
    assert rel < 1e-4
    for t, grad in enumerate(run.gradients()):
        err = check_gradient(g, t, grad, 1e-3)
        print(f'[result] transition {t} gradient rel-L2 {err:.2e}', flush=True)
    run.close()
    got = sampled_outputs(device, wl, g['sampled'])
    worst = max(rel_l2(got[r], g['outputs'][r]) for r in range(wl.rows))
    print(f'[result] worst sampled output row rel-L2 {worst:.2e}', flush=True)
    assert worst < 1e-3


def sampled_outputs(device, wl, idx):
    """Forward every chunk of the workload; return the output stack at points idx."""
    run = hip.MatchingRun(device, wl)
    R, n_out = wl.rows, wl.neurons[-1]
    dest = hip.Buffer(device, R * wl.size * n_out * 4)
    rows = np.arange(R, dtype=np.int32)
    for offset in range(0, wl.size, run.width):
        valid = min(run.width, wl.size - offset)
        run.plan.activate(run.data, wl.size, rows, offset, valid)
        run.plan.forward()
        run.plan.output(dest, wl.size, rows, offset, valid)
    out = dest.download(np.float32, R * wl.size * n_out).reshape(R, wl.size, n_out)
    dest.free()
    run.close()
    return out[:, idx, :]


@pytest.mark.parametrize('make', [W.fourier_large, W.fourier_3d], ids=['large_order6', '3d_order4'])
def test_outputs_at_sampled_points_match_the_oracle(device, make):
    wl = make()
    idx = np.linspace(0, wl.size - 1, 64).astype(int)
    print(f'[case] {wl.name} neurons={wl.neurons} R={wl.rows} P={wl.size} chunk={wl.chunk}', flush=True)
    got = sampled_outputs(device, wl, idx)
    x = np.ascontiguousarray(wl.inputs.transpose(0, 2, 1)[:, idx, :])
    want = oracle.forward(wl.neurons, wl.linear, wl.init, wl.schema, x)
    worst = max(rel_l2(got[r], want[r]) for r in range(wl.rows))
    print(f'[result] worst output row rel-L2 {worst:.2e}', flush=True)
    assert worst < 1e-3


def chunk_workload(wl, begin, end):
    return W.MatchingWorkload(f'{wl.name}[{begin}:{end}]', wl.neurons, wl.points[begin:end], wl.schema,
                              wl.target[:, begin:end], wl.row_weights, wl.init)


def epoch(device, wl):
    run = hip.MatchingRun(device, wl)
    run.step()
    device.synchronize()
    loss, grads = run.loss(), [g.astype(np.float64) for g in run.gradients()]
    run.close()
    return loss, grads


def test_chunked_epoch_is_the_sum_of_its_chunks(device):
    wl = W.fourier_large()
    assert wl.chunk == 65536 and wl.size == 4 * wl.chunk
    print(f'[case] {wl.name} P={wl.size} chunk={wl.chunk}', flush=True)
    loss, grads = epoch(device, wl)
    parts = [epoch(device, chunk_workload(wl, c, c + wl.chunk)) for c in range(0, wl.size, wl.chunk)]
    loss_sum = sum(p[0] for p in parts)
    print(f'[result] loss {loss!r} sum of chunks {loss_sum!r}', flush=True)
    assert abs(loss / loss_sum - 1) < 1e-6
    for t, g in enumerate(grads):
        err = rel_l2(g, sum(p[1][t] for p in parts))
        print(f'[result] transition {t} gradient rel-L2 {err:.2e}', flush=True)
        assert err < 1e-5
