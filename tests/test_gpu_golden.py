"""Parity of the HIP epoch with the reference CPU server's golden vectors,
through the C ABI, on the layer-fused (schema-specialised) kernels and on the
table-driven kernels.

Bars (the parity tolerances, order 6): loss relative error <= 1e-4; every
derivative output row and every weight gradient relative L2 <= 1e-3.  RPROP:
after one update from a fresh optimizer state, every weight whose reference
gradient exceeds 1e-3 of the largest must be bit-identical to the reference's.
"""
import numpy as np
import pytest

from cpde_amd import hip
from helpers import check_gradient, golden_workload, load_golden, rel_l2

pytestmark = pytest.mark.gpu

CASES = ['tiny_order6', 'tiny_3var_order4', 'fourier_order2', 'fourier_order6', 'fourier3d_reduced',
         'large_reduced']


def outputs_of(device, run, wl):
    """Forward every chunk and gather the output stack in wire layout."""
    R, n_out = wl.rows, wl.neurons[-1]
    dest = hip.Buffer(device, R * wl.size * n_out * 4)
    rows = np.arange(R, dtype=np.int32)
    for offset in range(0, wl.size, run.width):
        valid = min(run.width, wl.size - offset)
        run.plan.activate(run.data, wl.size, rows, offset, valid)
        run.plan.forward()
        run.plan.output(dest, wl.size, rows, offset, valid)
    run._loaded = None
    out = dest.download(np.float32, R * wl.size * n_out).reshape(R, wl.size, n_out)
    dest.free()
    return out


@pytest.mark.parametrize('name', CASES)
def test_epoch_against_reference_server(device, path, name):
    g = load_golden(name)
    wl = golden_workload(g)
    print(f'[case] {name} path={path} neurons={wl.neurons} R={wl.rows} P={wl.size} chunk={wl.chunk}', flush=True)
    run = hip.MatchingRun(device, wl)
    assert (run.plan.handle is not None)
    run.step()
    device.synchronize()
    loss = run.loss()
    rel = abs(loss / g['loss'] - 1)
    print(f'[result] loss {loss!r} reference {float(g["loss"])!r} rel {rel:.2e}', flush=True)
    assert rel < 1e-4
    for t, grad in enumerate(run.gradients()):
        err = check_gradient(g, t, grad, 1e-3)
        print(f'[result] transition {t} gradient rel-L2 {err:.2e}', flush=True)
    out = outputs_of(device, run, wl)
    worst = max(rel_l2(out[r], g['outputs'][r]) for r in range(wl.rows))
    print(f'[result] worst output row rel-L2 {worst:.2e}', flush=True)
    assert worst < 1e-3
    run.close()


@pytest.mark.parametrize('col_tile', [16, 'single16', 32, 'paired'])
@pytest.mark.parametrize('name', ['fourier_order6', 'fourier3d_reduced', 'large_reduced'])
def test_network_products_column_tiles(device, monkeypatch, name, col_tile):
    """The network-fused products on 16-column (v_mfma_f32_16x16x4f32) and
    32-column (v_mfma_f32_32x32x2f32) tiles, each forced on shapes where the
    other is the default (28 rows: 32 columns either way; 35 rows: 48 or 64),
    and the long-grid form ('paired': two points per workgroup on 16-column
    tiles, the product tile written over its operand tile) forced on these
    short grids, against the reference server's epoch at the order-6 bars.
    16-column products take 32-neuron blocks per wave (float2 weight pairs)
    where a width allows; 'single16' forces one 16-neuron block at a time."""
    monkeypatch.setenv('CPDE_FUSED', '2')
    if col_tile == 'single16':
        monkeypatch.setenv('CPDE_NET_COLTILE', '16')
        monkeypatch.setenv('CPDE_NET_BPAIR', '0')
        monkeypatch.setenv('CPDE_NET_ALIAS', '0')
    elif col_tile == 'paired':
        for k, v in (('CPDE_NET_COLTILE', '16'), ('CPDE_NET_POINTS', '2'), ('CPDE_NET_ALIAS', '1')):
            monkeypatch.setenv(k, v)
    else:
        monkeypatch.setenv('CPDE_NET_COLTILE', str(col_tile))
        monkeypatch.setenv('CPDE_NET_ALIAS', '0')
    g = load_golden(name)
    wl = golden_workload(g)
    print(f'[case] {name} col_tile={col_tile} R={wl.rows} P={wl.size}', flush=True)
    run = hip.MatchingRun(device, wl)
    run.step()
    device.synchronize()
    assert abs(run.loss() / g['loss'] - 1) < 1e-4
    for t, grad in enumerate(run.gradients()):
        assert check_gradient(g, t, grad, 1e-3) < 1e-3
    out = outputs_of(device, run, wl)
    assert max(rel_l2(out[r], g['outputs'][r]) for r in range(wl.rows)) < 1e-3
    run.close()


@pytest.mark.parametrize('name', ['tiny_order6', 'tiny_3var_order4'])
def test_first_rprop_step_against_reference_server(device, path, name):
    g = load_golden(name)
    wl = golden_workload(g)
    run = hip.MatchingRun(device, wl)
    run.step()
    run.net.rprop()
    device.synchronize()
    for t in range(len(wl.neurons) - 1):
        ref_g = g[f'grad{t}']
        sure = np.abs(ref_g) > 1e-3 * np.abs(ref_g).max()
        after = run.net.state(t, 0)
        np.testing.assert_array_equal(after[sure], g[f'after{t}'][sure])
        np.testing.assert_array_equal(run.net.state(t, 3)[sure], g[f'step{t}'][sure])
        assert run.net.active(t) == int(g[f'active{t}'])
    run.close()


def test_chunked_epoch_against_reference_server(device, path):
    g = load_golden('tiny_order6')
    wl = golden_workload(g)
    run = hip.MatchingRun(device, wl, chunk=7)
    run.step()
    device.synchronize()
    assert abs(run.loss() / g['chunk7_loss'] - 1) < 1e-4
    for t, grad in enumerate(run.gradients()):
        assert rel_l2(grad, g[f'chunk7_grad{t}']) < 1e-3
    run.close()


@pytest.mark.parametrize('name', ['fourier_order6', 'large_reduced'])
def test_one_pass_epoch_matches_separate_launches(device, path, name):
    """forward + matching + backward in one launch (cpde_epoch_matching) against
    the three separate entry points: the same output adjoint and backward, so
    bit-identical gradients; the loss differs only in its fp64 summation order."""
    g = load_golden(name)
    wl = golden_workload(g)
    results = []
    for one_pass in (True, False):
        run = hip.MatchingRun(device, wl, one_pass=one_pass)
        run.step()
        device.synchronize()
        results.append((run.loss(), run.gradients()))
        run.close()
    (l1, g1), (l2, g2) = results
    print(f'[result] one-pass loss {l1!r} separate {l2!r}', flush=True)
    assert abs(l1 / l2 - 1) < 1e-12
    for a, b in zip(g1, g2):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize('optimizer', ['rprop', 'adam'])
def test_one_pass_epochs_across_updates(device, optimizer):
    """Four epochs with an optimizer update after each: the one-pass epoch reads
    the row-major weight copy that RPROP and Adam keep current, and must track
    the separate launches (which transpose in the forward) bit for bit.  Then
    weights written through the state pointer must be seen by the next epoch."""
    g = load_golden('fourier_order6')
    wl = golden_workload(g)
    runs = [hip.MatchingRun(device, wl, one_pass=one_pass) for one_pass in (True, False)]
    for epoch in range(4):
        for run in runs:
            run.step()
            if optimizer == 'rprop':
                run.net.rprop()
            else:
                run.net.adam(epoch + 1, 0.01)
        device.synchronize()
        for t in range(len(wl.neurons) - 1):
            np.testing.assert_array_equal(runs[0].net.state(t, 0), runs[1].net.state(t, 0))
    print(f'[case] {optimizer}: 4 epochs, weights identical', flush=True)
    fresh = wl.init
    for run in runs:
        for t, w in enumerate(fresh):
            run.net.set_state(t, 0, w)
        run.step()
    device.synchronize()
    ref = hip.MatchingRun(device, wl, one_pass=True)
    ref.step()
    device.synchronize()
    for run in runs:
        assert abs(run.loss() / ref.loss() - 1) < 1e-12
        for a, b in zip(run.gradients(), ref.gradients()):
            np.testing.assert_array_equal(a, b)
    for run in runs + [ref]:
        run.close()
