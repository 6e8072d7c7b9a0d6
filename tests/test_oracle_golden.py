"""Pins the oracle against golden vectors written by the reference CPU server
(tests/golden/make_golden.py) and against the reference's published losses.
CPU only; no GPU and no reference tree needed."""
import numpy as np
import pytest

import oracle
from cpde_amd import workloads as W
from helpers import check_gradient, golden_form, load_golden as load, oracle_epoch, rel_l2
from published_workload import PUBLISHED_LOSSES, reference_benchmark


def transitions(g):
    return len(g['neurons']) - 1


def epoch(g, chunk=None):
    T = transitions(g)
    init = [g[f'init{t}'] for t in range(T)]
    schema = g['schema']
    inputs = W.input_stack(g['points'], schema)
    c = int(g['chunk']) if chunk is None else chunk
    return oracle.matching_epoch(g['neurons'], g['linear'], init, schema, inputs.transpose(0, 2, 1),
                                 g['target'][:, :, None], g['row_weights'][:, None, None], chunk=c)


MATCHING = ['tiny_order6', 'tiny_3var_order4', 'fourier_order2', 'fourier3d_reduced', 'large_reduced']


@pytest.mark.parametrize('name', MATCHING)
def test_epoch_against_reference_server(name):
    g = load(name)
    loss, grads, outputs = epoch(g)
    assert abs(loss / g['loss'] - 1) < 1e-5
    for t, grad in enumerate(grads):
        check_gradient(g, t, grad, 1e-5)
    if 'outputs' in g:
        assert rel_l2(outputs, g['outputs']) < 1e-6


@pytest.mark.slow
def test_order6_epoch_against_reference_server():
    g = load('fourier_order6')
    loss, grads, outputs = epoch(g)
    assert abs(loss / g['loss'] - 1) < 1e-5
    for t, grad in enumerate(grads):
        check_gradient(g, t, grad, 1e-5)
    for r in range(outputs.shape[0]):
        assert rel_l2(outputs[r], g['outputs'][r]) < 1e-5, r


def test_chunked_epoch_matches_reference_chunks():
    g = load('tiny_order6')
    loss, grads, _ = epoch(g, chunk=7)
    assert abs(loss / g['chunk7_loss'] - 1) < 1e-5
    for t, grad in enumerate(grads):
        assert rel_l2(grad, g[f'chunk7_grad{t}']) < 1e-5


@pytest.mark.parametrize('name', ['tiny_order6', 'tiny_3var_order4'])
def test_first_rprop_step_matches_reference(name):
    """From a fresh optimizer state the reference's one-epoch update is
    w - copysign(0.002, g) wherever g != 0: the oracle, fed the reference's own
    gradient, must reproduce its weights and steps bit for bit."""
    g = load(name)
    for t in range(transitions(g)):
        w = g[f'init{t}']
        grad = g[f'grad{t}']
        W_, S, ga, gi = oracle.rprop(w, np.full_like(w, 0.002), grad, np.zeros_like(w))
        np.testing.assert_array_equal(W_, g[f'after{t}'])
        np.testing.assert_array_equal(S, g[f'step{t}'])
        assert int(g[f'active{t}']) == 2


def test_published_losses():
    """The reference's Fourier benchmark workload at initial weights, orders 0..6:
    the reference CPU server, and the oracle, against the published CUDA losses
    (docs/benchmarks/fourier-rtx3090.json)."""
    g = load('published')
    assert np.allclose(g['published_losses'], PUBLISHED_LOSSES, rtol=2e-8)
    for order in (0, 3):
        wl = reference_benchmark(order)
        loss, _, _ = oracle.matching_epoch(wl.neurons, wl.linear, wl.init, wl.schema, wl.inputs.transpose(0, 2, 1),
                                           wl.target[:, :, None], wl.row_weights[:, None, None], outputs=False)
        assert abs(loss / PUBLISHED_LOSSES[order] - 1) < 1e-6, order


@pytest.mark.parametrize('record,prefix', [('matching_forms', 'persample'), ('matching_forms', 'subset'),
                                           ('matching_forms', 'subset_persample'), ('linear_hidden', 'inner'),
                                           ('linear_hidden', 'first')])
def test_cost_forms_against_reference_server(record, prefix):
    """Per-sample matching weights, a non-prefix row subset with remapped
    target rows, and linear hidden layers: the oracle's epoch against the
    reference server's op-14 value and gradient (and op-4 outputs)."""
    g = load(record)
    wl = golden_form(g, prefix)
    loss, grads, _ = oracle_epoch(wl)
    assert abs(loss / g[f'{prefix}_loss'] - 1) < 1e-5
    for t, grad in enumerate(grads):
        assert rel_l2(grad, g[f'{prefix}_grad{t}']) < 1e-5, t
    if f'{prefix}_outputs' in g:
        out = oracle.forward(wl.neurons, wl.linear, wl.init, wl.schema, wl.inputs.transpose(0, 2, 1))
        assert rel_l2(out, g[f'{prefix}_outputs']) < 1e-5
