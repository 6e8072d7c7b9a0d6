"""Training epochs replayed from a HIP graph recording (with CPDE_REPLAY=1 the
protocol server records an epoch's gradient work once per active-buffer parity
from the second epoch of a call on, then launches the recording) against the
same epochs issued launch by launch (the default): every frame and the final
state byte for byte, on a scalar-graph objective (the Poisson disk), a graph with
value-dependent multipliers and attached variations, and a matching cost under
periodic reports, evaluations, outputs, snapshots and step restoration, with
RPROP and with Adam.  The server's own counts show that epochs were replayed."""
import json
import os

import numpy as np
import pytest

from cpde_amd import hip, wire, workloads
from cpde_amd import workloads as W
from cpde_amd.build import SERVER
from helpers import golden_workload, load_golden

pytestmark = pytest.mark.gpu


def canonical(events):
    """Events as comparable tuples (arrays as bytes)."""
    out = []
    for e in events:
        item = []
        for k in sorted(e):
            v = e[k]
            if isinstance(v, np.ndarray):
                v = (v.dtype.str, v.shape, v.tobytes())
            elif isinstance(v, (list, tuple)):
                v = tuple(x.tobytes() if isinstance(x, np.ndarray) else x for x in v)
            item.append((k, v))
        out.append(tuple(item))
    return out


def run(env, tmp_path, body):
    counts = tmp_path / f'replay_{len(list(tmp_path.iterdir()))}.json'
    s = wire.Session(SERVER, env=dict(os.environ, CPDE_REPLAY_FILE=str(counts), **env))
    try:
        result = body(s)
    finally:
        s.close()
    return result, json.loads(counts.read_text())


def poisson(s):
    pw = W.PoissonWorkload(radial=16, angular=16, boundary=64)
    ids = pw.upload(s)
    res = s.train(ids['net'], ids['costs'], 12, method=0, fresh=1, log=1, graph=pw.graph())
    return canonical(res['events']), res['completed'], s.snapshot(ids['net'])


def nested(s):
    vw = W.VariationWorkload()
    n, _, costs = vw.upload(s)
    res = s.train(n, [costs['a'], costs['correction']], 10, method=0, fresh=1, log=1, graph=vw.nested_graph())
    return canonical(res['events']), res['completed'], s.snapshot(n)


def matching(method):
    def body(s):
        g = load_golden('protocol')
        wl = golden_workload(g)
        ids = wl.upload(s, int(g['chunk']))
        extra = dict(restore_every=2, restore_step=1e-3) if method == 0 else dict(lr=0.01)
        res = s.train(ids['net'], [ids['cost']], 11, method=method, fresh=1, log=1, eval_every=3, outputs=1,
                      save=4, **extra)
        res2 = s.train(ids['net'], [ids['cost']], 9, method=method, fresh=0, log=2)
        return (canonical(res['events']), res['completed'], canonical(res2['events']), res2['completed'],
                s.snapshot(ids['net']))
    return body


@pytest.mark.parametrize('name,body', [('poisson', poisson), ('nested', nested), ('rprop', matching(0)),
                                       ('adam', matching(1))])
def test_replayed_epochs_match_launched(tmp_path, name, body):
    replayed, counts = run({'CPDE_REPLAY': '1'}, tmp_path, body)
    launched, none = run({}, tmp_path, body)
    print(f'[result] {name}: recorded {counts["recorded"]} replayed {counts["replayed"]}', flush=True)
    assert (none['recorded'], none['replayed']) == (0, 0)
    assert counts['replayed'] > 0
    assert replayed == launched


def states(net, transitions):
    return [net.state(t, b).tobytes() for t in range(transitions) for b in range(4)]


@pytest.mark.parametrize('static', [False, True])
def test_replayed_matching_epochs_through_the_abi(static):
    """Eight RPROP epochs of the order-2 Fourier fit through the C ABI: one
    issued launch by launch, two recorded (each runs as its capture ends), then
    five replays of the recording for the current active-buffer parity, each
    followed by a scalar download; the losses and all four buffers of every
    transition are bit-identical to eight epochs issued launch by launch.  With
    `static`, the recording holds the epoch that allocates nothing
    (cpde_epoch_matching_static) and the separate RPROP launch, which flips the
    active buffers inside the recording."""
    wl = workloads.fourier_fit(2)
    T = len(wl.neurons) - 1
    dev = hip.Device(0)
    try:
        ref = hip.MatchingRun(dev, wl, static_scratch=static)
        expected = []
        for _ in range(8):
            ref.step(collect=True, update=True)
            expected.append(ref.loss())
        expected_state = states(ref.net, T)
        run = hip.MatchingRun(dev, wl, static_scratch=static)
        got = []
        run.step(collect=True, update=True)
        got.append(run.loss())
        recordings = {}
        for _ in range(2):
            parity = run.net.active(0)
            dev.capture_begin()
            run.step(collect=True, update=True)
            recordings[parity] = dev.capture_end()
            got.append(run.loss())
        for _ in range(5):
            recordings[run.net.active(0)].launch()
            got.append(run.loss())
        print(f'[result] static {static}: losses {got[0]!r} .. {got[-1]!r}', flush=True)
        assert got == expected
        assert states(run.net, T) == expected_state
        for r in recordings.values():
            r.destroy()
        run.close()
        ref.close()
    finally:
        dev.close()


def test_replay_refusals():
    """What a capture cannot hold is refused without side effects: a
    synchronising call inside a capture, a replay whose network has the other
    active-buffer parity, a replay after device memory was released; a
    discarded capture leaves the active buffers where they were."""
    wl = workloads.fourier_fit(2)
    dev = hip.Device(0)
    try:
        run = hip.MatchingRun(dev, wl)
        run.step(collect=True, update=True)
        parity = run.net.active(0)
        dev.capture_begin()
        with pytest.raises(hip.CpdeError) as e:
            dev.synchronize()
        assert e.value.code == hip.EINVAL
        run.step(collect=True, update=True)
        rec = dev.capture_end()
        assert run.net.active(0) != parity
        with pytest.raises(hip.CpdeError) as e:
            rec.launch()
        assert e.value.code == hip.EINVAL
        run.step(collect=True, update=True)
        assert run.net.active(0) == parity
        rec.launch()
        assert run.net.active(0) != parity
        before = run.net.active(0)
        dev.capture_begin()
        run.step(collect=True, update=True)
        assert dev.capture_end(keep=False) is None
        assert run.net.active(0) == before
        run.step(collect=True, update=True)
        assert run.net.active(0) == parity
        hip.Buffer(dev, 256).free()
        with pytest.raises(hip.CpdeError) as e:
            rec.launch()
        assert e.value.code == hip.EINVAL
        assert np.isfinite(run.loss())
        rec.destroy()
        run.close()
    finally:
        dev.close()
