"""Client for the cPDE stdin/stdout frame protocol.

Frames are ``uint64 LE length`` (counting the 4-byte kind) + ``uint32 kind`` +
payload; arrays are ``uint64 count`` + raw little-endian elements and strings
are ``uint64 length`` + bytes (cuda/protocol.hpp:10-51).  Request layouts follow
the server's parsers in cuda/cpde_server.cu:436-555 and the training request in
cuda/cpde_server.cu:364-371.  Replies are kind 0 (result) or kind 1 (string
error); training also streams event frames of kinds 2-6.

This module drives any executable that speaks the protocol: the MI355X server
built from this package, or the reference CPU server used as the oracle.
"""
from __future__ import annotations

import collections
import os
import queue
import struct
import subprocess
import threading

import numpy as np

# Capability bits advertised by op 1 (cuda/cpde_server.cu:438-447).
CAP_DIAGNOSTICS, CAP_GRAPHS, CAP_EXPRESSIONS, CAP_RESTORE, CAP_INIT = 1, 2, 4, 8, 16
CAP_CPU, CAP_PROBE = 32, 64

# Scalar expression IR opcodes (cuda/scalar_ops.cuh:5).
CONSTANT, COMPONENT, FIELD, ADD, SUB, MUL, DIV, POWER, NEG, EXP, LOG, SQRT, SIN, COS, TANH = range(15)
LEAF, ATTACH = 1, 15


class ServerError(RuntimeError):
    """A kind-1 reply: a validation or numerical error; the server stays usable.
    ``events`` holds the training event frames that came before it."""

    def __init__(self, message, events=()):
        super().__init__(message)
        self.events = list(events)


class Writer:
    def __init__(self):
        self.parts = []

    def put(self, fmt, value):
        self.parts.append(struct.pack('<' + fmt, value))
        return self

    def array(self, value, dtype):
        a = np.ascontiguousarray(value, dtype=np.dtype(dtype).newbyteorder('<'))
        self.put('Q', a.size)
        self.parts.append(a.tobytes())
        return self

    def string(self, value):
        b = value.encode('utf-8') if isinstance(value, str) else bytes(value)
        self.put('Q', len(b))
        self.parts.append(b)
        return self

    def raw(self, b):
        self.parts.append(bytes(b))
        return self

    def bytes(self):
        return b''.join(self.parts)


class Reader:
    def __init__(self, data):
        self.data, self.pos = data, 0

    def take(self, n):
        if self.pos + n > len(self.data):
            raise RuntimeError('truncated response')
        v = self.data[self.pos:self.pos + n]
        self.pos += n
        return v

    def get(self, fmt):
        return struct.unpack('<' + fmt, self.take(struct.calcsize('<' + fmt)))[0]

    def array(self, dtype):
        dt = np.dtype(dtype).newbyteorder('<')
        n = self.get('Q')
        return np.frombuffer(self.take(n * dt.itemsize), dtype=dt).copy()

    def string(self):
        return self.take(self.get('Q')).decode('utf-8', 'replace')

    def end(self):
        if self.pos != len(self.data):
            raise RuntimeError('unexpected response fields')


def decode_metadata(r):
    """State blob header (cuda/cpde_server.cu:193-198)."""
    if r.get('I') != 1:
        raise ValueError('unsupported state version')
    neurons, linear = r.array('i4').tolist(), r.array('i4').tolist()
    return dict(neurons=neurons, linear=linear, optimizer=r.get('i'), updates=r.get('Q'),
                adam_step=r.get('Q'), stage_done=r.get('Q'), remaining=r.get('Q'),
                learning_rate=r.get('f'), initial_step=r.get('f'), stage=r.string())


def decode_state(blob):
    """Full snapshot blob: metadata, then per layer ``i32 act_grad`` and four f32
    buffers W, G1, G2, step (cuda/cpde_server.cu:199-206)."""
    r = Reader(blob)
    meta = decode_metadata(r)
    layers = []
    for _ in range(len(meta['neurons']) - 1):
        active = r.get('i')
        layers.append(dict(active=active, buffers=[r.array('f4') for _ in range(4)]))
    r.end()
    return meta, layers


def encode_state(meta, layers):
    w = Writer().put('I', 1).array(meta['neurons'], 'i4').array(meta['linear'], 'i4')
    w.put('i', meta['optimizer'])
    for key in ('updates', 'adam_step', 'stage_done', 'remaining'):
        w.put('Q', meta[key])
    w.put('f', meta['learning_rate']).put('f', meta['initial_step']).string(meta['stage'])
    for layer in layers:
        w.put('i', layer['active'])
        for b in layer['buffers']:
            w.array(b, 'f4')
    return w.bytes()


def graph_bytes(nodes, constants, root):
    """Cost-graph trailer: i32[] (op,a,b) per node, f64[] constants, i32 root."""
    return Writer().array(np.asarray(nodes, np.int32).ravel(), 'i4').array(constants, 'f8').put('i', root).bytes()


class Session:
    """Owns one server process; requests are serialised, frames read on a thread."""

    def __init__(self, executable, device=0, env=None):
        self._lock = threading.RLock()
        self.stderr_lines = collections.deque(maxlen=200)
        self.proc = subprocess.Popen([str(executable), '--device', str(device)], stdin=subprocess.PIPE,
                                     stdout=subprocess.PIPE, stderr=subprocess.PIPE, bufsize=0,
                                     env=env if env is not None else os.environ.copy())
        self._responses = queue.Queue()
        threading.Thread(target=self._drain_err, daemon=True).start()
        threading.Thread(target=self._drain_out, daemon=True).start()
        self.closed = False
        r = self.request(1)
        self.protocol, self.version, self.capabilities = r.string(), r.get('i'), r.get('I')
        r.end()

    # ----------------------------------------------------------------- transport
    def _drain_err(self):
        for line in iter(self.proc.stderr.readline, b''):
            self.stderr_lines.append(line.decode('utf-8', 'replace').rstrip())

    def _read_exact(self, n):
        chunks = []
        while n:
            part = self.proc.stdout.read(n)
            if not part:
                raise RuntimeError('server stopped: ' + '\n'.join(self.stderr_lines))
            chunks.append(part)
            n -= len(part)
        return b''.join(chunks)

    def _drain_out(self):
        try:
            while True:
                size = struct.unpack('<Q', self._read_exact(8))[0]
                if not 4 <= size <= 4 * 1024 ** 3:
                    raise RuntimeError('invalid response frame')
                payload = self._read_exact(size)
                self._responses.put((struct.unpack_from('<I', payload)[0], Reader(payload[4:])))
        except BaseException as e:  # noqa: BLE001 - surfaced to the waiting request
            self._responses.put(e)

    def send(self, op, body=b''):
        frame = struct.pack('<QI', len(body) + 4, op) + body
        view = memoryview(frame)
        while view:
            n = self.proc.stdin.write(view)
            if not n:
                raise RuntimeError('server input closed')
            view = view[n:]
        self.proc.stdin.flush()

    def send_raw(self, data):
        self.proc.stdin.write(data)
        self.proc.stdin.flush()

    def receive(self, timeout=None):
        v = self._responses.get(timeout=timeout)
        if isinstance(v, BaseException):
            raise v
        return v

    def request(self, op, body=b''):
        with self._lock:
            self.send(op, body)
            kind, r = self.receive()
            if kind == 1:
                raise ServerError(r.string())
            if kind != 0:
                raise RuntimeError(f'unexpected response kind {kind}')
            return r

    def close(self):
        if self.closed:
            return
        self.closed = True
        try:
            self.request(0)
        except Exception:  # noqa: BLE001 - the process may already be gone
            pass
        try:
            self.proc.stdin.close()
        except OSError:
            pass
        try:
            self.proc.wait(timeout=30)
        except subprocess.TimeoutExpired:
            self.proc.kill()
            self.proc.wait()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ------------------------------------------------------------------ objects
    def data(self, samples, table):
        """op 2. ``samples`` has shape (rows, channels, points); ``table`` rows are
        (order, count_1..count_v).  Uploaded as [row][sample][channel]."""
        a = np.asarray(samples, np.float32)
        t = np.asarray(table, np.int32)
        d, h, w = a.shape
        body = Writer().put('i', d).put('i', h).put('i', w).put('i', t.shape[1] - 1)
        body.array(t, 'i4').array(a.transpose(0, 2, 1), 'f4')
        r = self.request(2, body.bytes())
        i = r.get('Q')
        r.end()
        return i

    def network(self, neurons, linear, weights):
        """op 3. ``weights[l]`` is n_out x (n_in+1) column-major with the bias last."""
        body = Writer().array(neurons, 'i4').array(linear, 'i4')
        for w in weights:
            body.array(np.asarray(w, np.float32).ravel(), 'f4')
        r = self.request(3, body.bytes())
        i = r.get('Q')
        r.end()
        return i

    def eval(self, net, data, chunk=0):
        r = self.request(4, Writer().put('Q', net).put('Q', data).put('i', chunk).bytes())
        i = r.get('Q')
        r.end()
        return i

    def download(self, data):
        """op 5: the whole storage, [row][sample][channel] flattened."""
        r = self.request(5, Writer().put('Q', data).bytes())
        a = r.array('f4')
        r.end()
        return a

    def download_shaped(self, data, rows, channels, samples):
        return self.download(data).reshape(rows, samples, channels).transpose(0, 2, 1)

    def replace(self, data, samples):
        a = np.asarray(samples, np.float32)
        self.request(6, Writer().put('Q', data).array(a.transpose(0, 2, 1), 'f4').bytes()).end()

    def matching_cost(self, net, inputs, targets, rows, target_rows, weights, weight_samples=1, chunk=0):
        """op 7 kind 0.  ``weights`` is (rows, weight_samples, outputs)."""
        body = Writer().put('Q', net).put('Q', inputs).put('Q', targets).put('i', 0).put('i', chunk)
        body.array(rows, 'i4').array(target_rows, 'i4').put('i', weight_samples)
        body.array(np.asarray(weights, np.float32).ravel(), 'f4')
        r = self.request(7, body.bytes())
        i = r.get('Q')
        r.end()
        return i

    def polynomial_cost(self, net, inputs, rows, equations, terms, coeffs, rhs, weights, chunk=0):
        """op 7 kind 1: sparse linear/quadratic residuals."""
        body = Writer().put('Q', net).put('Q', inputs).put('Q', 0).put('i', 1).put('i', chunk)
        body.array(rows, 'i4').put('i', equations).array(np.asarray(terms, np.int32).ravel(), 'i4')
        body.array(coeffs, 'f4').array(rhs, 'f4').array(weights, 'f4')
        r = self.request(7, body.bytes())
        i = r.get('Q')
        r.end()
        return i

    def integral_cost(self, net, inputs, nodes, constants, fields, quadrature_weights, chunk=0):
        """op 12: expression IR (op,a,b) with double constants; ``fields`` is
        (F, samples) double; returns the cost id."""
        f = np.asarray(fields, np.float64)
        qw = np.asarray(quadrature_weights, np.float64)
        samples = qw.size
        body = Writer().put('Q', net).put('Q', inputs).put('i', chunk).put('i', samples)
        body.array(np.asarray(nodes, np.int32).ravel(), 'i4').array(constants, 'f8')
        body.put('i', f.shape[0] if f.size else 0).array(f.ravel(), 'f8').array(qw, 'f8')
        r = self.request(12, body.bytes())
        i = r.get('Q')
        r.end()
        return i

    def inspect(self, cost, compile=False):
        r = self.request(13, Writer().put('Q', cost).put('i', int(compile)).bytes())
        src, log = r.string(), r.string()
        r.end()
        return src, log

    def graph_eval(self, net, costs, graph, gradient=False, layers=0):
        body = Writer().put('Q', net).array(costs, 'u8').put('i', int(gradient)).raw(graph)
        r = self.request(14, body.bytes())
        value = r.get('d')
        grads = None
        if gradient:
            grads = [r.array('f4') for _ in range(r.get('i'))]
        r.end()
        return value, grads

    def snapshot(self, net):
        return self.request(9, Writer().put('Q', net).bytes()).data

    def restore(self, net, blob):
        self.request(10, Writer().put('Q', net).raw(blob).bytes()).end()

    def close_object(self, kind, ident):
        self.request(11, Writer().put('i', kind).put('Q', ident).bytes()).end()

    def timing(self, net, cost, warm=20, iterations=100, batches=7, layers=0):
        """op 90 (benchmark command): returns wall ms, device ms, loss, gradients."""
        body = Writer().put('Q', net).put('Q', cost).put('i', warm).put('i', iterations).put('i', batches)
        r = self.request(90, body.bytes())
        wall, gpu, loss = r.array('f8'), r.array('f8'), r.get('d')
        grads = [r.array('f4') for _ in range(layers)]
        r.end()
        return dict(wall_ms=wall, gpu_ms=gpu, loss=loss, gradients=grads)

    def train(self, net, costs, epochs, method=0, fresh=0, steps=0.0, moments=0, lr=0.0, verbose=0,
              log=1, eval_every=0, outputs=0, save=0, stage='', diagnostics=0, graph=None,
              restore_every=0, restore_step=0.0, on_event=None):
        """op 8 (or op 15 with a graph).  Returns the event list and final result.
        ``on_event(session, event)`` is called for every event frame as it
        arrives (e.g. to send op 99 from there)."""
        w = Writer().put('Q', net).array(costs, 'u8').put('Q', epochs).put('i', method).put('i', fresh)
        w.put('f', steps).put('i', moments).put('f', lr)
        for v in (verbose, log, eval_every, outputs, save):
            w.put('i', v)
        w.string(stage).put('i', diagnostics)
        if graph is not None:
            w.raw(graph)
        if restore_every:
            w.put('Q', restore_every).put('f', restore_step)
        events = []
        with self._lock:
            self.send(15 if graph is not None else 8, w.bytes())
            while True:
                kind, r = self.receive()
                if kind == 1:
                    raise ServerError(r.string(), events)
                if kind in (2, 6):
                    ev = dict(kind=kind, completed=r.get('Q'), updates=r.get('Q'), after=r.get('i'),
                              values=r.array('f8'))
                    if kind == 6:
                        ev['total'] = r.get('d')
                    r.end()
                elif kind == 3:
                    ev = dict(kind=3, blob=r.data)
                elif kind == 4:
                    ev = dict(kind=4, cost=r.get('Q'), outputs=r.array('f4'))
                    r.end()
                elif kind == 5:
                    ev = dict(kind=5, epoch=r.get('Q'), updates=r.get('Q'))
                    n = r.get('i')
                    ev['layers'] = [dict(sq=r.get('d'), max=r.get('d'), nonfinite=r.get('Q'), first=r.get('i'))
                                    for _ in range(n)]
                    r.end()
                elif kind == 0:
                    completed, stopped = r.get('Q'), r.get('i')
                    meta = decode_metadata(Reader(r.take(r.get('Q'))))
                    r.end()
                    return dict(completed=completed, stopped=stopped, metadata=meta, events=events)
                else:
                    raise RuntimeError(f'unexpected training event {kind}')
                events.append(ev)
                if on_event is not None:
                    on_event(self, ev)

    def stop(self):
        self.send(99)
