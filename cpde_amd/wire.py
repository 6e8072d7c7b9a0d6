"""Client for the cPDE stdin/stdout frame protocol.

Transport (cuda/protocol.hpp:36-51): a frame is a little-endian u64 byte count
(the 4-byte kind included), a u32 kind and the payload.  Inside a payload,
scalars are little-endian fixed-width values, a vector is a u64 element count
followed by the raw elements, and a string is a u64 byte count followed by the
bytes (cuda/protocol.hpp:10-34).  Request layouts follow the server's parsers
(cuda/cpde_server.cu:436-555, the training request :364-371).  Replies are
kind 0 (result) or kind 1 (error string); training also streams event frames
of kinds 2-6.

Payloads are described, not hand-assembled: ``encode`` turns a sequence of
``(tag, value)`` fields into bytes and ``Cursor`` reads tagged fields back, both
from one table of field tags.  The snapshot blob is read and written from the
field table ``STATE_HEADER``.

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

# ----------------------------------------------------------------------------- field tags
# fixed-width scalars, by tag
_FIXED = {tag: struct.Struct('<' + code) for tag, code in
          (('i32', 'i'), ('u32', 'I'), ('u64', 'Q'), ('f32', 'f'), ('f64', 'd'))}
# counted vectors, by tag: element dtype (little-endian)
_COUNTED = {'i32[]': np.dtype('<i4'), 'u64[]': np.dtype('<u8'), 'f32[]': np.dtype('<f4'), 'f64[]': np.dtype('<f8')}
_COUNT = _FIXED['u64']
FRAME_HEAD = struct.Struct('<QI')  # byte count (kind included), kind
MAX_FRAME = 4 * 1024 ** 3


def _counted(values, dtype):
    a = np.asarray(values, dtype=dtype).ravel()
    return _COUNT.pack(a.size) + a.tobytes()


def _field_bytes(tag, value):
    fixed = _FIXED.get(tag)
    if fixed is not None:
        return fixed.pack(value)
    dtype = _COUNTED.get(tag)
    if dtype is not None:
        return _counted(value, dtype)
    if tag == 'str':
        b = value.encode('utf-8') if isinstance(value, str) else bytes(value)
        return _COUNT.pack(len(b)) + b
    if tag == 'raw':
        return bytes(value)
    raise ValueError(f'unknown field tag {tag!r}')


def encode(*fields):
    """Payload bytes of ``(tag, value)`` fields, in order.  Tags: i32, u32, u64,
    f32, f64 (scalars); i32[], u64[], f32[], f64[] (counted vectors); str
    (counted UTF-8); raw (bytes as they are)."""
    return b''.join(_field_bytes(tag, value) for tag, value in fields)


class Cursor:
    """Reads tagged fields from a payload front to back; ``finish`` checks that
    nothing is left over."""

    __slots__ = ('_view', '_at')

    def __init__(self, payload):
        self._view = memoryview(payload)
        self._at = 0

    def _span(self, n):
        start, stop = self._at, self._at + n
        if stop > len(self._view):
            raise RuntimeError(f'response ends after {len(self._view)} bytes, {stop} needed')
        self._at = stop
        return start

    def read(self, tag):
        fixed = _FIXED.get(tag)
        if fixed is not None:
            return fixed.unpack_from(self._view, self._span(fixed.size))[0]
        dtype = _COUNTED.get(tag)
        if dtype is not None:
            n = self.read('u64')
            start = self._span(n * dtype.itemsize)
            return np.frombuffer(self._view, dtype=dtype, count=n, offset=start).astype(dtype.newbyteorder('='))
        if tag == 'str':
            n = self.read('u64')
            start = self._span(n)
            return bytes(self._view[start:start + n]).decode('utf-8', 'replace')
        raise ValueError(f'unknown field tag {tag!r}')

    def read_all(self, *tags):
        return tuple(self.read(tag) for tag in tags)

    def blob(self, n):
        start = self._span(n)
        return bytes(self._view[start:start + n])

    def rest(self):
        return self.blob(len(self._view) - self._at)

    def finish(self):
        if self._at != len(self._view):
            raise RuntimeError(f'{len(self._view) - self._at} unread bytes at the end of a response')


# ----------------------------------------------------------------------------- snapshot blob
# The state blob header (cuda/cpde_server.cu:193-198), field by field; the
# version must be 1.  After it, per transition: i32 active gradient buffer,
# then four f32 vectors W, G1, G2, step/m (:199-206).
STATE_HEADER = (('version', 'u32'), ('neurons', 'i32[]'), ('linear', 'i32[]'), ('optimizer', 'i32'),
                ('updates', 'u64'), ('adam_step', 'u64'), ('stage_done', 'u64'), ('remaining', 'u64'),
                ('learning_rate', 'f32'), ('initial_step', 'f32'), ('stage', 'str'))
STATE_BUFFERS = 4


def read_metadata(cursor):
    meta = {name: cursor.read(tag) for name, tag in STATE_HEADER}
    if meta.pop('version') != 1:
        raise ValueError('unsupported state version')
    meta['neurons'], meta['linear'] = meta['neurons'].tolist(), meta['linear'].tolist()
    return meta


def decode_state(blob):
    """A snapshot blob: (metadata dict, per transition {'active', 'buffers'})."""
    c = Cursor(blob)
    meta = read_metadata(c)
    layers = [dict(active=c.read('i32'), buffers=[c.read('f32[]') for _ in range(STATE_BUFFERS)])
              for _ in range(len(meta['neurons']) - 1)]
    c.finish()
    return meta, layers


def encode_state(meta, layers):
    values = dict(meta, version=1)
    fields = [(tag, values[name]) for name, tag in STATE_HEADER]
    for layer in layers:
        fields.append(('i32', layer['active']))
        fields.extend(('f32[]', b) for b in layer['buffers'])
    return encode(*fields)


def graph_bytes(nodes, constants, root):
    """Cost-graph trailer: i32[] (op, a, b) per node, f64[] constants, i32 root."""
    return encode(('i32[]', np.asarray(nodes, np.int32)), ('f64[]', constants), ('i32', root))


# ----------------------------------------------------------------------------- events
# Training event frames (cuda/cpde_server.cu:364-435): kind -> field table.
_REPORT = (('completed', 'u64'), ('updates', 'u64'), ('after', 'i32'), ('values', 'f64[]'))
_EVENTS = {2: _REPORT, 6: _REPORT + (('total', 'f64'),), 4: (('cost', 'u64'), ('outputs', 'f32[]'))}
_LAYER_DIAGNOSTICS = (('sq', 'f64'), ('max', 'f64'), ('nonfinite', 'u64'), ('first', 'i32'))


def _event(kind, c):
    if kind in _EVENTS:
        ev = {name: c.read(tag) for name, tag in _EVENTS[kind]}
    elif kind == 3:
        return dict(kind=3, blob=c.rest())
    elif kind == 5:
        ev = dict(epoch=c.read('u64'), updates=c.read('u64'))
        ev['layers'] = [{name: c.read(tag) for name, tag in _LAYER_DIAGNOSTICS} for _ in range(c.read('i32'))]
    else:
        raise RuntimeError(f'unexpected training event {kind}')
    c.finish()
    ev['kind'] = kind
    return ev


class ServerError(RuntimeError):
    """A kind-1 reply: a validation or numerical error; the server stays usable.
    ``events`` holds the training event frames that came before it."""

    def __init__(self, message, events=()):
        super().__init__(message)
        self.events = list(events)


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
        self.protocol, self.version, self.capabilities = r.read_all('str', 'i32', 'u32')
        r.finish()

    # ----------------------------------------------------------------- transport
    def _drain_err(self):
        for line in iter(self.proc.stderr.readline, b''):
            self.stderr_lines.append(line.decode('utf-8', 'replace').rstrip())

    def _read_exact(self, n):
        buf = bytearray(n)
        view, got = memoryview(buf), 0
        while got < n:
            k = self.proc.stdout.readinto(view[got:])
            if not k:
                raise RuntimeError('server stopped: ' + '\n'.join(self.stderr_lines))
            got += k
        return bytes(buf)

    def _drain_out(self):
        try:
            while True:
                size = _COUNT.unpack(self._read_exact(_COUNT.size))[0]
                if not 4 <= size <= MAX_FRAME:
                    raise RuntimeError('invalid response frame')
                payload = self._read_exact(size)
                self._responses.put((_FIXED['u32'].unpack_from(payload)[0], Cursor(payload[4:])))
        except BaseException as e:  # noqa: BLE001 - surfaced to the waiting request
            self._responses.put(e)

    def send(self, op, body=b''):
        frame = FRAME_HEAD.pack(len(body) + 4, op) + bytes(body)
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
        """Send one request; the reply's Cursor (kind 0), or ServerError (kind 1)."""
        with self._lock:
            self.send(op, body)
            kind, r = self.receive()
            if kind == 1:
                raise ServerError(r.read('str'))
            if kind != 0:
                raise RuntimeError(f'unexpected response kind {kind}')
            return r

    def call(self, op, fields, *reply):
        """A request from ``fields`` whose reply is exactly the ``reply`` tags."""
        r = self.request(op, encode(*fields))
        out = r.read_all(*reply)
        r.finish()
        return out[0] if len(out) == 1 else out

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
        return self.call(2, [('i32', d), ('i32', h), ('i32', w), ('i32', t.shape[1] - 1), ('i32[]', t),
                             ('f32[]', a.transpose(0, 2, 1))], 'u64')

    def network(self, neurons, linear, weights):
        """op 3. ``weights[l]`` is n_out x (n_in+1) column-major with the bias last."""
        fields = [('i32[]', neurons), ('i32[]', linear)] + [('f32[]', w) for w in weights]
        return self.call(3, fields, 'u64')

    def eval(self, net, data, chunk=0):
        return self.call(4, [('u64', net), ('u64', data), ('i32', chunk)], 'u64')

    def download(self, data):
        """op 5: the whole storage, [row][sample][channel] flattened."""
        return self.call(5, [('u64', data)], 'f32[]')

    def download_shaped(self, data, rows, channels, samples):
        return self.download(data).reshape(rows, samples, channels).transpose(0, 2, 1)

    def replace(self, data, samples):
        a = np.asarray(samples, np.float32)
        self.call(6, [('u64', data), ('f32[]', a.transpose(0, 2, 1))])

    def matching_cost(self, net, inputs, targets, rows, target_rows, weights, weight_samples=1, chunk=0):
        """op 7 kind 0.  ``weights`` is (rows, weight_samples, outputs)."""
        return self.call(7, [('u64', net), ('u64', inputs), ('u64', targets), ('i32', 0), ('i32', chunk),
                             ('i32[]', rows), ('i32[]', target_rows), ('i32', weight_samples),
                             ('f32[]', weights)], 'u64')

    def polynomial_cost(self, net, inputs, rows, equations, terms, coeffs, rhs, weights, chunk=0):
        """op 7 kind 1: sparse linear/quadratic residuals."""
        return self.call(7, [('u64', net), ('u64', inputs), ('u64', 0), ('i32', 1), ('i32', chunk),
                             ('i32[]', rows), ('i32', equations), ('i32[]', terms), ('f32[]', coeffs),
                             ('f32[]', rhs), ('f32[]', weights)], 'u64')

    def integral_cost(self, net, inputs, nodes, constants, fields, quadrature_weights, chunk=0):
        """op 12: expression IR (op,a,b) with double constants; ``fields`` is
        (F, samples) double; returns the cost id."""
        f = np.asarray(fields, np.float64)
        qw = np.asarray(quadrature_weights, np.float64)
        return self.call(12, [('u64', net), ('u64', inputs), ('i32', chunk), ('i32', qw.size),
                              ('i32[]', np.asarray(nodes, np.int32)), ('f64[]', constants),
                              ('i32', f.shape[0] if f.size else 0), ('f64[]', f), ('f64[]', qw)], 'u64')

    def inspect(self, cost, compile=False):
        return self.call(13, [('u64', cost), ('i32', int(compile))], 'str', 'str')

    def graph_eval(self, net, costs, graph, gradient=False, layers=0):
        r = self.request(14, encode(('u64', net), ('u64[]', costs), ('i32', int(gradient)), ('raw', graph)))
        value = r.read('f64')
        grads = [r.read('f32[]') for _ in range(r.read('i32'))] if gradient else None
        r.finish()
        return value, grads

    def snapshot(self, net):
        return self.request(9, encode(('u64', net))).rest()

    def restore(self, net, blob):
        self.call(10, [('u64', net), ('raw', blob)])

    def close_object(self, kind, ident):
        self.call(11, [('i32', kind), ('u64', ident)])

    def timing(self, net, cost, warm=20, iterations=100, batches=7, layers=0):
        """op 90 (benchmark command): returns wall ms, device ms, loss, gradients."""
        r = self.request(90, encode(('u64', net), ('u64', cost), ('i32', warm), ('i32', iterations),
                                    ('i32', batches)))
        wall, gpu, loss = r.read_all('f64[]', 'f64[]', 'f64')
        grads = [r.read('f32[]') for _ in range(layers)]
        r.finish()
        return dict(wall_ms=wall, gpu_ms=gpu, loss=loss, gradients=grads)

    def train(self, net, costs, epochs, method=0, fresh=0, steps=0.0, moments=0, lr=0.0, verbose=0,
              log=1, eval_every=0, outputs=0, save=0, stage='', diagnostics=0, graph=None,
              restore_every=0, restore_step=0.0, on_event=None):
        """op 8 (or op 15 with a graph).  Returns the event list and final result.
        ``on_event(session, event)`` is called for every event frame as it
        arrives (e.g. to send op 99 from there)."""
        fields = [('u64', net), ('u64[]', costs), ('u64', epochs), ('i32', method), ('i32', fresh), ('f32', steps),
                  ('i32', moments), ('f32', lr), ('i32', verbose), ('i32', log), ('i32', eval_every),
                  ('i32', outputs), ('i32', save), ('str', stage), ('i32', diagnostics)]
        if graph is not None:
            fields.append(('raw', graph))
        if restore_every:
            fields += [('u64', restore_every), ('f32', restore_step)]
        events = []
        with self._lock:
            self.send(15 if graph is not None else 8, encode(*fields))
            while True:
                kind, r = self.receive()
                if kind == 1:
                    raise ServerError(r.read('str'), events)
                if kind == 0:
                    completed, stopped = r.read_all('u64', 'i32')
                    meta = read_metadata(Cursor(r.blob(r.read('u64'))))
                    r.finish()
                    return dict(completed=completed, stopped=stopped, metadata=meta, events=events)
                ev = _event(kind, r)
                events.append(ev)
                if on_event is not None:
                    on_event(self, ev)

    def stop(self):
        self.send(99)
