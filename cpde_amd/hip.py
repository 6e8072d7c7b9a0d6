"""ctypes binding of the device library's C ABI (include/cpde_hip.h).

Tests and the benchmark drive the kernels through exactly the entry points the
protocol server uses.  Loading fails loudly when the library is not built: there
is no CPU fallback.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / 'lib' / 'libcpde_hip.so'
HEADER = Path(__file__).resolve().parents[1] / 'include' / 'cpde_hip.h'

OK, EINVAL, EDEVICE, ECOMPILE = 0, 1, 2, 4


class CostStats(ctypes.Structure):
    _fields_ = [('value', ctypes.c_double), ('bad_sample', ctypes.c_int32), ('bad_component', ctypes.c_int32)]


class GradientStats(ctypes.Structure):
    _fields_ = [('squared_norm', ctypes.c_double), ('max_abs', ctypes.c_double),
                ('nonfinite_count', ctypes.c_uint64), ('first_nonfinite', ctypes.c_int32), ('pad_', ctypes.c_int32)]


class CpdeError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(f'[{code}] {message}')
        self.code = code


_lib = None
vp = ctypes.c_void_p
i32 = ctypes.c_int
f32 = ctypes.c_float

SIGNATURES = {
    'cpde_last_error': (ctypes.c_char_p, []),
    'cpde_device_open': (i32, [i32, ctypes.POINTER(vp)]),
    'cpde_device_close': (i32, [vp]),
    'cpde_device_synchronize': (i32, [vp]),
    'cpde_device_info': (i32, [vp, ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(i32)]),
    'cpde_buffer_alloc': (i32, [vp, ctypes.c_size_t, ctypes.POINTER(vp)]),
    'cpde_buffer_free': (i32, [vp, vp]),
    'cpde_buffer_upload': (i32, [vp, vp, vp, ctypes.c_size_t]),
    'cpde_buffer_download': (i32, [vp, vp, vp, ctypes.c_size_t]),
    'cpde_buffer_copy': (i32, [vp, vp, vp, ctypes.c_size_t]),
    'cpde_net_create': (i32, [vp, i32, vp, vp, vp, ctypes.POINTER(vp)]),
    'cpde_net_destroy': (i32, [vp]),
    'cpde_net_state': (i32, [vp, i32, i32, ctypes.POINTER(vp), ctypes.POINTER(i32)]),
    'cpde_net_active': (i32, [vp, i32]),
    'cpde_net_set_active': (i32, [vp, i32, i32]),
    'cpde_net_generation': (ctypes.c_uint64, [vp]),
    'cpde_plan_create': (i32, [vp, i32, i32, vp, i32, i32, ctypes.POINTER(vp)]),
    'cpde_plan_destroy': (i32, [vp]),
    'cpde_plan_stack': (i32, [vp, i32, i32, ctypes.POINTER(vp)]),
    'cpde_plan_stack_scale': (i32, [vp, i32, i32, vp]),
    'cpde_stacks_create': (i32, [vp, ctypes.POINTER(vp)]),
    'cpde_plan_bind': (i32, [vp, vp]),
    'cpde_stacks_destroy': (i32, [vp]),
    'cpde_activate': (i32, [vp, vp, i32, vp, i32, i32]),
    'cpde_forward': (i32, [vp]),
    'cpde_output': (i32, [vp, vp, i32, vp, i32, i32]),
    'cpde_gradients_defer': (i32, [vp, i32]),
    'cpde_costs_begin': (i32, [vp, i32]),
    'cpde_cost_matching': (i32, [vp, vp, i32, vp, vp, i32, i32, i32, i32, i32, i32]),
    'cpde_cost_polynomial': (i32, [vp, vp, i32, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32]),
    'cpde_scale_adjoint': (i32, [vp, vp]),
    'cpde_backward': (i32, [vp, i32]),
    'cpde_inspect_gradients': (i32, [vp]),
    'cpde_epoch_matching': (i32, [vp, vp, i32, vp, vp, i32, i32, i32, i32, i32, i32]),
    'cpde_epoch_matching_static': (i32, [vp, vp, i32, vp, vp, i32, i32, i32, i32, i32, i32]),
    'cpde_epoch_matching_rprop': (i32, [vp, vp, i32, vp, vp, i32, i32, i32, i32, i32, i32]),
    'cpde_scalars_download': (i32, [vp, i32, vp, i32, vp]),
    'cpde_scalars_download_graph': (i32, [vp, i32, vp, i32, vp, vp, vp]),
    'cpde_rprop': (i32, [vp]),
    'cpde_scalars_download_rprop': (i32, [vp, i32, vp, i32, vp, vp, vp, vp]),
    'cpde_update_issue': (i32, [vp, i32, i32, i32, vp, i32, i32, f32]),
    'cpde_inspect_update_issue': (i32, [vp, i32, i32, i32, vp, i32, i32, f32, i32]),
    'cpde_update_resolve': (i32, [vp, vp, vp, vp, vp]),
    'cpde_gradients_discard': (i32, [vp]),
    'cpde_adam': (i32, [vp, i32, f32]),
    'cpde_set_steps': (i32, [vp, f32]),
    'cpde_restore_steps': (i32, [vp, f32]),
    'cpde_zero_gradient': (i32, [vp]),
    'cpde_reset_optimizer': (i32, [vp]),
    'cpde_program_compile': (i32, [vp, ctypes.c_char_p, ctypes.POINTER(vp), ctypes.c_char_p, ctypes.c_size_t]),
    'cpde_program_destroy': (i32, [vp]),
    'cpde_cost_expression': (i32, [vp, vp, vp, vp, i32, i32, i32, vp, vp, i32, i32, i32]),
    'cpde_epoch_expression': (i32, [vp, vp, vp, vp, i32, i32, i32, vp, vp, i32, i32, i32]),
    'cpde_capture_begin': (i32, [vp]),
    'cpde_capture_end': (i32, [vp, i32, vp]),
    'cpde_replay_launch': (i32, [vp]),
    'cpde_replay_destroy': (i32, [vp]),
    'cpde_epoch_expression_fused': (i32, [vp, vp, vp]),
    'cpde_graph_execute': (i32, [vp, vp, i32, i32, i32, vp, vp, vp, vp, vp, i32]),
    'cpde_jit_prepare': (i32, [i32, i32, vp, i32, vp, i32, i32, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]),
    'cpde_trace_enable': (i32, [vp, i32]),
    'cpde_trace_read': (i32, [vp, i32, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_double),
                              ctypes.POINTER(ctypes.c_double)]),
    'cpde_trace_name': (ctypes.c_char_p, [i32]),
    'cpde_trace_kinds': (i32, []),
    'cpde_mark': (i32, [vp, i32]),
    'cpde_elapsed': (i32, [vp, i32, i32, ctypes.POINTER(f32)]),
}


def header_symbols():
    """Function names declared in include/cpde_hip.h."""
    import re
    text = HEADER.read_text()
    return sorted(set(re.findall(r'^\s*(?:int|uint64_t|const char\*)\s+(cpde_\w+)\s*\(', text, re.M)))


def load(path=None):
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(f'{p} is not built; run python -m cpde_amd.build')
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    if path is None:
        _lib = lib
    return lib


def check(code):
    if code != OK:
        raise CpdeError(code, load().cpde_last_error().decode('utf-8', 'replace'))


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


class Buffer:
    """A device allocation (bytes); upload/download take numpy arrays."""

    def __init__(self, device, nbytes):
        self.device, self.nbytes = device, int(nbytes)
        p = vp()
        check(load().cpde_buffer_alloc(device.handle, self.nbytes, ctypes.byref(p)))
        self.ptr = p

    @classmethod
    def of(cls, device, array):
        a = np.ascontiguousarray(array)
        b = cls(device, max(a.nbytes, 4))
        b.upload(a)
        return b

    def upload(self, array):
        a = np.ascontiguousarray(array)
        assert a.nbytes <= self.nbytes
        check(load().cpde_buffer_upload(self.device.handle, self.ptr, _ptr(a), a.nbytes))

    def download(self, dtype, count):
        a = np.empty(count, dtype)
        check(load().cpde_buffer_download(self.device.handle, _ptr(a), self.ptr, a.nbytes))
        return a

    def free(self):
        if self.ptr:
            check(load().cpde_buffer_free(self.device.handle, self.ptr))
            self.ptr = None


class Device:
    def __init__(self, ordinal=0):
        h = vp()
        check(load().cpde_device_open(ordinal, ctypes.byref(h)))
        self.handle = h

    def info(self):
        name = ctypes.create_string_buffer(256)
        cu = i32()
        check(load().cpde_device_info(self.handle, name, 256, ctypes.byref(cu)))
        return name.value.decode(), cu.value

    def synchronize(self):
        check(load().cpde_device_synchronize(self.handle))

    def download_ptr(self, ptr, dtype, count):
        a = np.empty(count, dtype)
        check(load().cpde_buffer_download(self.handle, _ptr(a), ptr, a.nbytes))
        return a

    def upload_ptr(self, ptr, array):
        a = np.ascontiguousarray(array)
        check(load().cpde_buffer_upload(self.handle, ptr, _ptr(a), a.nbytes))

    def costs_begin(self, n):
        check(load().cpde_costs_begin(self.handle, n))

    def scalars(self, costs, layers):
        c = (CostStats * max(costs, 1))()
        g = (GradientStats * max(layers, 1))()
        check(load().cpde_scalars_download(self.handle, costs, ctypes.cast(c, vp), layers, ctypes.cast(g, vp)))
        return list(c)[:costs], list(g)[:layers]

    def mark(self, slot):
        check(load().cpde_mark(self.handle, slot))

    def elapsed(self, a, b):
        ms = f32()
        check(load().cpde_elapsed(self.handle, a, b, ctypes.byref(ms)))
        return ms.value

    def trace(self, on):
        check(load().cpde_trace_enable(self.handle, int(on)))

    def trace_report(self):
        """{kernel class: (launches, total device ms, total algorithmic work)}."""
        out = {}
        lib = load()
        for k in range(lib.cpde_trace_kinds()):
            n, ms, work = ctypes.c_uint64(), ctypes.c_double(), ctypes.c_double()
            check(lib.cpde_trace_read(self.handle, k, ctypes.byref(n), ctypes.byref(ms), ctypes.byref(work)))
            if n.value:
                out[lib.cpde_trace_name(k).decode()] = (n.value, ms.value, work.value)
        return out

    def capture_begin(self):
        check(load().cpde_capture_begin(self.handle))

    def capture_end(self, keep=True):
        """End the open capture; with `keep`, a Replay of it (already run once)."""
        h = vp()
        check(load().cpde_capture_end(self.handle, int(keep), ctypes.byref(h) if keep else None))
        return Replay(self, h) if keep else None

    def close(self):
        if self.handle:
            check(load().cpde_device_close(self.handle))
            self.handle = None


class Replay:
    """A recorded sequence of launches (cpde_capture_end)."""

    def __init__(self, device, handle):
        self.device, self.handle = device, handle

    def launch(self):
        check(load().cpde_replay_launch(self.handle))

    def destroy(self):
        if self.handle:
            check(load().cpde_replay_destroy(self.handle))
            self.handle = None


class Net:
    def __init__(self, device, neurons, linear, weights=None):
        self.device, self.neurons, self.linear = device, list(neurons), list(linear)
        n = np.asarray(neurons, np.int32)
        l = np.asarray(linear, np.int32)
        self._keep = [np.ascontiguousarray(w, np.float32) for w in weights] if weights is not None else None
        arr = None
        if self._keep is not None:
            P = ctypes.c_void_p * len(self._keep)
            arr = P(*[w.ctypes.data for w in self._keep])
        h = vp()
        check(load().cpde_net_create(device.handle, len(neurons), _ptr(n), _ptr(l),
                                     ctypes.cast(arr, vp) if arr is not None else None, ctypes.byref(h)))
        self.handle = h

    def state_ptr(self, t, b):
        p, c = vp(), i32()
        check(load().cpde_net_state(self.handle, t, b, ctypes.byref(p), ctypes.byref(c)))
        return p, c.value

    def state(self, t, b):
        p, c = self.state_ptr(t, b)
        return self.device.download_ptr(p, np.float32, c)

    def set_state(self, t, b, values):
        p, c = self.state_ptr(t, b)
        v = np.ascontiguousarray(values, np.float32)
        assert v.size == c
        self.device.upload_ptr(p, v)

    def active(self, t):
        return load().cpde_net_active(self.handle, t)

    def gradient(self, t):
        return self.state(t, self.active(t))

    def rprop(self):
        check(load().cpde_rprop(self.handle))

    def download_rprop(self, costs):
        """The scalar download with RPROP behind it (no graph): cost and
        gradient totals, and whether the update applied."""
        layers = len(self.neurons) - 1
        c = (CostStats * max(costs, 1))()
        g = (GradientStats * layers)()
        updated = i32()
        check(load().cpde_scalars_download_rprop(self.device.handle, costs, ctypes.cast(c, vp), layers,
                                                 ctypes.cast(g, vp), None, self.handle, ctypes.byref(updated)))
        return list(c)[:costs], list(g), updated.value

    def issue_update(self, costs=0, method=0, step=0, lr=0.0, inspect=None):
        """cpde_update_issue (no graph); with `inspect` ('full' or 'short'),
        cpde_inspect_update_issue: the gradient statistics taken first, or the
        update launch's own finiteness test where the network allows."""
        layers = len(self.neurons) - 1
        if inspect is None:
            check(load().cpde_update_issue(self.device.handle, costs, layers, 0, self.handle, method, step, lr))
        else:
            check(load().cpde_inspect_update_issue(self.device.handle, costs, layers, 0, self.handle, method, step, lr,
                                                   int(inspect == 'full')))

    def resolve_update(self, costs=0):
        """cpde_update_resolve: cost and gradient totals, and whether the update applied."""
        layers = len(self.neurons) - 1
        c = (CostStats * max(costs, 1))()
        g = (GradientStats * layers)()
        updated = i32()
        check(load().cpde_update_resolve(self.device.handle, ctypes.cast(c, vp), ctypes.cast(g, vp), None,
                                         ctypes.byref(updated)))
        return list(c)[:costs], list(g), updated.value

    def adam(self, step, lr):
        check(load().cpde_adam(self.handle, step, lr))

    def set_steps(self, v):
        check(load().cpde_set_steps(self.handle, v))

    def restore_steps(self, v):
        check(load().cpde_restore_steps(self.handle, v))

    def inspect_gradients(self):
        check(load().cpde_inspect_gradients(self.handle))

    def destroy(self):
        if self.handle:
            check(load().cpde_net_destroy(self.handle))
            self.handle = None


class Plan:
    def __init__(self, net, table, width, backward=True):
        self.net, self.width = net, width
        self.table = np.ascontiguousarray(table, np.int32)
        self.rows = self.table.shape[0]
        h = vp()
        check(load().cpde_plan_create(net.handle, self.rows, self.table.shape[1] - 1, _ptr(self.table), width,
                                      int(backward), ctypes.byref(h)))
        self.handle = h

    def stack_ptr(self, layer, kind):
        p = vp()
        check(load().cpde_plan_stack(self.handle, layer, kind, ctypes.byref(p)))
        return p

    def stack(self, layer, kind):
        """(width, rows, n) float32 view of a stack."""
        n = self.net.neurons[layer]
        a = self.net.device.download_ptr(self.stack_ptr(layer, kind), np.float32, self.width * self.rows * n)
        return a.reshape(self.width, self.rows, n)

    def stack_scale(self, layer, kind):
        """(rows,) factors turning stored rows of a stack into unscaled rows."""
        f = np.zeros(self.rows, np.float32)
        check(load().cpde_plan_stack_scale(self.handle, layer, kind, _ptr(f)))
        return f

    def unscaled_stack(self, layer, kind):
        """stack() with every row in the reference's (unscaled) form."""
        return self.stack(layer, kind) * self.stack_scale(layer, kind)[None, :, None]

    def set_stack(self, layer, kind, values):
        self.net.device.upload_ptr(self.stack_ptr(layer, kind), np.ascontiguousarray(values, np.float32))

    def activate(self, data_buffer, data_width, rows, offset, valid):
        r = np.ascontiguousarray(rows, np.int32)
        check(load().cpde_activate(self.handle, data_buffer.ptr, data_width, _ptr(r), offset, valid))

    def forward(self):
        check(load().cpde_forward(self.handle))

    def backward(self, accumulate=False):
        check(load().cpde_backward(self.handle, int(accumulate)))

    def output(self, dest_buffer, dest_width, rows, offset, valid):
        r = np.ascontiguousarray(rows, np.int32)
        check(load().cpde_output(self.handle, dest_buffer.ptr, dest_width, _ptr(r), offset, valid))

    def epoch_matching(self, target, target_width, target_rows, weights, weight_samples, offset, valid, cost_index,
                       collect=True, accumulate=False):
        """forward + matching cost + backward of the activated chunk in one pass."""
        check(load().cpde_epoch_matching(self.handle, target.ptr, target_width, target_rows.ptr, weights.ptr,
                                         weight_samples, offset, valid, cost_index, int(collect), int(accumulate)))

    def epoch_matching_rprop(self, target, target_width, target_rows, weights, weight_samples, offset, valid,
                             cost_index, collect=True, accumulate=False):
        """epoch_matching, then RPROP on the network, the update riding in the
        gradient reduction's launch."""
        check(load().cpde_epoch_matching_rprop(self.handle, target.ptr, target_width, target_rows.ptr, weights.ptr,
                                               weight_samples, offset, valid, cost_index, int(collect),
                                               int(accumulate)))

    def epoch_matching_static(self, target, target_width, target_rows, weights, weight_samples, offset, valid,
                              cost_index, collect=True, accumulate=False):
        """epoch_matching with the library's static scratch: no allocation."""
        check(load().cpde_epoch_matching_static(self.handle, target.ptr, target_width, target_rows.ptr, weights.ptr,
                                                weight_samples, offset, valid, cost_index, int(collect),
                                                int(accumulate)))

    def matching(self, target, target_width, target_rows, weights, weight_samples, offset, valid, cost_index,
                 collect=True, gradient=True):
        check(load().cpde_cost_matching(self.handle, target.ptr, target_width, target_rows.ptr, weights.ptr,
                                        weight_samples, offset, valid, cost_index, int(collect), int(gradient)))

    def destroy(self):
        if self.handle:
            check(load().cpde_plan_destroy(self.handle))
            self.handle = None


def jit_prepare(table, neurons, width=0, compute_units=256, arch='gfx950'):
    """Compile the fused kernels of (schema, architecture) for chunks of `width`
    points on a device of `compute_units` CUs into the code-object cache; no
    device needed.  Returns the compiler log."""
    t = np.ascontiguousarray(table, np.int32)
    n = np.ascontiguousarray(neurons, np.int32)
    log = ctypes.create_string_buffer(1 << 16)
    code = load().cpde_jit_prepare(t.shape[0], t.shape[1] - 1, _ptr(t), len(n), _ptr(n), width, compute_units,
                                   arch.encode(), log, len(log))
    if code != OK:
        raise CpdeError(code, load().cpde_last_error().decode('utf-8', 'replace') + log.value.decode())
    return log.value.decode()


def wire_to_stack(a):
    """(rows, channels, points) -> (points, rows, channels)."""
    return np.ascontiguousarray(np.asarray(a).transpose(2, 0, 1))


def stack_to_reference(s):
    """(points, rows, n) -> reference layout (rows, points, n)."""
    return np.ascontiguousarray(np.asarray(s).transpose(1, 0, 2))


class MatchingRun:
    """One matching cost on one plan: the unit of work of the benchmark step
    (forward + cost + weight gradient), driven through the C ABI."""

    def __init__(self, device, workload, chunk=None, one_pass=True, static_scratch=False):
        wl = workload
        self.device, self.wl = device, wl
        self.one_pass = one_pass
        self.static_scratch = static_scratch
        self.net = Net(device, wl.neurons, wl.linear, wl.init)
        self.samples = wl.size
        self.width = min(chunk or wl.chunk or wl.size, wl.size)
        self.plan = Plan(self.net, wl.cost_schema, self.width, True)
        # wire layouts: data [rows][samples][channels], weights [R][weight_samples][outputs]
        self.data = Buffer.of(device, np.ascontiguousarray(wl.inputs.transpose(0, 2, 1), np.float32))
        self.target = Buffer.of(device, np.ascontiguousarray(wl.target[:, :, None], np.float32))
        self.target_rows = Buffer.of(device, np.ascontiguousarray(wl.target_rows, np.int32))
        self.weights = Buffer.of(device, np.ascontiguousarray(wl.weight_block(), np.float32))
        self.weight_samples = wl.weight_samples
        self.rows = np.ascontiguousarray(wl.cost_rows, np.int32)
        self._loaded = None
        device.costs_begin(1)

    def step(self, collect=True, update=False):
        """forward + cost + backward over every chunk (Server::pass).  As in
        Server::activate (cuda/cpde_server.cu:163) the input copy is skipped when
        the loaded chunk is unchanged.  `update`: then RPROP, riding in the last
        chunk's gradient reduction (one-pass epochs) or launched after it."""
        self.device.costs_begin(1)
        first = True
        for offset in range(0, self.samples, self.width):
            valid = min(self.width, self.samples - offset)
            if self._loaded != (offset, valid):
                self.plan.activate(self.data, self.samples, self.rows, offset, valid)
                self._loaded = (offset, valid)
            last = offset + self.width >= self.samples
            cost = (self.target, self.samples, self.target_rows, self.weights, self.weight_samples, offset, valid, 0,
                    collect)
            if update and last and self.one_pass and not self.static_scratch:
                self.plan.epoch_matching_rprop(*cost, not first)
                return
            if self.static_scratch:
                self.plan.epoch_matching_static(*cost, not first)
            elif self.one_pass:
                self.plan.epoch_matching(*cost, not first)
            else:
                self.plan.forward()
                self.plan.matching(*cost, True)
                self.plan.backward(not first)
            first = False
        if update:
            self.net.rprop()

    def loss(self):
        c, _ = self.device.scalars(1, 0)
        return c[0].value

    def gradients(self):
        return [self.net.gradient(t) for t in range(len(self.wl.neurons) - 1)]

    def close(self):
        for b in (self.data, self.target, self.target_rows, self.weights):
            b.free()
        self.plan.destroy()
        self.net.destroy()
