"""ctypes view of the C oracle -- TEST INFRASTRUCTURE ONLY.

Loaded only by tests/, the package smoke() and bench.py's cpu_baseline leg, as
the oracle; the product path never imports it.  Functions mirror
oracle/cpde_oracle.h and take numpy arrays in the reference's layouts:
stacks [row][point][neuron], weight blocks n_out x (n_in+1) column-major.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / 'liboracle.so'
REF_SERVER = HERE / '_ref' / 'cpde_cpu_server'

_f32p = np.ctypeslib.ndpointer(np.float32, flags='C_CONTIGUOUS')
_i32p = np.ctypeslib.ndpointer(np.int32, flags='C_CONTIGUOUS')


class GradStats(ctypes.Structure):
    _fields_ = [('squared_norm', ctypes.c_double), ('max_abs', ctypes.c_double),
                ('nonfinite', ctypes.c_ulonglong), ('first', ctypes.c_int)]


def build():
    subprocess.run(['make', '-s', '-C', str(HERE), 'liboracle.so'], check=True)


def _load():
    if not LIB.exists():
        build()
    lib = ctypes.CDLL(str(LIB))
    lib.orc_pair_tables.argtypes = [ctypes.c_int, ctypes.c_int, _i32p, _i32p, _i32p]
    lib.orc_compose.argtypes = [ctypes.c_int, ctypes.c_int, _i32p, ctypes.c_long, _f32p, _f32p]
    lib.orc_compose_adjoint.argtypes = [ctypes.c_int, ctypes.c_int, _i32p, ctypes.c_long, _f32p, _f32p]
    lib.orc_compose_prime.argtypes = [ctypes.c_int, ctypes.c_int, _i32p, ctypes.c_long, _f32p, _f32p]
    lib.orc_gemm.argtypes = [ctypes.c_int] * 5 + [ctypes.c_float, _f32p, ctypes.c_int, _f32p, ctypes.c_int,
                                                  ctypes.c_float, _f32p, ctypes.c_int]
    lib.orc_matching.restype = ctypes.c_double
    lib.orc_matching.argtypes = [ctypes.c_int] * 6 + [_f32p, _f32p, _f32p, _i32p, _f32p, ctypes.c_int, ctypes.c_int,
                                                      ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
    pp = ctypes.POINTER(ctypes.POINTER(ctypes.c_float))
    lib.orc_matching_epoch.restype = ctypes.c_double
    lib.orc_matching_epoch.argtypes = [ctypes.c_int, _i32p, _i32p, pp, pp, ctypes.c_int, ctypes.c_int, _i32p,
                                       ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_int, _i32p, _f32p, _i32p, _f32p,
                                       ctypes.c_int, ctypes.c_void_p]
    lib.orc_forward.argtypes = [ctypes.c_int, _i32p, _i32p, pp, ctypes.c_int, ctypes.c_int, _i32p, ctypes.c_int,
                                _f32p, _f32p]
    lib.orc_gradient_stats.restype = GradStats
    lib.orc_gradient_stats.argtypes = [_f32p, ctypes.c_int]
    for name in ('orc_rprop',):
        getattr(lib, name).argtypes = [ctypes.c_int, _f32p, _f32p, _f32p, _f32p]
    for name in ('orc_restore_steps', 'orc_set_steps'):
        getattr(lib, name).argtypes = [ctypes.c_int, ctypes.c_float, _f32p, _f32p, _f32p]
    lib.orc_adam.argtypes = [ctypes.c_int, _f32p, _f32p, _f32p, _f32p] + [ctypes.c_float] * 5
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _table(table):
    return np.ascontiguousarray(table, np.int32)


def pair_tables(table):
    t = _table(table)
    R, V = t.shape[0], t.shape[1] - 1
    d = np.zeros(R * R, np.int32)
    c = np.zeros(R * R, np.int32)
    lib().orc_pair_tables(R, V, t, d, c)
    return d.reshape(R, R), c.reshape(R, R)


def compose(table, z):
    """z: (R, count) float32 -> y (R, count)."""
    t = _table(table)
    z = np.ascontiguousarray(z, np.float32)
    y = np.zeros_like(z)
    if lib().orc_compose(t.shape[0], t.shape[1] - 1, t, z.shape[1], z, y):
        raise ValueError('invalid schema')
    return y


def compose_prime(table, z):
    """z: (R, count) float32 -> u (R, count): the jet of sigma'(z)."""
    t = _table(table)
    z = np.ascontiguousarray(z, np.float32)
    u = np.zeros_like(z)
    if lib().orc_compose_prime(t.shape[0], t.shape[1] - 1, t, z.shape[1], z, u):
        raise ValueError('invalid schema')
    return u


def compose_adjoint(table, z, gy):
    t = _table(table)
    z = np.ascontiguousarray(z, np.float32)
    g = np.array(gy, np.float32, copy=True, order='C')
    if lib().orc_compose_adjoint(t.shape[0], t.shape[1] - 1, t, z.shape[1], z, g):
        raise ValueError('invalid schema')
    return g


def gemm(ta, tb, m, n, k, alpha, a, lda, b, ldb, beta, c, ldc):
    a = np.ascontiguousarray(a, np.float32).ravel()
    b = np.ascontiguousarray(b, np.float32).ravel()
    c = np.array(c, np.float32, copy=True).ravel()
    lib().orc_gemm(ta, tb, m, n, k, alpha, a, lda, b, ldb, beta, c, ldc)
    return c


def _ptrs(arrays):
    P = ctypes.POINTER(ctypes.c_float)
    return (P * len(arrays))(*[a.ctypes.data_as(P) for a in arrays])


def matching(y, target, target_rows, weights, weight_samples, width, valid, offset, samples, gradient=True):
    """y: (R, width, outputs); target: (Rt, samples, outputs); weights (R, ws, outputs)."""
    y = np.ascontiguousarray(y, np.float32)
    R, _, outputs = y.shape
    g = np.zeros_like(y)
    bs, bc = ctypes.c_int(), ctypes.c_int()
    loss = lib().orc_matching(R, outputs, width, valid, offset, samples, y, g,
                              np.ascontiguousarray(target, np.float32), _table(target_rows),
                              np.ascontiguousarray(weights, np.float32), weight_samples, int(gradient),
                              ctypes.byref(bs), ctypes.byref(bc))
    return loss, g, bs.value, bc.value


def matching_epoch(neurons, linear, weights, table, x, target, row_weights, chunk=0, rows=None,
                   target_rows=None, weight_samples=1, outputs=True):
    """One epoch of one matching cost.  x: (Rd, samples, n0) [row][sample][channel];
    target: (Rt, samples, n_out); row_weights: (R, weight_samples, n_out).
    Returns loss, gradients (list of flattened blocks) and outputs (R, samples, n_out)."""
    t = _table(table)
    R, V = t.shape[0], t.shape[1] - 1
    L = len(neurons)
    x = np.ascontiguousarray(x, np.float32)
    samples = x.shape[1]
    W = [np.ascontiguousarray(w, np.float32).ravel() for w in weights]
    G = [np.zeros_like(w) for w in W]
    rows = np.arange(R, dtype=np.int32) if rows is None else _table(rows)
    target_rows = np.arange(R, dtype=np.int32) if target_rows is None else _table(target_rows)
    out = np.zeros((R, samples, neurons[-1]), np.float32) if outputs else None
    loss = lib().orc_matching_epoch(L, _table(neurons), _table(linear), _ptrs(W), _ptrs(G), R, V, t, samples, chunk,
                                    x, x.shape[0], rows, np.ascontiguousarray(target, np.float32), target_rows,
                                    np.ascontiguousarray(row_weights, np.float32), weight_samples,
                                    out.ctypes.data if out is not None else None)
    return loss, G, out


def forward(neurons, linear, weights, table, x):
    """x: (R, w, n0) -> (R, w, n_out), one unpadded chunk."""
    t = _table(table)
    x = np.ascontiguousarray(x, np.float32)
    W = [np.ascontiguousarray(w, np.float32).ravel() for w in weights]
    out = np.zeros((t.shape[0], x.shape[1], neurons[-1]), np.float32)
    lib().orc_forward(len(neurons), _table(neurons), _table(linear), _ptrs(W), t.shape[0], t.shape[1] - 1, t,
                      x.shape[1], x, out)
    return out


def gradient_stats(g):
    s = lib().orc_gradient_stats(np.ascontiguousarray(g, np.float32), int(np.size(g)))
    return dict(squared_norm=s.squared_norm, max_abs=s.max_abs, nonfinite=s.nonfinite,
                first=-1 if s.first == 0x7fffffff else s.first)


def rprop(W, step, ga, gi):
    arrays = [np.array(a, np.float32, copy=True) for a in (W, step, ga, gi)]
    lib().orc_rprop(arrays[0].size, *arrays)
    return arrays


def restore_steps(floor, step, ga, gi):
    arrays = [np.array(a, np.float32, copy=True) for a in (step, ga, gi)]
    lib().orc_restore_steps(arrays[0].size, floor, *arrays)
    return arrays


def set_steps(value, step, ga, gi):
    arrays = [np.array(a, np.float32, copy=True) for a in (step, ga, gi)]
    lib().orc_set_steps(arrays[0].size, value, *arrays)
    return arrays


def adam(W, g, m, v, lr, step):
    W, m, v = (np.array(a, np.float32, copy=True) for a in (W, m, v))
    b1, b2 = np.float32(0.9), np.float32(0.999)
    lib().orc_adam(W.size, W, np.ascontiguousarray(g, np.float32), m, v, lr, b1, b2,
                   float(np.float32(b1) ** np.float32(step)), float(np.float32(b2) ** np.float32(step)))
    return W, m, v


def reference_server():
    """Path of the reference CPU server built by ``make -C oracle ref`` (or None)."""
    return REF_SERVER if REF_SERVER.exists() and os.access(REF_SERVER, os.X_OK) else None
