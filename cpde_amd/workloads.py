"""Synthetic workloads: derivative schemas, input stacks, targets and weights.

Schemas follow the reference's ``table`` ordering: every sub-multi-index of a
requested derivative is included and rows sort by (order, count tuple)
(cpde/quadrature.py:16-38, closure semantics cpde/_prepare.py:84-90).

Input stacks put coordinates in the value row, unit vectors in the first-order
rows and zeros above (scripts/benchmark_fourier_performance.py:47-50).

The named workloads are:
  * ``fourier_fit``: 2->128^4->1 on a 27x27 grid in [0,1]^2, a seeded Fourier sum
    target with analytic derivatives, Xavier-uniform weights (seed 3407), matching
    weights 1/var per row; order 2 and order 6 variants;
  * ``poisson_disk``: 2->64^3->1, 64 Gauss-Legendre radii x 64 angles interior
    quadrature plus 256 boundary points, residual u_xx+u_yy+f;
  * ``fourier_3d``: 3->128^5->1 on a 32^3 grid, all mixed partials through order 4;
  * ``fourier_large``: 2->256^4->1 on a 512x512 grid, order 6, chunked.
"""
from __future__ import annotations

import itertools
import math

import numpy as np


# ----------------------------------------------------------------------------- schemas
def full_schema(variables, order):
    """All multi-indices of total order <= ``order`` in ``variables`` variables,
    rows (order, counts...) sorted by (order, counts)."""
    counts = [c for c in itertools.product(range(order + 1), repeat=variables) if sum(c) <= order]
    counts.sort(key=lambda c: (sum(c), c))
    return np.array([(sum(c), *c) for c in counts], np.int32)


def closed_schema(variables, requested):
    """Closure of explicit count tuples (value row always included)."""
    keys = {(0,) * variables}
    for key in requested:
        keys.update(itertools.product(*(range(c + 1) for c in key)))
    rows = sorted(keys, key=lambda c: (sum(c), c))
    return np.array([(sum(c), *c) for c in rows], np.int32)


def input_stack(points, schema):
    """(rows, channels=variables, points) stack for an identity input layer."""
    pts = np.asarray(points, np.float64)
    n, v = pts.shape
    a = np.zeros((len(schema), v, n), np.float32)
    for r, row in enumerate(schema):
        if row[0] == 0:
            a[r] = pts.T
        elif row[0] == 1:
            a[r] = np.asarray(row[1:], np.float32)[:, None]
    return a


# ----------------------------------------------------------------------------- weights
def xavier_weights(neurons, seed=3407):
    """Column-major n_out x (n_in+1) blocks, Xavier-uniform weights, zero biases."""
    rng = np.random.default_rng(seed)
    out = []
    for n_in, n_out in zip(neurons, neurons[1:]):
        bound = math.sqrt(6.0 / (n_in + n_out))
        w = rng.uniform(-bound, bound, n_out * n_in)
        out.append(np.concatenate((w, np.zeros(n_out))).astype(np.float32))
    return out


def linear_flags(neurons):
    return [1] + [0] * (len(neurons) - 2) + [1]


# ----------------------------------------------------------------------------- targets
def fourier_modes(variables, modes, max_frequency, seed=2026):
    rng = np.random.default_rng(seed)
    freq = rng.integers(1, max_frequency + 1, size=(modes, variables))
    coef = rng.standard_normal(modes)
    phase = rng.uniform(0, 2 * np.pi, size=(modes, variables))
    return freq, coef, phase


def fourier_target(points, schema, freq, coef, phase):
    """u = sum_m c_m prod_v sin(f_mv x_v + phi_mv); d^alpha multiplies by f^alpha and
    shifts each phase by alpha_v * pi/2.  Returns (rows, points) float64."""
    pts = np.asarray(points, np.float64)
    out = np.zeros((len(schema), len(pts)))
    for r, row in enumerate(schema):
        alpha = row[1:]
        for m in range(len(coef)):
            term = np.full(len(pts), coef[m])
            for v in range(pts.shape[1]):
                term = term * freq[m, v] ** alpha[v] * np.sin(freq[m, v] * pts[:, v] + phase[m, v] + alpha[v] * np.pi / 2)
            out[r] += term
    return out


def uniform_grid(n, dims):
    axes = [np.linspace(0, 1, n)] * dims
    mesh = np.meshgrid(*axes, indexing='ij')
    return np.column_stack([m.ravel() for m in mesh])


class MatchingWorkload:
    """Everything a matching-cost run needs, in protocol layouts.

    ``schema`` holds the data's derivative rows and ``rows`` the cost's rows,
    as indices into it (default: all; the network runs on schema[rows]).
    ``target`` holds the rows of the target data object, whose derivative rows
    are ``target_schema`` (default ``schema``), and ``target_rows`` names the
    target row of each cost row (default: the same index).  ``weights`` is one
    weight per cost row, shape (R,), or one per cost row and sample, shape
    (R, points) (the [R][P][1] form, weight_samples = P).  ``linear`` flags
    each layer (default: linear input and output, sigmoid hidden layers)."""

    def __init__(self, name, neurons, points, schema, target, weights, init, chunk=0, linear=None, rows=None,
                 target_schema=None, target_rows=None):
        self.name, self.neurons = name, list(neurons)
        self.linear = linear_flags(neurons) if linear is None else [int(v) for v in linear]
        self.points = np.asarray(points, np.float32)
        self.schema = np.asarray(schema, np.int32)
        self.inputs = input_stack(self.points, self.schema)
        self.cost_rows = np.arange(len(self.schema), dtype=np.int32) if rows is None else np.asarray(rows, np.int32)
        self.target = np.asarray(target, np.float32)            # (target rows, points)
        self.target_schema = self.schema if target_schema is None else np.asarray(target_schema, np.int32)
        self.target_rows = self.cost_rows.copy() if target_rows is None else np.asarray(target_rows, np.int32)
        self.row_weights = np.asarray(weights, np.float32)      # (R,) or (R, points)
        self.init = init
        self.chunk = chunk

    @property
    def rows(self):
        """Rows of the cost (the network's derivative rows)."""
        return len(self.cost_rows)

    @property
    def cost_schema(self):
        return self.schema[self.cost_rows]

    @property
    def weight_samples(self):
        return 1 if self.row_weights.ndim == 1 else self.row_weights.shape[1]

    def weight_block(self):
        """The weights as the wire sends them: [R][weight_samples][outputs=1]."""
        return self.row_weights.reshape(self.rows, self.weight_samples, 1)

    @property
    def size(self):
        return len(self.points)

    def flops_per_epoch(self):
        """Algorithmic GEMM flops: forward + transposed (not the input layer) + wgrad."""
        pairs = list(zip(self.neurons, self.neurons[1:]))
        rp = self.rows * self.size
        fwd = sum(a * b for a, b in pairs)
        return 2 * rp * (fwd + sum(a * b for a, b in pairs[1:]) + fwd)

    def bytes_per_epoch(self):
        """Algorithmic HBM bytes: per hidden layer composition (read z, write y) and
        adjoint (read z, read g_y, write g_z) = 5n floats per row-point, the output
        cost 3*n_out, and RPROP 28 bytes per parameter."""
        rp = self.rows * self.size
        hidden = sum(self.neurons[1:-1])
        params = sum(b * (a + 1) for a, b in zip(self.neurons, self.neurons[1:]))
        return 4 * rp * (5 * hidden + 3 * self.neurons[-1]) + 28 * params

    def points_slice(self, idx, name=None):
        """The same workload (network, rows, row weights) on the points ``idx``,
        unchunked; per-sample weights follow their points."""
        idx = np.asarray(idx)
        weights = self.row_weights if self.weight_samples == 1 else self.row_weights[:, idx]
        return MatchingWorkload(name or f'{self.name}[{len(idx)} points]', self.neurons, self.points[idx],
                                self.schema, self.target[:, idx], weights, self.init, linear=self.linear,
                                rows=self.cost_rows, target_schema=self.target_schema, target_rows=self.target_rows)

    def subset(self, count):
        """The same workload on `count` evenly spaced points, unchunked."""
        return self.points_slice(np.linspace(0, self.size - 1, count).astype(int))

    def upload(self, session, chunk=None):
        """Creates data, target, network and cost objects; returns their ids."""
        d = session.data(self.inputs, self.schema)
        t = session.data(self.target[:, None, :], self.target_schema)
        n = session.network(self.neurons, self.linear, self.init)
        c = session.matching_cost(n, d, t, self.cost_rows, self.target_rows, self.weight_block(), self.weight_samples,
                                  self.chunk if chunk is None else chunk)
        return dict(data=d, target=t, net=n, cost=c)


def fourier_fit(order=6, grid=27, neurons=(2, 128, 128, 128, 128, 1), modes=8, max_frequency=4, seed=3407):
    schema = full_schema(2, order)
    pts = uniform_grid(grid, 2)
    freq, coef, phase = fourier_modes(2, modes, max_frequency)
    target = fourier_target(pts, schema, freq, coef, phase)
    weights = 1.0 / target.var(axis=1)
    return MatchingWorkload(f'fourier_fit_order{order}', neurons, pts, schema, target, weights,
                            xavier_weights(neurons, seed))


def fourier_3d(grid=32, order=4, neurons=(3, 128, 128, 128, 128, 128, 1), modes=12, max_frequency=3, points=None):
    schema = full_schema(3, order)
    pts = uniform_grid(grid, 3)
    if points is not None:
        pts = pts[np.linspace(0, len(pts) - 1, points).astype(int)]
    freq, coef, phase = fourier_modes(3, modes, max_frequency)
    target = fourier_target(pts, schema, freq, coef, phase)
    return MatchingWorkload('fourier_3d_order4', neurons, pts, schema, target, 1.0 / target.var(axis=1),
                            xavier_weights(neurons))


def fourier_large(grid=512, order=6, neurons=(2, 256, 256, 256, 256, 1), modes=16, chunk=65536, points=None):
    schema = full_schema(2, order)
    pts = uniform_grid(grid, 2)
    if points is not None:
        pts = pts[np.linspace(0, len(pts) - 1, points).astype(int)]
    freq, coef, phase = fourier_modes(2, modes, 4)
    target = fourier_target(pts, schema, freq, coef, phase)
    return MatchingWorkload('fourier_large_order6', neurons, pts, schema, target, 1.0 / target.var(axis=1),
                            xavier_weights(neurons), chunk=min(chunk, len(pts)))


# ----------------------------------------------------------------------------- Poisson
def disk_quadrature(radial=64, angular=64):
    """Interior: Gauss-Legendre radii r=(t+1)/2 with weight (w/2) r (2 pi/angular),
    uniform angles.  Returns points (N,2) and weights (N,)."""
    t, w = np.polynomial.legendre.leggauss(radial)
    r = (t + 1) / 2
    wr = w / 2 * r
    th = 2 * np.pi * np.arange(angular) / angular
    R, T = np.meshgrid(r, th, indexing='ij')
    W = np.repeat(wr, angular) * (2 * np.pi / angular)
    pts = np.column_stack(((R * np.cos(T)).ravel(), (R * np.sin(T)).ravel()))
    return pts, W


def circle_points(count=256):
    th = 2 * np.pi * np.arange(count) / count
    return np.column_stack((np.cos(th), np.sin(th))), np.full(count, 2 * np.pi / count)


def gaussian_source(points, count=4, seed=2026):
    rng = np.random.default_rng(seed)
    amp = rng.standard_normal(count)
    rad = 0.5 * np.sqrt(rng.uniform(0, 1, count))
    ang = rng.uniform(0, 2 * np.pi, count)
    centres = np.column_stack((rad * np.cos(ang), rad * np.sin(ang)))
    width = rng.uniform(0.15, 0.3, count)
    p = np.asarray(points, np.float64)
    f = np.zeros(len(p))
    for a, c, s in zip(amp, centres, width):
        f += a * np.exp(-np.sum((p - c) ** 2, axis=1) / (2 * s * s))
    return f


class PoissonWorkload:
    """Config: 2->64^3->1 sigmoid; interior cost (u_xx+u_yy+f)^2 with quadrature
    weights, boundary cost u^2; the graph root is their sum."""

    def __init__(self, neurons=(2, 64, 64, 64, 1), radial=64, angular=64, boundary=256, seed=3407):
        self.neurons = list(neurons)
        self.linear = linear_flags(neurons)
        self.interior, self.interior_w = disk_quadrature(radial, angular)
        self.boundary, self.boundary_w = circle_points(boundary)
        self.f = gaussian_source(self.interior)
        self.schema = closed_schema(2, [(2, 0), (0, 2)])   # rows: 1, y, x, yy, xx
        self.init = xavier_weights(neurons, seed)

    name = 'poisson_disk_order2'

    def leaves(self):
        """(rows, points) of the interior and boundary costs."""
        return [(len(self.schema), len(self.interior)), (1, len(self.boundary))]

    @property
    def size(self):
        return len(self.interior) + len(self.boundary)

    def point_rows(self):
        return sum(r * p for r, p in self.leaves())

    def flops_per_epoch(self):
        """Forward + transposed (not the input layer) + weight-gradient flops of
        one forward and one backward per leaf (the graph's multipliers are known)."""
        pairs = list(zip(self.neurons, self.neurons[1:]))
        fwd = sum(a * b for a, b in pairs)
        return 2 * self.point_rows() * (2 * fwd + sum(a * b for a, b in pairs[1:]))

    def bytes_per_epoch(self):
        hidden = sum(self.neurons[1:-1])
        params = sum(b * (a + 1) for a, b in zip(self.neurons, self.neurons[1:]))
        return 4 * self.point_rows() * (5 * hidden + 3 * self.neurons[-1]) + 28 * params

    def row_of(self, counts):
        for r, row in enumerate(self.schema):
            if tuple(row[1:]) == tuple(counts):
                return r
        raise KeyError(counts)

    def interior_ir(self):
        """(u_xx + u_yy + f)**2: components index row*outputs + output."""
        xx, yy = self.row_of((2, 0)), self.row_of((0, 2))
        nodes = [(1, xx, 0), (1, yy, 0), (3, 0, 1), (2, 0, 0), (3, 2, 3), (7, 4, 0)]
        consts = [0, 0, 0, 0, 0, 2.0]
        return nodes, consts

    @staticmethod
    def boundary_ir():
        return [(1, 0, 0), (7, 0, 0)], [0, 2.0]

    @staticmethod
    def graph():
        """Root = leaf0 + leaf1."""
        from .wire import graph_bytes
        return graph_bytes([(1, 0, 0), (1, 1, 0), (3, 0, 1)], [0.0, 0.0, 0.0], 2)

    @staticmethod
    def value_dependent_graph():
        """Root = leaf0 / leaf1 + log(leaf0) + leaf1 ** 1.5: every leaf multiplier
        depends on the leaf values (scalar ops Leaf 1, Add 3, Div 6, Power 7,
        Log 10, cuda/scalar_ops.cuh:5)."""
        from .wire import graph_bytes
        nodes = [(1, 0, 0), (1, 1, 0), (6, 0, 1), (10, 0, 0), (3, 2, 3), (7, 1, 0), (3, 4, 5)]
        return graph_bytes(nodes, [0.0, 0.0, 0.0, 0.0, 0.0, 1.5, 0.0], 6)

    def upload(self, session):
        vschema = closed_schema(2, [])
        di = session.data(input_stack(self.interior, self.schema), self.schema)
        db = session.data(input_stack(self.boundary, vschema), vschema)
        n = session.network(self.neurons, self.linear, self.init)
        nodes, consts = self.interior_ir()
        ci = session.integral_cost(n, di, nodes, consts, self.f[None, :], self.interior_w)
        bnodes, bconsts = self.boundary_ir()
        cb = session.integral_cost(n, db, bnodes, bconsts, np.zeros((0, len(self.boundary))), self.boundary_w)
        return dict(interior=di, boundary=db, net=n, costs=[ci, cb])


# ----------------------------------------------------------------------------- variations
class VariationWorkload:
    """2->6->5->1 sigmoid network on 12 quadrature points in [0,1]^2 with rows
    (value, x); components u = 0, u_x = 1 (row * outputs + output)."""

    def __init__(self, seed=61):
        rng = np.random.default_rng(seed)
        self.neurons = [2, 6, 5, 1]
        self.schema = closed_schema(2, [(1, 0)])
        self.points = rng.uniform(0, 1, (12, 2))
        self.weights = rng.uniform(0.02, 0.1, 12)
        self.init = xavier_weights(self.neurons, seed)

    # expression IR of the leaves: (op, a, b) with b = frozen flag on components
    A = ([(1, 0, 0)], [0.0])                                    # u
    CORRECTION = ([(1, 0, 0), (1, 1, 1), (5, 0, 1)], [0.0, 0.0, 0.0])   # u * u_x, u_x frozen
    FROZEN = ([(1, 0, 1), (7, 0, -1)], [0.0, 2.0])              # u ** 2, u frozen
    FREE = ([(1, 0, 0), (7, 0, -1)], [0.0, 2.0])                # u ** 2

    @staticmethod
    def nested_graph():
        """(a*a).with_variation(correction.with_variation(a)) + correction + a
        (tests/test_integrals.py:176-186), nodes as the reference client's
        prepare_graph numbers them: leaf a, Mul, leaf correction, Attach,
        Attach, Add, Add."""
        from .wire import graph_bytes
        nodes = [(1, 0, -1), (5, 0, 0), (1, 1, -1), (15, 2, 0), (15, 1, 3), (3, 4, 2), (3, 5, 0)]
        return graph_bytes(nodes, [0.0] * 7, 6)

    @staticmethod
    def cancelled_graph():
        """a.with_variation(-a) (tests/test_audit_fixes.py:69-77)."""
        from .wire import graph_bytes
        return graph_bytes([(1, 0, -1), (8, 0, -1), (15, 0, 1)], [0.0] * 3, 2)

    def upload(self, s):
        d = s.data(input_stack(self.points, self.schema), self.schema)
        n = s.network(self.neurons, linear_flags(self.neurons), self.init)
        costs = {}
        for name, (nodes, consts) in (('a', self.A), ('correction', self.CORRECTION), ('frozen', self.FROZEN),
                                      ('free', self.FREE)):
            costs[name] = s.integral_cost(n, d, nodes, consts, np.zeros((0, 12)), self.weights, chunk=5)
        return n, d, costs
