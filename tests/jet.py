"""Truncated multivariate Taylor series in float64/complex128 -- an independent
statement of what the derivative stack means, used to pin the oracle.

A derivative stack at one point is the set of partials d^alpha f(x0) for the
schema's multi-indices.  As a truncated power series in h = x - x0 it is
f(x0+h) = sum_alpha d^alpha f(x0) h^alpha / alpha!.  Composition with the
sigmoid is then plain series arithmetic (exp, reciprocal), with no
set-partition bookkeeping at all; reading the coefficients back gives every
d^alpha sigma(z(x)) (the same idea as the reference's independent audit,
scripts/audit_cuda.py:123-226, restated here).  Complex inputs give the
complex-step derivative of the whole map, which pins the adjoint.
"""
from __future__ import annotations

import math

import numpy as np


class Jet:
    def __init__(self, variables, order, dtype=np.float64):
        self.V, self.K = variables, order
        self.shape = (order + 1,) * variables
        idx = np.indices(self.shape).reshape(variables, -1).T
        self.mask = (idx.sum(axis=1) <= order).reshape(self.shape)
        self.dtype = dtype

    def zeros(self):
        return np.zeros(self.shape, self.dtype)

    def from_stack(self, schema, values):
        """Series of a function whose partials d^alpha are ``values`` on the
        schema rows (rows missing from the schema are zero)."""
        s = np.zeros(self.shape, np.result_type(self.dtype, np.asarray(values).dtype))
        for row, v in zip(schema, values):
            alpha = tuple(int(a) for a in row[1:])
            s[alpha] = v / math.prod(math.factorial(a) for a in alpha)
        return s

    def to_stack(self, schema, series):
        return np.array([series[tuple(int(a) for a in row[1:])] * math.prod(math.factorial(int(a)) for a in row[1:])
                         for row in schema])

    def mul(self, a, b):
        out = np.zeros(self.shape, np.result_type(a, b))
        for idx in zip(*np.nonzero(self.mask)):
            if a[idx] == 0:
                continue
            # shift b by idx, truncated at total order K
            sl_src = tuple(slice(0, self.K + 1 - i) for i in idx)
            sl_dst = tuple(slice(i, self.K + 1) for i in idx)
            out[sl_dst] += a[idx] * b[sl_src]
        out[~self.mask] = 0
        return out

    def _power_series(self, a, coefficients):
        """sum_k coefficients[k] * (a - a0)^k for k = 0..K."""
        d = a.copy()
        d[(0,) * self.V] = 0
        out = np.zeros(self.shape, np.result_type(a, np.asarray(coefficients)))
        p = np.zeros(self.shape, d.dtype)
        p[(0,) * self.V] = 1
        for k, c in enumerate(coefficients):
            out = out + c * p
            p = self.mul(p, d)
        return out

    def exp(self, a):
        a0 = a[(0,) * self.V]
        return self._power_series(a, [np.exp(a0) / math.factorial(k) for k in range(self.K + 1)])

    def reciprocal(self, a):
        a0 = a[(0,) * self.V]
        return self._power_series(a, [(-1) ** k / a0 ** (k + 1) for k in range(self.K + 1)])

    def sigmoid(self, a):
        one = np.zeros(self.shape, a.dtype)
        one[(0,) * self.V] = 1
        return self.reciprocal(one + self.exp(-a))


def compose_stack(schema, z):
    """d^alpha sigma(z(x)) for every schema row, from the stack z (rows,)."""
    schema = np.asarray(schema)
    V, K = schema.shape[1] - 1, int(schema[:, 0].max())
    j = Jet(V, K, np.complex128 if np.iscomplexobj(z) else np.float64)
    return j.to_stack(schema, j.sigmoid(j.from_stack(schema, z)))


def compose_prime_stack(schema, z):
    """d^alpha sigma'(z(x)) for every schema row: sigma' = sigma (1 - sigma) as series."""
    schema = np.asarray(schema)
    V, K = schema.shape[1] - 1, int(schema[:, 0].max())
    j = Jet(V, K, np.complex128 if np.iscomplexobj(z) else np.float64)
    y = j.sigmoid(j.from_stack(schema, z))
    return j.to_stack(schema, y - j.mul(y, y))


def compose_jacobian(schema, z, h=1e-30):
    """J[i, j] = d y_i / d z_j by complex step (exact to rounding)."""
    R = len(schema)
    J = np.zeros((R, R))
    for col in range(R):
        zc = np.asarray(z, np.complex128).copy()
        zc[col] += 1j * h
        J[:, col] = compose_stack(schema, zc).imag / h
    return J
