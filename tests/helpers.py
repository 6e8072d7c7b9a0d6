"""Shared numerics helpers for the parity tests."""
import numpy as np


def scaled_error(got, want, axis=None):
    """max |got-want| / max(|want|, rms of the row): a relative error that does
    not blow up on entries that cancel to ~0 inside a derivative row."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    if axis is None:
        scale = np.maximum(np.abs(want), np.sqrt(np.mean(want ** 2)) + 1e-30)
    else:
        rms = np.sqrt(np.mean(want ** 2, axis=axis, keepdims=True)) + 1e-30
        scale = np.maximum(np.abs(want), rms)
    return float(np.max(np.abs(got - want) / scale))


def rel_l2(got, want):
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))
