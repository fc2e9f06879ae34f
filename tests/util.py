"""Shared test helpers (comparison with stated tolerances, margins)."""
import numpy as np


def max_rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = max(float(np.max(np.abs(ref))), 1e-30)
    return float(np.max(np.abs(got - ref))) / scale


def top2_margin(x):
    x = np.asarray(x, np.float64)
    i = int(np.argmax(x))
    y = x.copy()
    y[i] = -np.inf
    return float(x[i] - np.max(y))


def f16_bits_to_f32(a):
    return np.asarray(a, np.uint16).view(np.float16).astype(np.float32)
