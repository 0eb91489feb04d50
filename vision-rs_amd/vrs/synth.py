"""Deterministic synthetic parameters and inputs (there is no network for
checkpoints or datasets).

Conv weights ~ N(0, sqrt(2/fan_in)) (Kaiming-normal, fan_in = Cin/g * k * k),
biases 0, BatchNorm identity (gamma 1, beta 0, mean 0, var 1) -- BASELINE
configs 1 and 5.  ``bn="random"`` draws non-trivial BN statistics instead
(gamma U[0.5,1.5), beta N(0,0.1), mean N(0,0.1), var U[0.5,1.5); plain-conv
biases N(0,0.1)) so parity tests exercise the BN fold.  Each parameter has its
own PCG64 stream keyed by (seed, crc32(name)), so the draw does not depend on
parameter order.
"""
from __future__ import annotations

import zlib

import numpy as np


def seeded_params(specs, seed=0, bn="identity"):
    P = {}
    for name, shape in specs:
        rng = np.random.default_rng([seed, zlib.crc32(name.encode())])
        shape = tuple(int(s) for s in shape)
        if name.endswith("weight") and len(shape) == 4:
            fan_in = shape[1] * shape[2] * shape[3]
            P[name] = (rng.standard_normal(shape) * np.sqrt(2.0 / fan_in)).astype(np.float32)
        elif name.endswith("bn.weight"):
            P[name] = (np.ones(shape) if bn == "identity" else rng.uniform(0.5, 1.5, shape)).astype(np.float32)
        elif name.endswith("bn.bias") or name.endswith("bn.running_mean"):
            P[name] = (np.zeros(shape) if bn == "identity" else rng.normal(0, 0.1, shape)).astype(np.float32)
        elif name.endswith("bn.running_var"):
            P[name] = (np.ones(shape) if bn == "identity" else rng.uniform(0.5, 1.5, shape)).astype(np.float32)
        elif name.endswith("bias"):
            P[name] = (np.zeros(shape) if bn == "identity" else rng.normal(0, 0.1, shape)).astype(np.float32)
        else:
            raise KeyError(name)
    return P


def images(n, h, w, seed=0):
    """U[0,1) NCHW float32 image batch (BASELINE configs 1 and 5)."""
    return np.random.default_rng(seed).uniform(0, 1, (n, 3, h, w)).astype(np.float32)
